"""FP16 caches under the 1e-5 contract with a peaked softmax.

The exact kernels feed the softmax weights to FP16 MFMAs as three FP16 parts.
FP16's exponent stops at 2^-24, so a weight far below the row maximum must
still reach the numerator, or the output is biased (it still counts in the
FP32 row sum). These rows hold one dominant key (the sink, key 0) and
thousands of keys 25 to 26 log2 units below it, whose weights together are
about 1e-4 of the row: dropping them moves the output far past 1e-5. The
exact prefill (kvflux_paged_prefill_exact) and the batch decode
(kvflux_paged_attention) must both stay within 1e-5 of the double-precision
oracle (reference_attention.cpp:28-91 restated) on every checked row.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from gpu_util import buffer_like
from kvflux_amd import capi, device
from oracle import oracle

pytestmark = pytest.mark.gpu

D, BS = 128, 16
SCALE_LOG2 = 1.4426950408889634 / np.sqrt(D)


def peaked_cache(tokens, kv_heads, rng, blocks_extra=3):
    """K/V of one sequence in a paged FP16 cache: key 0's first dim makes
    its score (with q = 8 e_0) 25-26 log2 units above every other key's.
    V ~ N(0,1) for key 0, 1 + 0.5 N(0,1) for the rest: the small keys' share
    of a row (about 1e-4 at 4096 keys) moves the output the same way for
    every dim, as correlated values do, instead of averaging out."""
    a = 8.0
    k = np.zeros((tokens, kv_heads, D), np.float32)
    top = 30.0
    k[:, :, 0] = top - rng.uniform(25.0, 26.0, (tokens, kv_heads)) / (a * SCALE_LOG2)
    k[0, :, 0] = top
    k[:, :, 1:] = rng.uniform(-1, 1, (tokens, kv_heads, D - 1)).astype(np.float32)
    v = (1.0 + 0.5 * rng.standard_normal((tokens, kv_heads, D))).astype(np.float32)
    v[0] = rng.standard_normal((kv_heads, D))
    k16, v16 = k.astype(np.float16), v.astype(np.float16)
    npg = (tokens + BS - 1) // BS
    blocks = npg + blocks_extra
    table = rng.permutation(blocks)[:npg].astype(np.uint64)
    kc = np.zeros((blocks, kv_heads, BS, D), np.float16)
    vc = np.zeros_like(kc)
    t = np.arange(tokens)
    kc[table[t // BS], :, t % BS, :] = k16
    vc[table[t // BS], :, t % BS, :] = v16
    return kc.view(np.uint16).reshape(-1), vc.view(np.uint16).reshape(-1), table, blocks, a


def query_rows(n, q_heads, a, rng):
    """q = a e_0 plus a small N(0, 0.01) remainder (the sink still dominates)."""
    q = (0.01 * rng.standard_normal((n, q_heads, D))).astype(np.float32)
    q[:, :, 0] = a
    return q.reshape(-1)


@pytest.mark.parametrize("q_heads,kv_heads", [(1, 1), (4, 2)])
def test_exact_prefill_f16_peaked_rows(gpu, q_heads, kv_heads):
    T = 4096
    rng = np.random.default_rng(61 + q_heads)
    kh, vh, table, blocks, a = peaked_cache(T, kv_heads, rng)
    q = query_rows(T, q_heads, a, rng)
    kc, vc, td, qd = buffer_like(kh), buffer_like(vh), buffer_like(table), buffer_like(q)
    out = buffer_like(np.full(q.size + 4, 777.0, np.float32))
    lib = capi.lib()
    assert lib.kvflux_paged_prefill_exact(kc.ptr, vc.ptr, blocks, kv_heads, BS, D, capi.DTYPE_F16, td.ptr,
                                          len(table), T, T, q_heads, qd.ptr, out.ptr, None, 0, None) == 0, \
        capi.last_error()
    device.synchronize()
    got = out.download(np.float32)
    assert np.all(got[q.size:] == 777.0)
    got = got[:q.size].reshape(T, q_heads * D)
    rows = [0, 1, 17, 1000, 2047, 3001, 4094, 4095]
    exp = oracle.paged_attention_rows(kh, vh, kv_heads, BS, D, oracle.F16, np.tile(table, len(rows)), len(table),
                                      np.array([t + 1 for t in rows], np.uint64),
                                      q.reshape(T, q_heads * D)[rows].reshape(-1), q_heads, threads=8)
    err = np.abs(got[rows].reshape(-1) - exp).max()
    assert err < 1e-5, err
    # The small keys carry weight: the row differs from the sink's V alone.
    sink_v = oracle.decode(vh, oracle.F16).reshape(blocks, kv_heads, BS, D)[table[0], :, 0, :]
    assert np.abs(exp.reshape(len(rows), q_heads, D)[-1] - np.repeat(sink_v, q_heads // kv_heads, 0)).max() > 1e-5


def test_decode_f16_peaked_rows(gpu):
    q_heads, kv_heads = 8, 2
    lens = np.array([32768, 4096, 9000], np.uint64)
    rng = np.random.default_rng(67)
    per = []
    for L in lens.tolist():
        per.append(peaked_cache(int(L), kv_heads, rng, blocks_extra=0))
    # one pool: the rows' pages back to back
    page = kv_heads * BS * D
    kh = np.concatenate([p[0] for p in per])
    vh = np.concatenate([p[1] for p in per])
    base, tables = 0, []
    for p in per:
        tables.append(p[2] + np.uint64(base))
        base += p[3]
    width = max(len(t) for t in tables)
    table = np.full((len(lens), width), 2**64 - 1, np.uint64)
    for i, t in enumerate(tables):
        table[i, :len(t)] = t
    blocks = base
    assert kh.size == blocks * page
    q = query_rows(len(lens), q_heads, per[0][4], rng)
    kc, vc, td, ld, qd = (buffer_like(x) for x in (kh, vh, table.reshape(-1), lens, q))
    out = buffer_like(np.zeros(q.size, np.float32))
    ws = C.c_size_t(0)
    capi.call("kvflux_paged_attention_workspace_size", len(lens), int(lens.max()), kv_heads, q_heads, BS, D,
              C.byref(ws))
    wd = device.DeviceBuffer(max(ws.value, 16))
    lib = capi.lib()
    assert lib.kvflux_paged_attention(kc.ptr, vc.ptr, blocks, kv_heads, BS, D, capi.DTYPE_F16, td.ptr, width, ld.ptr,
                                      int(lens.max()), len(lens), q_heads, qd.ptr, out.ptr, wd.ptr, ws.value,
                                      None) == 0, capi.last_error()
    device.synchronize()
    got = out.download(np.float32)
    exp = oracle.paged_attention_rows(kh, vh, kv_heads, BS, D, oracle.F16, table.reshape(-1), width, lens, q, q_heads,
                                      threads=8)
    err = np.abs(got - exp).max()
    assert err < 1e-5, err
    # The small keys carry weight: every row differs from its sink's V alone.
    for i, p in enumerate(per):
        sink = oracle.decode(p[1], oracle.F16).reshape(p[3], kv_heads, BS, D)[p[2][0], :, 0, :]
        row = exp.reshape(len(lens), q_heads, D)[i]
        assert np.abs(row - np.repeat(sink, q_heads // kv_heads, 0)).max() > 1e-5

