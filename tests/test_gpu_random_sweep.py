"""Seeded random sweep over the attention kernels' shape space, through the
C ABI, against the CPU oracle.

Each case draws a cache dtype, head_size, kv heads, GQA group, page size and
a batch, then checks
  * decode (kvflux_paged_attention): every output against the oracle at
    1e-5 (head sizes 16-512, so the split-K, MFMA and generic kernels all
    run), nothing written past the output;
  * batch prefill (kvflux_paged_prefill_batch): sampled rows of every
    sequence (first, middle, last, one random) against the oracle at 2e-2,
    nothing written past the output;
  * write then gather (kvflux_write_paged_kv, kvflux_gather_paged_kv): random
    bit patterns, bit-exact against the oracle over the whole arena and the
    whole outputs, and kvflux_gather_paged_kv_live identical to the table
    launch;
  * the exact prefill (kvflux_paged_prefill_exact): every output of one
    sequence against the oracle at 1e-5 (a quarter as many cases).
KVFLUX_SWEEP_CASES sets the number of cases per test (default 40);
KVFLUX_SWEEP_SEED the seed (default 777). The oracle's work per case is
bounded so a case takes well under a second.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np
import pytest

from gpu_util import DTYPES, buffer_like
from kvflux_amd import capi, device
from oracle import oracle

pytestmark = pytest.mark.gpu

CASES = int(os.environ.get("KVFLUX_SWEEP_CASES", "40"))
SEED = int(os.environ.get("KVFLUX_SWEEP_SEED", "777"))


def decode_case(rng, i):
    name = ("BFloat16", "Float16", "Float32")[int(rng.integers(3))]
    D = int(rng.choice([16, 32, 64, 80, 96, 128, 160, 256, 512]))
    H = int(rng.choice([1, 2, 4, 8]))
    Hq = H * int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 10, 12, 16, 24]))
    bs = int(rng.choice([1, 2, 4, 8, 16, 32, 64, 128, 256]))
    rows = int(rng.integers(1, 33))
    lens = rng.integers(1, int(rng.choice([64, 600, 5000, 20000])) + 1, rows).astype(np.uint64)
    while int(lens.sum()) * Hq * D > 4e8:  # bound the oracle's work
        lens = (lens // 2 + 1).astype(np.uint64)
    code, host = DTYPES[name]
    max_len = int(lens.max())
    width = (max_len + bs - 1) // bs
    P = width + 8
    page = H * bs * D
    kc = device.DeviceBuffer(P * page * np.dtype(host).itemsize)
    vc = device.DeviceBuffer(P * page * np.dtype(host).itemsize)
    device.fill_random(kc.ptr, P * page, code, 1, 1000 + i)
    device.fill_random(vc.ptr, P * page, code, 1, 2000 + i)
    table = rng.integers(0, P, (rows, width)).astype(np.uint64)
    for r in range(rows):
        table[r, (int(lens[r]) + bs - 1) // bs:] = 2**64 - 1
    q = oracle.random_elements(0, rows * Hq * D, oracle.F32, 1, 3000 + i)
    td, ld, qd = buffer_like(table.reshape(-1)), buffer_like(lens), buffer_like(q)
    lib = capi.lib()
    ws = C.c_size_t(0)
    capi.check(lib.kvflux_paged_attention_workspace_size(rows, max_len, H, Hq, bs, D, C.byref(ws)))
    wd = device.DeviceBuffer(max(ws.value, 256))
    od = buffer_like(np.full(q.size + 8, 7.0, np.float32))
    capi.check(lib.kvflux_paged_attention(kc.ptr, vc.ptr, P, H, bs, D, code, td.ptr, width, ld.ptr, max_len, rows,
                                          Hq, qd.ptr, od.ptr, wd.ptr, ws.value, None))
    device.synchronize()
    out = od.download(np.float32)
    cfg = f"decode {name} D={D} H={H} Hq={Hq} bs={bs} rows={rows} max_len={max_len}"
    assert np.all(out[q.size:] == 7.0), cfg
    exp = oracle.paged_attention_rows(kc.download(host), vc.download(host), H, bs, D, code, table.reshape(-1),
                                      width, lens, q, Hq, threads=8)
    err = float(np.abs(out[:q.size] - exp).max())
    assert err < 1e-5, (cfg, err)


def prefill_case(rng, i):
    name = ("BFloat16", "Float16")[int(rng.integers(2))]
    D = int(rng.choice([64, 128, 256]))
    H = int(rng.choice([1, 2, 4]))
    Hq = H * int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 10, 12, 16, 32]))
    bs = int(rng.choice([1, 2, 4, 8, 16, 32, 64, 128, 256]))
    seqs = []
    for _ in range(int(rng.integers(1, 6))):
        kv = int(rng.integers(1, int(rng.choice([200, 2000, 9000])) + 1))
        seqs.append((kv, kv if rng.random() < 0.5 else int(rng.integers(1, kv + 1))))
    n = len(seqs)
    code = DTYPES[name][0]
    width = max((kv + bs - 1) // bs for kv, _ in seqs) + 2
    blocks = n * width + 3
    page = H * bs * D
    kc, vc = device.DeviceBuffer(blocks * page * 2), device.DeviceBuffer(blocks * page * 2)
    device.fill_random(kc.ptr, blocks * page, code, 1, 4000 + i)
    device.fill_random(vc.ptr, blocks * page, code, 1, 5000 + i)
    order = rng.permutation(blocks).astype(np.uint64)
    table = np.full((n, width), 2**64 - 1, np.uint64)
    for k, (kv, _) in enumerate(seqs):
        npg = (kv + bs - 1) // bs
        table[k, :npg] = order[k * width:k * width + npg]
    q_lens = np.array([ql for _, ql in seqs], np.uint64)
    kv_lens = np.array([kv for kv, _ in seqs], np.uint64)
    offsets = np.concatenate([[0], np.cumsum(q_lens)[:-1]]).astype(np.uint64)
    rows_total, row = int(q_lens.sum()), Hq * D
    q = oracle.random_elements(0, rows_total * row, oracle.F32, 1, 6000 + i)
    td, qd = buffer_like(table.reshape(-1)), buffer_like(q)
    kd, ld, od_ = buffer_like(kv_lens), buffer_like(q_lens), buffer_like(offsets)
    out = buffer_like(np.full(rows_total * row + 8, 555.0, np.float32))
    lib = capi.lib()
    capi.check(lib.kvflux_paged_prefill_batch(kc.ptr, vc.ptr, blocks, H, bs, D, code, td.ptr, width, kd.ptr, ld.ptr,
                                              od_.ptr, n, int(q_lens.max()), int(kv_lens.max()), Hq, qd.ptr, out.ptr,
                                              None))
    device.synchronize()
    got = out.download(np.float32)
    cfg = f"prefill {name} D={D} H={H} Hq={Hq} bs={bs} seqs={seqs}"
    assert np.all(got[rows_total * row:] == 555.0), cfg
    got = got[:rows_total * row].reshape(rows_total, row)
    kh, vh = kc.download(np.uint16), vc.download(np.uint16)
    for k, (kv, ql) in enumerate(seqs):
        o0 = int(offsets[k])
        qi = q.reshape(rows_total, row)[o0:o0 + ql]
        pick = sorted({0, ql - 1, ql // 2, int(rng.integers(ql))})
        exp = oracle.paged_attention_rows(kh, vh, H, bs, D, code, np.tile(table[k], len(pick)), width,
                                          np.array([kv - ql + t + 1 for t in pick], np.uint64),
                                          qi[pick].reshape(-1), Hq, threads=8)
        err = float(np.abs(got[o0:o0 + ql][pick].reshape(-1) - exp).max())
        assert err < 2e-2, (cfg, k, err)


def write_gather_case(rng, i):
    """A scattered write of random bit patterns (NaN encodings included) into
    a pre-filled arena, then a ragged gather of random sequences: both
    bit-exact against the oracle, whole arena and whole outputs compared."""
    name = ("BFloat16", "Float16", "Float32")[int(rng.integers(3))]
    code, host = DTYPES[name]
    H = int(rng.integers(1, 9))
    D = int(rng.choice([1, 2, 3, 5, 8, 16, 24, 64, 96, 128, 256, 512]))
    bs = int(rng.choice([1, 2, 4, 8, 16, 32, 64, 128, 256]))
    page = H * bs * D
    itemsize = np.dtype(host).itemsize
    blocks = int(min(rng.integers(1, 200), max(1, 32e6 // (page * itemsize))))  # arenas up to 32 MB
    bits = np.uint32 if itemsize == 4 else np.uint16
    arena_k = rng.integers(0, np.iinfo(bits).max, blocks * page, dtype=np.uint64).astype(bits)
    arena_v = rng.integers(0, np.iinfo(bits).max, blocks * page, dtype=np.uint64).astype(bits)
    kc, vc = buffer_like(arena_k), buffer_like(arena_v)
    tokens = int(rng.integers(1, min(blocks * bs, 4096) + 1))
    slots = rng.choice(blocks * bs, tokens, replace=False).astype(np.uint64)
    kn = rng.integers(0, np.iinfo(bits).max, tokens * H * D, dtype=np.uint64).astype(bits)
    vn = rng.integers(0, np.iinfo(bits).max, tokens * H * D, dtype=np.uint64).astype(bits)
    knd, vnd, sd = buffer_like(kn), buffer_like(vn), buffer_like(slots)
    lib = capi.lib()
    capi.check(lib.kvflux_write_paged_kv(kc.ptr, vc.ptr, blocks, H, bs, D, code, knd.ptr, vnd.ptr, sd.ptr, tokens,
                                         None))
    device.synchronize()
    oracle.write_paged_kv(arena_k, arena_v, H, bs, D, code, kn, vn, slots)
    cfg = f"write {name} H={H} D={D} bs={bs} blocks={blocks} tokens={tokens}"
    assert np.array_equal(kc.download(bits), arena_k), cfg
    assert np.array_equal(vc.download(bits), arena_v), cfg
    # gather: 1-6 sequences over random pages of the written arena
    n = int(rng.integers(1, 7))
    lens = rng.integers(1, blocks * bs + 1, n).astype(np.uint64)
    while int(lens.sum()) * H * D * itemsize > 32e6:  # outputs up to 32 MB
        lens = (lens // 2 + 1).astype(np.uint64)
    width = int((lens.max() + bs - 1) // bs)
    table = rng.integers(0, blocks, (n, width)).astype(np.uint64)
    offsets = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.uint64)
    total = int(lens.sum())
    row = H * D
    ko = buffer_like(np.full(total * row + 8, 0x5A, bits))
    vo = buffer_like(np.full(total * row + 8, 0x5A, bits))
    td, ld, od_ = buffer_like(table.reshape(-1)), buffer_like(lens), buffer_like(offsets)
    capi.check(lib.kvflux_gather_paged_kv(kc.ptr, vc.ptr, blocks, H, bs, D, code, td.ptr, width, ld.ptr, od_.ptr, n,
                                          int(lens.max()), ko.ptr, vo.ptr, None))
    device.synchronize()
    kg, vg = ko.download(bits), vo.download(bits)
    cfg = f"gather {name} H={H} D={D} bs={bs} lens={lens.tolist()}"
    assert np.all(kg[total * row:] == 0x5A) and np.all(vg[total * row:] == 0x5A), cfg
    for k in range(n):
        o0, L = int(offsets[k]) * row, int(lens[k])
        ek, ev = oracle.gather_paged_kv(arena_k, arena_v, H, bs, D, code, table[k], L)
        assert np.array_equal(kg[o0:o0 + L * row], ek.view(bits)), cfg
        assert np.array_equal(vg[o0:o0 + L * row], ev.view(bits)), cfg
    # the live-page launch on the same batch: identical outputs, nothing past them
    counts = (lens + bs - 1) // bs
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.uint64)
    ko2 = buffer_like(np.full(total * row + 8, 0x33, bits))
    vo2 = buffer_like(np.full(total * row + 8, 0x33, bits))
    sd2 = buffer_like(starts)
    capi.check(lib.kvflux_gather_paged_kv_live(kc.ptr, vc.ptr, blocks, H, bs, D, code, td.ptr, width, ld.ptr,
                                               od_.ptr, sd2.ptr, n, int(counts.sum()), ko2.ptr, vo2.ptr, None))
    device.synchronize()
    kg2, vg2 = ko2.download(bits), vo2.download(bits)
    assert np.all(kg2[total * row:] == 0x33) and np.all(vg2[total * row:] == 0x33), cfg
    assert np.array_equal(kg2[:total * row], kg[:total * row]), cfg
    assert np.array_equal(vg2[:total * row], vg[:total * row]), cfg


def exact_prefill_case(rng, i):
    """kvflux_paged_prefill_exact on one sequence (a whole prompt or a
    trailing chunk, with its workspace so keys may split; 16-bit or FP32
    caches): every output against the oracle at 1e-5."""
    name = ("BFloat16", "Float16", "Float32")[int(rng.integers(3))]
    D = int(rng.choice([64, 128]))
    H = int(rng.choice([1, 2, 4]))
    Hq = H * int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 10, 12, 16]))
    bs = int(rng.choice([1, 2, 4, 8, 16, 32, 64, 128, 256]))
    kv = int(rng.integers(16, int(rng.choice([300, 3000, 12000])) + 1))
    ql = kv if rng.random() < 0.5 else int(rng.integers(16, kv + 1))
    while ql * kv * Hq * D > 2e9:  # bound the oracle's work
        ql = max(16, ql // 2)
    code, host = DTYPES[name]
    esize = np.dtype(host).itemsize
    npg = (kv + bs - 1) // bs
    blocks = npg + 5
    page = H * bs * D
    kc, vc = device.DeviceBuffer(blocks * page * esize), device.DeviceBuffer(blocks * page * esize)
    device.fill_random(kc.ptr, blocks * page, code, 1, 7000 + i)
    device.fill_random(vc.ptr, blocks * page, code, 1, 8000 + i)
    table = rng.permutation(blocks)[:npg].astype(np.uint64)
    q = oracle.random_elements(0, ql * Hq * D, oracle.F32, 1, 9000 + i)
    lib = capi.lib()
    ws = C.c_size_t(0)
    capi.check(lib.kvflux_paged_prefill_workspace_size(H, D, kv, ql, Hq, C.byref(ws)))
    wd = device.DeviceBuffer(max(ws.value, 256))
    td, qd = buffer_like(table), buffer_like(q)
    od = buffer_like(np.full(q.size + 8, 555.0, np.float32))
    capi.check(lib.kvflux_paged_prefill_exact(kc.ptr, vc.ptr, blocks, H, bs, D, code, td.ptr, npg, kv, ql, Hq, qd.ptr,
                                              od.ptr, wd.ptr, ws.value, None))
    device.synchronize()
    out = od.download(np.float32)
    cfg = f"exact prefill {name} D={D} H={H} Hq={Hq} bs={bs} kv={kv} q={ql}"
    assert np.all(out[q.size:] == 555.0), cfg
    exp = oracle.paged_attention_causal(kc.download(host), vc.download(host), H, bs, D, code, table, kv, q,
                                        ql, Hq, threads=8)
    err = float(np.abs(out[:q.size] - exp).max())
    assert err < 1e-5, (cfg, err)


def test_random_exact_prefill(gpu):
    rng = np.random.default_rng(SEED + 2)
    for i in range(max(1, CASES // 4)):
        exact_prefill_case(rng, i)


def test_random_sweep(gpu):
    rng = np.random.default_rng(SEED)
    for i in range(CASES):
        (decode_case if i % 2 == 0 else prefill_case)(rng, i)


def test_random_write_gather(gpu):
    rng = np.random.default_rng(SEED + 1)
    for i in range(CASES):
        write_gather_case(rng, i)
