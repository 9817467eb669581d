"""kvflux_paged_attention_noalloc: the decode entry point that allocates
nothing (chunk partials in a static device array) against
kvflux_paged_attention with a caller workspace.

Both run the same kernels with the same partial layout, so outputs must be
bit-identical; sampled rows are also checked against the oracle at 1e-5.
Two calls in a row, the second on a smaller batch, show that the scratch
left by the first call does not leak into the second. A call whose partials
exceed the static array is rejected before anything is launched.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from gpu_util import DTYPES, buffer_like
from kvflux_amd import capi, device
from oracle import oracle

pytestmark = pytest.mark.gpu
TOL = 1e-5
SCRATCH_BYTES = 32 << 20


def _batch(rng, rows, max_len, P, bs):
    lens = rng.integers(1, max_len + 1, rows).astype(np.uint64)
    lens[0] = max_len
    width = (max_len + bs - 1) // bs
    table = rng.integers(0, P, (rows, width)).astype(np.uint64)
    for r in range(rows):  # entries past a row's pages are never read: poison them
        table[r, (int(lens[r]) + bs - 1) // bs:] = 2**64 - 1
    return lens, table, width


@pytest.mark.parametrize("name,H,Hq,head_size", [("BFloat16", 8, 32, 128), ("Float32", 2, 8, 128),
                                                 ("Float16", 2, 10, 64)])
def test_noalloc_matches_workspace_entry(gpu, name, H, Hq, head_size):
    lib = capi.lib()
    bs, P = 16, 2048
    code = DTYPES[name][0]
    esize = 4 if name == "Float32" else 2
    page = H * bs * head_size
    kc, vc = device.DeviceBuffer(P * page * esize), device.DeviceBuffer(P * page * esize)
    device.fill_random(kc.ptr, P * page, code, 1, 71)
    device.fill_random(vc.ptr, P * page, code, 1, 72)
    kh = kc.download(np.float32 if esize == 4 else np.uint16)
    vh = vc.download(np.float32 if esize == 4 else np.uint16)
    rng = np.random.default_rng(Hq * 1000 + head_size)
    for rows, max_len in ((48, 12000), (9, 2500)):  # the second call is smaller
        print(f"noalloc case {name} H={H} Hq={Hq} D={head_size} rows={rows} max_len={max_len}", flush=True)
        lens, table, width = _batch(rng, rows, max_len, P, bs)
        td, ld = buffer_like(table.reshape(-1)), buffer_like(lens)
        q = oracle.random_elements(0, rows * Hq * head_size, oracle.F32, 1, rows + max_len)
        qd = buffer_like(q)
        ws = C.c_size_t(0)
        capi.check(lib.kvflux_paged_attention_workspace_size(rows, max_len, H, Hq, bs, head_size, C.byref(ws)))
        wd = device.DeviceBuffer(max(ws.value, 256))
        ref_out = buffer_like(np.full(q.size, 7.0, np.float32))
        capi.check(lib.kvflux_paged_attention(kc.ptr, vc.ptr, P, H, bs, head_size, code, td.ptr, width, ld.ptr,
                                              max_len, rows, Hq, qd.ptr, ref_out.ptr, wd.ptr, ws.value, None))
        got_out = buffer_like(np.full(q.size, 9.0, np.float32))
        capi.check(lib.kvflux_paged_attention_noalloc(kc.ptr, vc.ptr, P, H, bs, head_size, code, td.ptr, width,
                                                      ld.ptr, max_len, rows, Hq, qd.ptr, got_out.ptr, None))
        device.synchronize()
        ref, got = ref_out.download(np.float32), got_out.download(np.float32)
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32))
        sample = np.array(sorted({0, rows - 1, *rng.choice(rows, 4, replace=False).tolist()}))
        exp = oracle.paged_attention_rows(kh, vh, H, bs, head_size, code, table[sample].reshape(-1), width,
                                          lens[sample], q.reshape(rows, -1)[sample].reshape(-1), Hq, threads=8)
        assert np.abs(got.reshape(rows, -1)[sample].reshape(-1) - exp).max() < TOL


def test_noalloc_rejects_partials_beyond_the_scratch(gpu):
    """256 rows of 64K tokens at 32 query heads with an FP32 cache take
    4096-token work items on the block-size-16 kernel: 16 chunk partials per
    (row, query head), 68 MB. The call fails on the host with
    KVFLUX_ERR_UNSUPPORTED; nothing is launched and the output is
    untouched."""
    lib = capi.lib()
    H, Hq, D, bs = 8, 32, 128, 16
    rows, kv_len = 256, 65536
    dummy = device.DeviceBuffer(1 << 12)
    out = buffer_like(np.full(rows * Hq * D, 5.0, np.float32))
    status = lib.kvflux_paged_attention_noalloc(dummy.ptr, dummy.ptr, 1, H, bs, D, capi.DTYPE_F32, dummy.ptr, 1,
                                                dummy.ptr, kv_len, rows, Hq, dummy.ptr, out.ptr, None)
    assert status == capi.ERR_UNSUPPORTED
    assert b"static scratch" in capi.lib().kvflux_last_error()
    device.synchronize()
    assert np.all(out.download(np.float32) == 5.0)
