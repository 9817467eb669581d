"""Live-page gather over many sequences, the page-list copy and the bandwidth
probe, through the C ABI.

* kvflux_gather_paged_kv_live finds each workgroup's sequence with a 64-ary
  search over the scan of the page counts: one level up to 64 sequences, two
  up to 4096, three beyond. The batches below take 1, 2 and 3 levels, with
  runs of empty sequences (equal scan entries) at the start, the middle and
  the end; the output is bit-exact against the oracle gather
  (paged_kv_read.cu:67-87 restated) and identical to the table launch's.
* kvflux_copy_page_list: page i of the destination equals page src_pages[i]
  of the source (numpy indexing is the check), ids past the source are
  skipped (the destination keeps its bytes).
* kvflux_bandwidth_probe: the copy moves every byte, the write stores its
  fixed pattern, the read leaves its sink alone; bad shapes are rejected.
  kvflux_bandwidth_probe_pages: the same for the page-list read.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import buffer_like
from kvflux_amd import capi, device
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("num_seqs", [64, 700, 5000])
def test_live_gather_many_sequences(gpu, num_seqs):
    H, D, bs = 2, 8, 4  # FP16 rows of 16 bytes: pages of 128 bytes
    rng = np.random.default_rng(num_seqs)
    lens = rng.integers(0, 3 * bs + 2, num_seqs)
    lens[:5] = 0
    lens[num_seqs // 2:num_seqs // 2 + 7] = 0
    lens[-3:] = 0
    lens[1 + num_seqs // 3] = 1
    counts = (lens + bs - 1) // bs
    blocks = int(counts.sum()) + 17
    width = int(counts.max())
    perm = rng.permutation(blocks).astype(np.uint64)
    table = np.full((num_seqs, width), 2**64 - 1, np.uint64)
    used = 0
    for i, c in enumerate(counts.tolist()):
        table[i, :c] = perm[used:used + c]
        used += c
    page = H * bs * D
    k_host = rng.integers(0, 2**16, blocks * page, dtype=np.uint16)
    v_host = rng.integers(0, 2**16, blocks * page, dtype=np.uint16)
    kc, vc = buffer_like(k_host), buffer_like(v_host)
    offsets = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.uint64)
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.uint64)
    total = int(lens.sum())
    td, ld, od, sd = (buffer_like(a) for a in (table.reshape(-1), lens.astype(np.uint64), offsets, starts))
    out = {}
    for entry in ("table", "live"):
        ko = buffer_like(np.full(total * H * D + 32, 0xA5A5, np.uint16))
        vo = buffer_like(np.full(total * H * D + 32, 0xA5A5, np.uint16))
        if entry == "table":
            st = capi.lib().kvflux_gather_paged_kv(kc.ptr, vc.ptr, blocks, H, bs, D, capi.DTYPE_F16, td.ptr, width,
                                                   ld.ptr, od.ptr, num_seqs, int(lens.max()), ko.ptr, vo.ptr, None)
        else:
            st = capi.lib().kvflux_gather_paged_kv_live(kc.ptr, vc.ptr, blocks, H, bs, D, capi.DTYPE_F16, td.ptr,
                                                        width, ld.ptr, od.ptr, sd.ptr, num_seqs, int(counts.sum()),
                                                        ko.ptr, vo.ptr, None)
        assert st == 0, capi.last_error()
        device.synchronize()
        out[entry] = (ko.download(np.uint16), vo.download(np.uint16))
    kg, vg = out["live"]
    assert np.all(kg[total * H * D:] == 0xA5A5) and np.all(vg[total * H * D:] == 0xA5A5)
    assert np.array_equal(kg, out["table"][0]) and np.array_equal(vg, out["table"][1])
    for i in range(num_seqs):
        n = int(lens[i])
        if n == 0:
            continue
        ek, ev = oracle.gather_paged_kv(k_host, v_host, H, bs, D, oracle.F16, table[i], n)
        o = int(offsets[i]) * H * D
        assert np.array_equal(kg[o:o + n * H * D], ek), i
        assert np.array_equal(vg[o:o + n * H * D], ev), i


@pytest.mark.parametrize("page_bytes", [16384, 32768, 48, 5])
def test_copy_page_list(gpu, page_bytes):
    rng = np.random.default_rng(page_bytes)
    blocks, n = 40, 25
    src_host = rng.integers(0, 256, blocks * page_bytes, dtype=np.uint8)
    dst_host = rng.integers(0, 256, n * page_bytes, dtype=np.uint8)
    ids = rng.choice(blocks, n, replace=False).astype(np.uint64)
    ids[7] = blocks + 3  # past the source: skipped
    src, dst, idd = buffer_like(src_host), buffer_like(dst_host), buffer_like(ids)
    assert capi.lib().kvflux_copy_page_list(dst.ptr, src.ptr, blocks, page_bytes, idd.ptr, n, None) == 0, \
        capi.last_error()
    device.synchronize()
    got = dst.download(np.uint8).reshape(n, page_bytes)
    pages = src_host.reshape(blocks, page_bytes)
    for i in range(n):
        want = dst_host.reshape(n, page_bytes)[i] if i == 7 else pages[int(ids[i])]
        assert np.array_equal(got[i], want), i


@pytest.mark.parametrize("threads,vpt,grid,nt", [(512, 1, 0, 1), (256, 4, 64, 0), (1024, 8, 0, 1), (512, 2, 3, 0)])
def test_bandwidth_probe(gpu, threads, vpt, grid, nt):
    step = 16 * threads * vpt
    nbytes = 5 * step
    rng = np.random.default_rng(threads + vpt)
    src_host = rng.integers(0, 256, nbytes, dtype=np.uint8)
    src = buffer_like(src_host)
    dst = buffer_like(np.zeros(nbytes, np.uint8))
    lib = capi.lib()
    assert lib.kvflux_bandwidth_probe(0, dst.ptr, src.ptr, nbytes, threads, vpt, grid, nt, None) == 0
    device.synchronize()
    assert np.array_equal(dst.download(np.uint8), src_host)
    assert lib.kvflux_bandwidth_probe(1, dst.ptr, None, nbytes, threads, vpt, grid, nt, None) == 0
    device.synchronize()
    words = dst.download(np.uint32).reshape(-1, 4)
    lane = np.arange(words.shape[0]) % threads
    assert np.all(words[:, 0] == 0x6B766678) and np.all(words[:, 1] == 0x75782031)
    assert np.all(words[:, 2] == (0x6B766678 ^ lane)) and np.all(words[:, 3] == 0x75782032)
    sink = buffer_like(np.full(threads * 16, 0x3C, np.uint8))
    assert lib.kvflux_bandwidth_probe(2, sink.ptr, src.ptr, nbytes, threads, vpt, grid, nt, None) == 0
    device.synchronize()
    assert np.all(sink.download(np.uint8) == 0x3C)
    # shapes outside the instantiated set and sizes off the step are rejected
    assert lib.kvflux_bandwidth_probe(0, dst.ptr, src.ptr, nbytes, 128, vpt, grid, nt, None) != 0
    assert lib.kvflux_bandwidth_probe(0, dst.ptr, src.ptr, nbytes, threads, 3, grid, nt, None) != 0
    assert lib.kvflux_bandwidth_probe(0, dst.ptr, src.ptr, nbytes - 16, threads, vpt, grid, nt, None) != 0
    assert lib.kvflux_bandwidth_probe(3, dst.ptr, src.ptr, nbytes, threads, vpt, grid, nt, None) != 0


@pytest.mark.parametrize("threads,vpt,nt", [(256, 1, 1), (512, 2, 0), (1024, 2, 1)])
def test_bandwidth_probe_pages(gpu, threads, vpt, nt):
    """The page-list read probe reads in bounds (ids past the pool skipped),
    leaves its sink alone and rejects page sizes off its part size."""
    page_bytes = 16 * 1024 * 2  # 32 KiB: one part at 1024 x 2, eight at 256 x 1
    blocks = 12
    rng = np.random.default_rng(threads * 3 + vpt)
    kc = buffer_like(rng.integers(0, 256, blocks * page_bytes, dtype=np.uint8))
    vc = buffer_like(rng.integers(0, 256, blocks * page_bytes, dtype=np.uint8))
    pages = buffer_like(np.array([3, 0, 11, 7, blocks, 2**64 - 1, 5], np.uint64))
    sink = buffer_like(np.full(threads * 16, 0x5A, np.uint8))
    lib = capi.lib()
    assert lib.kvflux_bandwidth_probe_pages(kc.ptr, vc.ptr, blocks, page_bytes, pages.ptr, 7, threads, vpt, nt,
                                            sink.ptr, None) == 0, capi.last_error()
    device.synchronize()
    assert np.all(sink.download(np.uint8) == 0x5A)
    assert lib.kvflux_bandwidth_probe_pages(kc.ptr, vc.ptr, blocks, page_bytes, pages.ptr, 0, threads, vpt, nt,
                                            sink.ptr, None) == 0
    assert lib.kvflux_bandwidth_probe_pages(kc.ptr, vc.ptr, blocks, page_bytes - 16, pages.ptr, 7, threads, vpt,
                                            nt, sink.ptr, None) != 0
    assert lib.kvflux_bandwidth_probe_pages(kc.ptr, vc.ptr, blocks, page_bytes, pages.ptr, 7, 128, vpt, nt,
                                            sink.ptr, None) != 0
