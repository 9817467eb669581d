"""The benchmark configurations at full size, through properties that do not
need the oracle to process the whole workload:

* write (4096 tokens x 8 heads x 128, BF16, 65536-page pool): every touched
  page bit-exact against the oracle's scatter, untouched slots keep 0xA5;
* gather (64 sequences, L ~ U[512, 8192], odd pages of a full pool, BF16 and
  FP16): write -> batched gather round trip is the identity, checked on the
  device byte for byte;
* batch decode (B=128, L ~ U[1024, 32768], 32/8 heads, shared 2048-token
  prefix, 2^18-page pool): sampled rows against the oracle at 1e-5,
  bit-identical repeat, and with every V row equal to one constant the output
  equals that constant (the softmax weights sum to one);
* causal prefill (4096-token sequences, 32/8 heads): sampled rows against
  the oracle at 2e-2.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from gpu_util import buffer_like
from kvflux_amd import capi, device
from oracle import oracle

pytestmark = pytest.mark.gpu


def fragment(pool, order):
    """Allocate every page, free `order` reversed: allocations then follow `order`."""
    held = [pool.allocate() for _ in range(pool.capacity())]
    for idx in np.asarray(order)[::-1]:
        pool.free(held[int(idx)])
    keep = np.ones(pool.capacity(), bool)
    keep[np.asarray(order)] = False
    return [held[i] for i in np.nonzero(keep)[0]]


def test_write_full_size(gpu, v2):
    H, D, bs = 8, 128, 16
    rng = np.random.default_rng(11)
    pool = v2.PhysicalBlockPool(65536, bs)
    storage = v2.PagedKVStorage(pool, H, D, v2.DType.BFloat16)
    fragment(pool, rng.permutation(pool.capacity()))
    capi.call("kvflux_fill_bytes", C.c_void_p(storage.key_base()), 0xA5, storage.layout().total_bytes(), None)
    seqs, writes = [], []
    for i, L0 in enumerate(rng.integers(0, 2048, 256).tolist()):
        s = v2.SequenceState(i, pool)
        s.append_tokens(L0 + 16)
        seqs.append(s)
        writes += [(s, L0 + j) for j in range(16)]
    slots = np.array(v2.build_slot_mapping(writes), np.uint64)
    N = slots.size
    kn, vn = device.DeviceBuffer(N * H * D * 2), device.DeviceBuffer(N * H * D * 2)
    device.fill_random(kn.ptr, N * H * D, capi.DTYPE_BF16, 1, 12)
    device.fill_random(vn.ptr, N * H * D, capi.DTYPE_BF16, 1, 13)
    v2.write_paged_kv(storage, kn.ptr, vn.ptr, slots.tolist())
    page_elems = H * bs * D
    pages = np.unique(slots // bs)
    remap = {int(p): j for j, p in enumerate(pages.tolist())}
    host_k = np.full(pages.size * page_elems, 0xA5A5, np.uint16)
    host_v = host_k.copy()
    oracle.write_paged_kv(host_k, host_v, H, bs, D, oracle.BF16, kn.download(np.uint16), vn.download(np.uint16),
                          np.array([remap[int(s // bs)] * bs + int(s % bs) for s in slots], np.uint64))
    kb, vb = storage.key_base(), storage.value_base()
    for j, pg in enumerate(pages.tolist()):
        assert np.array_equal(device.memcpy_d2h(kb + pg * page_elems * 2, page_elems * 2, np.uint16),
                              host_k[j * page_elems:(j + 1) * page_elems])
        assert np.array_equal(device.memcpy_d2h(vb + pg * page_elems * 2, page_elems * 2, np.uint16),
                              host_v[j * page_elems:(j + 1) * page_elems])
    # a page nobody wrote is still all 0xA5
    untouched = int(np.setdiff1d(np.arange(200), pages)[0])
    assert np.all(device.memcpy_d2h(kb + untouched * page_elems * 2, page_elems * 2, np.uint8) == 0xA5)


@pytest.mark.parametrize("name", ["BFloat16", "Float16"])
def test_gather_round_trip_full_size(gpu, v2, name):
    H, D, bs, S = 8, 128, 16, 64
    code = capi.DTYPE_BF16 if name == "BFloat16" else capi.DTYPE_F16
    rng = np.random.default_rng(21)
    lens = rng.integers(512, 8192 + 1, S)
    pool = v2.PhysicalBlockPool(65536, bs)
    storage = v2.PagedKVStorage(pool, H, D, getattr(v2.DType, name))
    fragment(pool, rng.permutation(np.arange(1, pool.capacity(), 2)))
    seqs = []
    for i, L in enumerate(lens.tolist()):
        s = v2.SequenceState(i, pool)
        s.append_tokens(L)
        seqs.append(s)
    assert all(int(seqs[0].physical_block_id(b)) % 2 == 1 for b in range(4))
    total = int(lens.sum())
    kn, vn = device.DeviceBuffer(total * H * D * 2), device.DeviceBuffer(total * H * D * 2)
    device.fill_random(kn.ptr, total * H * D, code, 0, 22)
    device.fill_random(vn.ptr, total * H * D, code, 0, 23)
    writes = [(s, t) for s, L in zip(seqs, lens.tolist()) for t in range(L)]
    v2.write_paged_kv(storage, kn.ptr, vn.ptr, v2.build_slot_mapping(writes))
    ko, vo = device.DeviceBuffer(total * H * D * 2), device.DeviceBuffer(total * H * D * 2)
    ko.fill(0x5A)
    vo.fill(0x5A)
    v2.read_paged_kv_batch(storage, seqs, ko.ptr, vo.ptr)
    assert device.compare_bytes(ko.ptr, kn.ptr, total * H * D * 2) == 0
    assert device.compare_bytes(vo.ptr, vn.ptr, total * H * D * 2) == 0


@pytest.fixture(scope="module")
def decode_batch(v2):
    """The decode benchmark batch: 128 rows, shared prefix, 2^18-page pool."""
    from kvflux_amd import capi as _capi
    if _capi.device_count() == 0:
        pytest.skip("no GPU visible")
    _capi.call("kvflux_set_device", 0)
    B, H, Hq, D, bs, prefix = 128, 8, 32, 128, 16, 2048
    rng = np.random.default_rng(2024)
    lens = rng.integers(1024, 32768 + 1, B)
    lens[3] = prefix  # one row that is exactly the shared prefix
    pool = v2.PhysicalBlockPool(1 << 18, bs)
    storage = v2.PagedKVStorage(pool, H, D, v2.DType.BFloat16)
    fragment(pool, rng.permutation(pool.capacity()))
    base = v2.SequenceState(10**9, pool)
    base.append_tokens(prefix)
    seqs = []
    for i, L in enumerate(lens.tolist()):
        if L >= prefix:  # shares the prefix pages, like the benchmark batch
            s = base.fork_shared(i)
            s.append_tokens(L - prefix)
        else:
            s = v2.SequenceState(i, pool)
            s.append_tokens(L)
        seqs.append(s)
    n = storage.layout().cache_bytes() // 2
    device.fill_random(storage.key_base(), n, _capi.DTYPE_BF16, 1, 2025)
    device.fill_random(storage.value_base(), n, _capi.DTYPE_BF16, 1, 2026)
    q = oracle.random_elements(0, B * Hq * D, oracle.F32, 1, 2027)
    return dict(pool=pool, storage=storage, seqs=seqs, base=base, lens=lens, q=q, B=B, H=H, Hq=Hq, D=D, bs=bs)


def test_decode_full_size_rows_and_repeat(gpu, v2, decode_batch):
    d = decode_batch
    qd = buffer_like(d["q"])
    od, od2 = buffer_like(np.zeros_like(d["q"])), buffer_like(np.zeros_like(d["q"]))
    v2.paged_attention_batch(d["storage"], d["seqs"], qd.ptr, od.ptr, d["Hq"])
    v2.paged_attention_batch(d["storage"], d["seqs"], qd.ptr, od2.ptr, d["Hq"])
    got = od.download(np.float32)
    assert np.array_equal(got.view(np.uint32), od2.download(np.float32).view(np.uint32))
    assert np.all(np.isfinite(got))
    H, Hq, D, bs = d["H"], d["Hq"], d["D"], d["bs"]
    page_elems = H * bs * D
    kb, vb = d["storage"].key_base(), d["storage"].value_base()
    lens = d["lens"]
    # 32+ rows: the shortest, the longest, the prefix-only row, rows just
    # below and above the prefix length, and a seeded sample of the rest.
    shared = int(np.flatnonzero(lens == 2048)[0])
    near = [int(np.argmin(np.where(lens < 2048, 2048 - lens, 1 << 30))),
            int(np.argmin(np.where(lens > 2048, lens - 2048, 1 << 30)))]
    picked = {int(np.argmin(lens)), int(np.argmax(lens)), shared, *near}
    picked |= set(np.random.default_rng(7).choice(d["B"], 40, replace=False).tolist())
    picked = sorted(picked)[:max(32, len(picked))]
    assert len(picked) >= 32
    for r in picked:
        L = int(lens[r])
        ids = v2.build_read_block_table(d["seqs"][r])
        kc = np.concatenate([device.memcpy_d2h(kb + p * page_elems * 2, page_elems * 2, np.uint16) for p in ids])
        vc = np.concatenate([device.memcpy_d2h(vb + p * page_elems * 2, page_elems * 2, np.uint16) for p in ids])
        exp = oracle.paged_attention_rows(kc, vc, H, bs, D, oracle.BF16, np.arange(len(ids), dtype=np.uint64),
                                          len(ids), np.array([L], np.uint64), d["q"][r * Hq * D:(r + 1) * Hq * D],
                                          Hq, threads=8)
        assert np.abs(got[r * Hq * D:(r + 1) * Hq * D] - exp).max() < 1e-5


def test_decode_full_size_constant_values(gpu, v2, decode_batch):
    """Every V element = 0x3F3F (0.74609375 in BF16): every output equals it."""
    d = decode_batch
    storage = d["storage"]
    capi.call("kvflux_fill_bytes", C.c_void_p(storage.value_base()), 0x3F, storage.layout().cache_bytes(), None)
    qd = buffer_like(d["q"])
    od = buffer_like(np.zeros_like(d["q"]))
    v2.paged_attention_batch(storage, d["seqs"], qd.ptr, od.ptr, d["Hq"])
    got = od.download(np.float32)
    assert np.abs(got - np.float32(0.74609375)).max() < 1e-6


def test_prefill_full_size_sampled_rows(gpu, v2):
    """The prefill configuration in full: 8 sequences of 4096 tokens written
    through slot mappings into random pages of one pool, each prefilled on the
    MFMA kernel; 16+ rows of every sequence, spread over its length (first and
    last tokens, tile and page boundaries, a seeded sample), within 2e-2 of
    the reference attention on that sequence's contiguous K/V."""
    S, H, Hq, D, bs, T = 8, 8, 32, 128, 16, 4096
    rng = np.random.default_rng(31)
    pool = v2.PhysicalBlockPool(S * T // bs + 64, bs)
    storage = v2.PagedKVStorage(pool, H, D, v2.DType.BFloat16)
    fragment(pool, rng.permutation(pool.capacity()))
    kn, vn = device.DeviceBuffer(T * H * D * 2), device.DeviceBuffer(T * H * D * 2)
    qd, od = device.DeviceBuffer(T * Hq * D * 4), device.DeviceBuffer(T * Hq * D * 4)
    seqs = []  # all eight stay alive: their pages are distinct
    for i in range(S):
        seq = v2.SequenceState(i, pool)
        seqs.append(seq)
        seq.append_tokens(T)
        device.fill_random(kn.ptr, T * H * D, capi.DTYPE_BF16, 1, 32 + 3 * i)
        device.fill_random(vn.ptr, T * H * D, capi.DTYPE_BF16, 1, 33 + 3 * i)
        v2.write_paged_kv(storage, kn.ptr, vn.ptr, v2.build_slot_mapping([(seq, t) for t in range(T)]))
        q = oracle.random_elements(0, T * Hq * D, oracle.F32, 1, 34 + 3 * i)
        qd.upload(q)
        v2.paged_attention(storage, seq, qd.ptr, od.ptr, T, Hq, v2.AttentionPrecision.Fast)
        got = od.download(np.float32).reshape(T, Hq * D)
        assert np.all(np.isfinite(got))
        k_host = kn.download(np.uint16).reshape(T, H, D)
        v_host = vn.download(np.uint16).reshape(T, H, D)
        qr = q.reshape(T, Hq * D)
        rows = {0, 1, 15, 16, 63, 64, 1000, 2047, 2048, 4094, 4095} | set(rng.integers(0, T, 6).tolist())
        for t in sorted(rows):
            # token t sees tokens 0..t: contiguous K/V of those tokens, one query row
            exp = oracle.reference_attention(qr[t], oracle.decode(k_host[:t + 1].reshape(-1), oracle.BF16),
                                             oracle.decode(v_host[:t + 1].reshape(-1), oracle.BF16), 1, t + 1,
                                             Hq, H, D)
            assert np.abs(got[t] - exp).max() < 2e-2, (i, t)


def test_prefill_batch_launch_full_size(gpu, v2):
    """The launch the prefill benchmark times, at its full size:
    kvflux_paged_prefill_batch over 8 sequences of 4096 tokens (32 q / 8 kv
    heads, D=128, BF16) written through slot mappings into random pages of
    one pool, Q of all sequences in one buffer, the tables as the rows of one
    batch table. Every sequence's output is bit-identical to
    kvflux_paged_prefill on that sequence alone, and 16+ rows of every
    sequence, spread over its length (first and last tokens, tile and page
    boundaries, a seeded sample), are within 2e-2 of the reference attention
    on that sequence's contiguous K/V (tests/paged_attention_test.cu:86-129
    checks every prefill output against the CPU reference the same way)."""
    S, H, Hq, D, bs, T = 8, 8, 32, 128, 16, 4096
    rng = np.random.default_rng(41)
    pool = v2.PhysicalBlockPool(S * T // bs + 64, bs)
    storage = v2.PagedKVStorage(pool, H, D, v2.DType.BFloat16)
    fragment(pool, rng.permutation(pool.capacity()))
    lib = capi.lib()
    kn, vn = device.DeviceBuffer(S * T * H * D * 2), device.DeviceBuffer(S * T * H * D * 2)
    q_all = oracle.random_elements(0, S * T * Hq * D, oracle.F32, 1, 42)
    seqs, tables = [], []
    for i in range(S):
        seq = v2.SequenceState(i, pool)
        seq.append_tokens(T)
        seqs.append(seq)
        kp, vp = kn.ptr + i * T * H * D * 2, vn.ptr + i * T * H * D * 2
        device.fill_random(kp, T * H * D, capi.DTYPE_BF16, 1, 43 + 2 * i)
        device.fill_random(vp, T * H * D, capi.DTYPE_BF16, 1, 44 + 2 * i)
        v2.write_paged_kv(storage, kp, vp, v2.build_slot_mapping([(seq, t) for t in range(T)]))
        tables.append(np.array(v2.build_read_block_table(seq), np.uint64))
    npages = T // bs
    kb, vb = storage.key_base(), storage.value_base()
    qd = buffer_like(q_all)
    td = buffer_like(np.concatenate(tables))
    lens = buffer_like(np.full(S, T, np.uint64))
    offs = buffer_like((np.arange(S) * T).astype(np.uint64))
    out = buffer_like(np.full(S * T * Hq * D + 8, 777.0, np.float32))
    assert lib.kvflux_paged_prefill_batch(kb, vb, pool.capacity(), H, bs, D, capi.DTYPE_BF16, td.ptr, npages,
                                          lens.ptr, lens.ptr, offs.ptr, S, T, T, Hq, qd.ptr, out.ptr, None) == 0, \
        capi.last_error()
    device.synchronize()
    got = out.download(np.float32)
    assert np.all(got[S * T * Hq * D:] == 777.0)
    got = got[:S * T * Hq * D].reshape(S, T, Hq * D)
    assert np.all(np.isfinite(got))
    single = device.DeviceBuffer(T * Hq * D * 4)
    k_all = kn.download(np.uint16).reshape(S, T, H, D)
    v_all = vn.download(np.uint16).reshape(S, T, H, D)
    qr = q_all.reshape(S, T, Hq * D)
    for i in range(S):
        ti = buffer_like(tables[i])
        assert lib.kvflux_paged_prefill(kb, vb, pool.capacity(), H, bs, D, capi.DTYPE_BF16, ti.ptr, npages, T, T,
                                        Hq, qd.ptr + i * T * Hq * D * 4, single.ptr, None) == 0, capi.last_error()
        device.synchronize()
        one = single.download(np.float32).reshape(T, Hq * D)
        assert np.array_equal(got[i].view(np.uint32), one.view(np.uint32)), i
        rows = {0, 1, 15, 16, 63, 64, 127, 128, 1000, 2047, 2048, 3071, 4094, 4095} | \
            set(rng.integers(0, T, 6).tolist())
        assert len(rows) >= 16
        for t in sorted(rows):
            exp = oracle.reference_attention(qr[i, t], oracle.decode(k_all[i, :t + 1].reshape(-1), oracle.BF16),
                                             oracle.decode(v_all[i, :t + 1].reshape(-1), oracle.BF16), 1, t + 1,
                                             Hq, H, D)
            assert np.abs(got[i, t] - exp).max() < 2e-2, (i, t)
