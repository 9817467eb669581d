"""Callers of the hot path on the GPU: copy-on-write (single and batched),
the single-request lifecycle, the device-resident batch table and the
batched decode step.

* The first two tests restate the reference's own GPU tests
  (tests/copy_on_write_gpu_test.cpp:25-130 with its raw patterns
  0x1100+i / 0x2200+i / 0x3300+i ..., and tests/sequence_lifecycle_test.cpp:
  56-167 with its literal inputs, checked at 1e-5 against reference
  attention plus the 12345.0 sentinel).
* Batched copy-on-write is checked against the sequential reference
  semantics (append_token_cow one request at a time) on twin pools:
  identical locations, tables, reference counts and page bytes.
* The device batch table is checked against build_batch_block_table (the
  reference's host algorithm, pinned by its KATs in the CPU suite).
* The decode step is checked against the step the reference API composes
  (append_token_cow + write_paged_kv + paged_attention_batch): bit-identical
  cache bytes and outputs, and outputs within 1e-5 of the oracle.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from gpu_util import DTYPES, buffer_like, read_cache
from kvflux_amd import capi, device
from oracle import oracle

pytestmark = pytest.mark.gpu


def upload(values, dtype):
    return buffer_like(np.asarray(values, dtype))


def read_tokens(v2, storage, seq, name, tokens):
    """Gathered K/V of `seq` ([tokens][H][D] as storage integers)."""
    layout = storage.layout()
    per = layout.num_kv_heads() * layout.head_size()
    dt = DTYPES[name][1]
    k = device.DeviceBuffer(max(tokens * per, 1) * np.dtype(dt).itemsize)
    v = device.DeviceBuffer(max(tokens * per, 1) * np.dtype(dt).itemsize)
    v2.read_paged_kv(storage, seq, k.ptr, v.ptr)
    return k.download(dt, tokens * per), v.download(dt, tokens * per)


@pytest.mark.parametrize("name", ["Float16", "BFloat16", "Float32"])
def test_reference_copy_on_write_gpu(gpu, v2, name):
    """tests/copy_on_write_gpu_test.cpp:25-130, same pool, shapes and patterns."""
    bits = np.uint32 if name == "Float32" else np.uint16
    heads, dims, per = 2, 3, 6
    pool = v2.PhysicalBlockPool(3, 4)
    storage = v2.PagedKVStorage(pool, heads, dims, getattr(v2.DType, name))
    a = v2.SequenceState(1, pool)
    a.append_tokens(3)
    old_page = a.physical_block_id(0)
    init_k = (0x1100 + np.arange(3 * per)).astype(bits)
    init_v = (0x2200 + np.arange(3 * per)).astype(bits)
    kd, vd = upload(init_k, bits), upload(init_v, bits)
    v2.write_paged_kv(storage, kd.ptr, vd.ptr, v2.build_slot_mapping([(a, 0), (a, 1), (a, 2)]))
    b = a.fork_shared(2)
    assert pool.ref_count(a.block_table().handle(0)) == 2
    a_new = v2.append_token_cow(storage, a)
    assert a_new.physical_block != old_page and a_new.offset_in_block == 3
    assert a.num_tokens() == 4 and b.num_tokens() == 3 and b.physical_block_id(0) == old_page
    a_k, a_v = (0x3300 + np.arange(per)).astype(bits), (0x4400 + np.arange(per)).astype(bits)
    b_k, b_v = (0x5500 + np.arange(per)).astype(bits), (0x6600 + np.arange(per)).astype(bits)
    akd, avd, bkd, bvd = (upload(x, bits) for x in (a_k, a_v, b_k, b_v))
    v2.write_paged_kv(storage, akd.ptr, avd.ptr, v2.build_slot_mapping([(a, 3)]))
    got_ak, got_av = read_tokens(v2, storage, a, name, 4)
    got_bk, got_bv = read_tokens(v2, storage, b, name, 3)
    assert np.array_equal(got_ak.view(bits), np.concatenate([init_k, a_k]))
    assert np.array_equal(got_av.view(bits), np.concatenate([init_v, a_v]))
    assert np.array_equal(got_bk.view(bits), init_k) and np.array_equal(got_bv.view(bits), init_v)
    b_new = b.append_token()  # the old page is now B's alone: no copy
    assert b_new.physical_block == old_page and b_new.offset_in_block == 3
    v2.write_paged_kv(storage, bkd.ptr, bvd.ptr, v2.build_slot_mapping([(b, 3)]))
    got_bk, got_bv = read_tokens(v2, storage, b, name, 4)
    assert np.array_equal(got_bk.view(bits), np.concatenate([init_k, b_k]))
    assert np.array_equal(got_bv.view(bits), np.concatenate([init_v, b_v]))
    got_ak, got_av = read_tokens(v2, storage, a, name, 4)
    assert np.array_equal(got_ak.view(bits), np.concatenate([init_k, a_k]))
    assert np.array_equal(got_av.view(bits), np.concatenate([init_v, a_v]))
    assert a.physical_block_id(0) != b.physical_block_id(0)


def _expect_attention(out, query, keys, values, q_tokens):
    exp = oracle.reference_attention(np.asarray(query, np.float32), np.asarray(keys, np.float32),
                                      np.asarray(values, np.float32), q_tokens, len(keys) // 2, 2, 1, 2)
    got = out.download(np.float32)
    assert np.all(np.isfinite(got[:exp.size]))
    assert np.abs(got[:exp.size] - exp).max() < 1e-5
    assert got[exp.size] == np.float32(12345.0)  # nothing written past the output


def test_reference_sequence_lifecycle(gpu, v2):
    """tests/sequence_lifecycle_test.cpp:56-167 (full request, then the
    failure and capacity cases), same literal inputs."""
    pool = v2.PhysicalBlockPool(4, 2)
    storage = v2.PagedKVStorage(pool, 1, 2, v2.DType.Float32)
    capi.call("kvflux_fill_bytes", C.c_void_p(storage.key_base()), 0xFF, storage.layout().total_bytes(), None)
    keys = [0.2, -0.1, 0.3, 0.4, -0.2, 0.5]
    values = [1.0, 2.0, 3.0, -1.0, 0.5, 4.0]
    prompt_q = [0.1, 0.2, -0.3, 0.4, 0.5, -0.2, 0.1, 0.3, -0.4, 0.6, 0.2, -0.1]
    steps = [([0.6, -0.3], [2.0, 1.5], [0.2, 0.7, -0.1, 0.4]),
             ([-0.5, 0.2], [-2.0, 3.0], [0.8, -0.2, 0.3, 0.1])]
    pk, pv, pq = (upload(x, np.float32) for x in (keys, values, prompt_q))
    pout = upload([12345.0] * (len(prompt_q) + 1), np.float32)
    req = v2.SequenceLifecycle(1001, pool, storage, 2)
    assert req.sequence().num_tokens() == 0 and pool.available() == 4
    with pytest.raises(ValueError):
        req.prefill(0, pk.ptr, pv.ptr, pq.ptr, pout.ptr)
    assert not req.finished()
    req.prefill(3, pk.ptr, pv.ptr, pq.ptr, pout.ptr)
    assert req.sequence().num_tokens() == 3
    assert req.sequence().num_allocated_blocks() == 2 and pool.available() == 2
    _expect_attention(pout, prompt_q, keys, values, 3)
    with pytest.raises(v2.LogicError):
        req.prefill(3, pk.ptr, pv.ptr, pq.ptr, pout.ptr)
    one_out = upload([12345.0] * 5, np.float32)
    with pytest.raises(ValueError):
        req.decode(0, pv.ptr, pq.ptr, one_out.ptr)
    assert not req.finished() and req.sequence().num_tokens() == 3
    locations = []
    for k_new, v_new, q_new in steps:
        kd, vd, qd = upload(k_new, np.float32), upload(v_new, np.float32), upload(q_new, np.float32)
        one_out.upload(np.full(5, 12345.0, np.float32))
        loc = req.decode(kd.ptr, vd.ptr, qd.ptr, one_out.ptr)
        locations.append(loc)
        keys += k_new
        values += v_new
        _expect_attention(one_out, q_new, keys, values, 1)
    assert locations[0].offset_in_block == 1
    assert locations[0].physical_block == req.sequence().physical_block_id(1)
    assert locations[1].offset_in_block == 0
    assert locations[1].physical_block == req.sequence().physical_block_id(2)
    assert req.sequence().num_tokens() == 5 and pool.available() == 1
    req.finish()
    assert req.finished() and pool.available() == pool.capacity()
    req.finish()
    with pytest.raises(v2.LogicError):
        req.sequence()
    # Q on the host: attention validation fails after the pages and the KV write
    failed = v2.SequenceLifecycle(1002, pool, storage, 2)
    host_q = np.asarray(prompt_q, np.float32)
    with pytest.raises(ValueError):
        failed.prefill(1, pk.ptr, pv.ptr, host_q.ctypes.data, one_out.ptr)
    assert failed.finished() and pool.available() == pool.capacity()
    # capacity failure releases the request
    pool1 = v2.PhysicalBlockPool(1, 2)
    storage1 = v2.PagedKVStorage(pool1, 1, 2, v2.DType.Float32)
    kv = upload([0.1, 0.2, 0.3, 0.4], np.float32)
    q = upload([0.2, 0.1, 0.4, 0.3, 0.6, 0.5, 0.8, 0.7], np.float32)
    out = upload(np.zeros(9), np.float32)
    r = v2.SequenceLifecycle(2001, pool1, storage1, 2)
    r.prefill(2, kv.ptr, kv.ptr, q.ptr, out.ptr)
    assert pool1.available() == 0
    with pytest.raises(v2.CapacityError):
        r.decode(kv.ptr, kv.ptr, q.ptr, out.ptr)
    assert r.finished() and pool1.available() == 1


@pytest.mark.parametrize("name,H,D,bs", [("BFloat16", 8, 128, 16), ("Float32", 2, 5, 3), ("Float16", 1, 1, 48)])
def test_copy_blocks_batch(gpu, v2, name, H, D, bs):
    """Every destination page equals its source page (K and V), every other
    page is untouched; invalid batches are rejected before any copy."""
    pool = v2.PhysicalBlockPool(96, bs)
    storage = v2.PagedKVStorage(pool, H, D, getattr(v2.DType, name))
    layout = storage.layout()
    n = layout.cache_bytes() * 2 // np.dtype(DTYPES[name][1]).itemsize
    device.fill_random(storage.key_base(), n, {"Float32": 2, "Float16": 0, "BFloat16": 1}[name], 0, 7)
    held = [pool.allocate() for _ in range(96)]
    rng = np.random.default_rng(3)
    order = rng.permutation(96)
    srcs, dsts = order[:40], order[40:80]
    pairs = [(held[int(s)], held[int(d)]) for s, d in zip(srcs, dsts)]
    before_k, before_v = read_cache(storage, name)
    storage.copy_blocks(pairs)
    after_k, after_v = read_cache(storage, name)
    page = layout.page_bytes() // np.dtype(DTYPES[name][1]).itemsize
    expect_k, expect_v = before_k.copy(), before_v.copy()
    for s, d in zip(srcs, dsts):
        expect_k[d * page:(d + 1) * page] = before_k[s * page:(s + 1) * page]
        expect_v[d * page:(d + 1) * page] = before_v[s * page:(s + 1) * page]
    assert np.array_equal(after_k.view(np.uint8), expect_k.view(np.uint8))
    assert np.array_equal(after_v.view(np.uint8), expect_v.view(np.uint8))
    # rejected batches: duplicate destination, destination also a source,
    # shared destination, source == destination
    bad = [[(held[0], held[1]), (held[2], held[1])],
           [(held[0], held[1]), (held[1], held[2])],
           [(held[3], held[3])]]
    pool.retain(held[5])
    bad.append([(held[4], held[5])])
    for batch in bad:
        with pytest.raises(ValueError):
            storage.copy_blocks(batch)
    pool.free(held[5])
    assert np.array_equal(read_cache(storage, name)[0].view(np.uint8), after_k.view(np.uint8))
    storage.copy_blocks([])


def _twin(v2, name, H, D, bs, capacity, seed):
    """A pool/storage with requests in every append state: private tails,
    shared partial tails (forked mid-page), block boundaries, empty."""
    pool = v2.PhysicalBlockPool(capacity, bs)
    storage = v2.PagedKVStorage(pool, H, D, getattr(v2.DType, name))
    n = storage.layout().cache_bytes() * 2 // np.dtype(DTYPES[name][1]).itemsize
    device.fill_random(storage.key_base(), n, {"Float32": 2, "Float16": 0, "BFloat16": 1}[name], 0, seed)
    rng = np.random.default_rng(seed)
    seqs = []
    for i in range(6):
        s = v2.SequenceState(100 + i, pool)
        s.append_tokens(int(rng.integers(1, 4 * bs)))
        seqs.append(s)
    base = v2.SequenceState(200, pool)
    base.append_tokens(2 * bs + bs // 2 + 1 if bs > 2 else 5)  # partial tail
    forks = [base.fork_shared(300 + i) for i in range(3)]
    edge = v2.SequenceState(400, pool)
    edge.append_tokens(2 * bs)  # at a block boundary
    empty = v2.SequenceState(500, pool)
    return pool, storage, seqs + forks + [base, edge, empty], (base, forks)


@pytest.mark.parametrize("name,H,D,bs", [("BFloat16", 2, 64, 16), ("Float32", 1, 3, 4)])
def test_append_tokens_cow_matches_sequential(gpu, v2, name, H, D, bs):
    pa, sa, seq_a, keep_a = _twin(v2, name, H, D, bs, 128, 5)
    pb, sb, seq_b, keep_b = _twin(v2, name, H, D, bs, 128, 5)
    for step in range(3):
        got = v2.append_tokens_cow(sa, seq_a)
        exp = [v2.append_token_cow(sb, s) for s in seq_b]
        assert [(g.physical_block, g.offset_in_block) for g in got] == \
               [(e.physical_block, e.offset_in_block) for e in exp]
        for x, y in zip(seq_a, seq_b):
            assert x.num_tokens() == y.num_tokens()
            assert [x.physical_block_id(i) for i in range(x.num_allocated_blocks())] == \
                   [y.physical_block_id(i) for i in range(y.num_allocated_blocks())]
            assert [x.block_table().ref_count(i) for i in range(x.num_allocated_blocks())] == \
                   [y.block_table().ref_count(i) for i in range(y.num_allocated_blocks())]
        assert pa.available() == pb.available()
        ka, va = read_cache(sa, name)
        kb, vb = read_cache(sb, name)
        assert np.array_equal(ka.view(np.uint8), kb.view(np.uint8))
        assert np.array_equal(va.view(np.uint8), vb.view(np.uint8))
    assert v2.append_tokens_cow(sa, []) == []
    with pytest.raises(ValueError):
        v2.append_tokens_cow(sa, [seq_a[0], seq_a[0]])


def test_append_tokens_cow_all_or_nothing(gpu, v2):
    """Pool too small for the batch: CapacityError, no request changes."""
    pool = v2.PhysicalBlockPool(8, 4)
    storage = v2.PagedKVStorage(pool, 1, 2, v2.DType.Float32)
    base = v2.SequenceState(1, pool)
    base.append_tokens(6)  # 2 pages, partial tail
    forks = [base.fork_shared(10 + i) for i in range(7)]  # 7 copies needed, 6 pages free
    state = [(s.num_tokens(), [s.physical_block_id(i) for i in range(s.num_allocated_blocks())])
             for s in [base] + forks]
    avail = pool.available()
    with pytest.raises(v2.CapacityError):
        v2.append_tokens_cow(storage, [base] + forks)
    assert pool.available() == avail
    assert state == [(s.num_tokens(), [s.physical_block_id(i) for i in range(s.num_allocated_blocks())])
                     for s in [base] + forks]


def _check_table(v2, table, seqs):
    host = v2.build_batch_block_table(seqs)
    width = table.capacity_blocks()
    got = device.memcpy_d2h(table.device_table(), len(seqs) * width * 8, np.uint64).reshape(len(seqs), width)
    lens = device.memcpy_d2h(table.device_lengths(), len(seqs) * 8, np.uint64)
    exp = np.array(host.block_table(), np.uint64).reshape(len(seqs), host.max_blocks_per_sequence())
    mb = host.max_blocks_per_sequence()
    assert np.array_equal(got[:, :mb], exp)
    assert np.all(got[:, mb:] == np.uint64(2**64 - 1))
    assert np.array_equal(lens, np.array(host.sequence_lengths(), np.uint64))
    assert list(table.lengths()) == list(host.sequence_lengths())


def test_device_batch_table_tracks_host_table(gpu, v2):
    pool, storage, seqs, _keep = _twin(v2, "Float32", 1, 2, 4, 256, 9)
    seqs = [s for s in seqs if s.num_tokens() > 0]
    table = v2.DeviceBatchTable(storage, seqs, 16)
    _check_table(v2, table, seqs)
    for step in range(9):  # appends across page boundaries and copy-on-write
        if step % 3 == 2:
            for s in seqs[::2]:
                s.append_token()
        else:
            v2.append_tokens_cow(storage, seqs)
        table.refresh()
        _check_table(v2, table, seqs)
    table.refresh()  # nothing changed
    _check_table(v2, table, seqs)
    seqs[0].append_tokens(16 * 4)
    with pytest.raises(v2.LogicError):
        table.refresh()
    with pytest.raises(ValueError):
        v2.DeviceBatchTable(storage, [seqs[1], seqs[1]], 16)


@pytest.mark.parametrize("name,H,Hq,D,bs", [("BFloat16", 2, 8, 128, 16), ("Float16", 2, 4, 64, 16),
                                             ("Float32", 1, 2, 4, 4)])
def test_decode_step_matches_composed_reference_step(gpu, v2, name, H, Hq, D, bs):
    code = DTYPES[name][0]
    esize = np.dtype(DTYPES[name][1]).itemsize
    pa, sa, seq_a, keep_a = _twin(v2, name, H, D, bs, 512, 21)
    pb, sb, seq_b, keep_b = _twin(v2, name, H, D, bs, 512, 21)
    seq_a = [s for s in seq_a if s.num_tokens() > 0]
    seq_b = [s for s in seq_b if s.num_tokens() > 0]
    table = v2.DeviceBatchTable(sa, seq_a, 64)
    rows = len(seq_a)
    kv_elems, q_elems = rows * H * D, rows * Hq * D
    for step in range(2 * bs + 2):  # crosses page boundaries, starts with copy-on-write
        kn = device.DeviceBuffer(kv_elems * esize)
        vn = device.DeviceBuffer(kv_elems * esize)
        device.fill_random(kn.ptr, kv_elems, {"Float32": 2, "Float16": 0, "BFloat16": 1}[name], 0, 1000 + step)
        device.fill_random(vn.ptr, kv_elems, {"Float32": 2, "Float16": 0, "BFloat16": 1}[name], 0, 2000 + step)
        q = oracle.random_elements(0, q_elems, oracle.F32, 0, 3000 + step)
        qd = buffer_like(q)
        oa, ob = buffer_like(np.zeros(q_elems, np.float32)), buffer_like(np.zeros(q_elems, np.float32))
        got = v2.decode_step(sa, table, kn.ptr, vn.ptr, qd.ptr, oa.ptr, Hq)
        # the reference API's composition of the same step
        exp = [v2.append_token_cow(sb, s) for s in seq_b]
        v2.write_paged_kv(sb, kn.ptr, vn.ptr, v2.build_slot_mapping([(s, s.num_tokens() - 1) for s in seq_b]))
        v2.paged_attention_batch(sb, seq_b, qd.ptr, ob.ptr, Hq)
        assert [(g.physical_block, g.offset_in_block) for g in got] == \
               [(e.physical_block, e.offset_in_block) for e in exp]
        out_a, out_b = oa.download(np.float32), ob.download(np.float32)
        assert np.array_equal(out_a.view(np.uint32), out_b.view(np.uint32))
        ka, va = read_cache(sa, name)
        kb, vb = read_cache(sb, name)
        assert np.array_equal(ka.view(np.uint8), kb.view(np.uint8))
        assert np.array_equal(va.view(np.uint8), vb.view(np.uint8))
        if step in (0, 2 * bs + 1):  # against the oracle: gather + reference attention
            page = H * bs * D
            for r in (0, rows - 1):
                s = seq_a[r]
                ids = np.array([s.physical_block_id(i) for i in range(s.num_allocated_blocks())], np.uint64)
                kc = np.concatenate([ka[int(p) * page:(int(p) + 1) * page] for p in ids])
                vc = np.concatenate([va[int(p) * page:(int(p) + 1) * page] for p in ids])
                ref = oracle.paged_attention_rows(kc, vc, H, bs, D, code, np.arange(len(ids), dtype=np.uint64),
                                                  len(ids), np.array([s.num_tokens()], np.uint64),
                                                  q[r * Hq * D:(r + 1) * Hq * D], Hq)
                assert np.abs(out_a[r * Hq * D:(r + 1) * Hq * D] - ref).max() < 1e-5
    assert list(table.lengths()) == [s.num_tokens() for s in seq_a]
    _check_table(v2, table, seq_a)


def test_decode_step_capacity_and_validation(gpu, v2):
    pool = v2.PhysicalBlockPool(16, 4)
    storage = v2.PagedKVStorage(pool, 1, 2, v2.DType.Float32)
    s = v2.SequenceState(1, pool)
    s.append_tokens(8)  # two full pages: the next token needs a third
    table = v2.DeviceBatchTable(storage, [s], 2)
    buf = upload(np.zeros(16), np.float32)
    with pytest.raises(v2.LogicError):  # row capacity
        v2.decode_step(storage, table, buf.ptr, buf.ptr, buf.ptr, buf.ptr + 32, 2)
    assert s.num_tokens() == 8 and pool.available() == 14
    table2 = v2.DeviceBatchTable(storage, [s], 4)
    with pytest.raises(ValueError):  # null K_new
        v2.decode_step(storage, table2, 0, buf.ptr, buf.ptr, buf.ptr + 32, 2)
    with pytest.raises(ValueError):  # head count
        v2.decode_step(storage, table2, buf.ptr, buf.ptr, buf.ptr, buf.ptr + 32, 0)
    assert s.num_tokens() == 8 and pool.available() == 14


def test_tail_write_and_table_apply_c_abi(gpu):
    """Rows with no valid tail slot are skipped; out-of-range records are
    ignored; everything else lands where the host formula says."""
    lib = capi.lib()
    nb, H, bs, D = 8, 2, 4, 4
    cache_elems = nb * H * bs * D
    kc = buffer_like(np.full(cache_elems, 0xA5A5, np.uint16))
    vc = buffer_like(np.full(cache_elems, 0xA5A5, np.uint16))
    width = 3
    table = np.array([[5, 2, 7], [1, 2**64 - 1, 2**64 - 1], [9, 0, 0], [3, 4, 6]], np.uint64)
    lens = np.array([10, 5, 2, 0], np.uint64)  # row 1: block 1 missing; row 2: page 9 >= nb; row 3: empty
    td, ld = buffer_like(table), buffer_like(lens)
    upd = np.array([[0, 10, 2, 6], [3, 1, 0, 4], [7, 1, 0, 1], [1, 5, 5, 3]], np.uint64)  # row 7 and block 5 ignored
    ud = buffer_like(upd)
    assert lib.kvflux_table_apply(td.ptr, width, ld.ptr, 4, ud.ptr, 4, None) == 0
    device.synchronize()
    table[0, 2] = 6
    table[3, 0] = 4
    lens[[0, 3, 1]] = [10, 1, 5]
    assert np.array_equal(td.download(np.uint64), table.reshape(-1))
    assert np.array_equal(ld.download(np.uint64), lens)
    kn = (0x1000 + np.arange(4 * H * D)).astype(np.uint16)
    vn = (0x2000 + np.arange(4 * H * D)).astype(np.uint16)
    knd, vnd = buffer_like(kn), buffer_like(vn)
    assert lib.kvflux_write_paged_kv_tail(kc.ptr, vc.ptr, nb, H, bs, D, capi.DTYPE_BF16, knd.ptr, vnd.ptr,
                                          td.ptr, width, ld.ptr, 4, None) == 0
    device.synchronize()
    exp_k = np.full(cache_elems, 0xA5A5, np.uint16)
    exp_v = exp_k.copy()
    # host restatement: row r writes at table[r][(len-1)//bs] * bs + (len-1) % bs when valid
    slots = []
    for r in range(4):
        ln = int(lens[r])
        if ln == 0 or (ln - 1) // bs >= width or int(table[r, (ln - 1) // bs]) >= nb:
            slots.append(2**64 - 1)
        else:
            slots.append(int(table[r, (ln - 1) // bs]) * bs + (ln - 1) % bs)
    assert slots[0] == 6 * bs + 1 and slots[3] == 4 * bs and slots[1] == 2**64 - 1 and slots[2] == 2**64 - 1
    live = [r for r in range(4) if slots[r] != 2**64 - 1]
    rows_k, rows_v = kn.reshape(4, H * D)[live].reshape(-1), vn.reshape(4, H * D)[live].reshape(-1)
    oracle.write_paged_kv(exp_k, exp_v, H, bs, D, oracle.BF16, rows_k, rows_v,
                          np.array([slots[r] for r in live], np.uint64))
    assert np.array_equal(kc.download(np.uint16), exp_k)
    assert np.array_equal(vc.download(np.uint16), exp_v)
