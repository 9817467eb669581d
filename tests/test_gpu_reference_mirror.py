"""GPU tests that restate the reference's own GPU tests through the
kvflux::v2 binding (the C++ layer, which reaches the GPU through the C ABI):

  write    reference tests/paged_kv_write_test.cpp:33-113
  read     reference tests/paged_kv_read_test.cpp:35-108
  gather   reference tests/paged_kv_gather_test.cpp:26-98
  storage  reference tests/paged_kv_storage_test.cpp:20-83
  attention        reference tests/paged_attention_test.cu:50-167
  attention batch  reference tests/paged_attention_batch_test.cu:44-146

Raw bit patterns, 0xA5 sentinels, NaN-filled caches and the 1e-5 bound for
all three dtypes are the reference's.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import DTYPES, buffer_like, decode, encode, fill_cache, raw
from kvflux_amd import device
from oracle import oracle

pytestmark = pytest.mark.gpu
ALL = ["Float16", "BFloat16", "Float32"]


def sentinel(name):
    return 0xA5A5A5A5 if name == "Float32" else 0xA5A5


def bits(a: np.ndarray) -> np.ndarray:
    return a.view(np.uint32) if a.dtype == np.float32 else a


@pytest.mark.parametrize("name", ALL)
def test_write_three_slots_and_untouched_neighbours(gpu, v2, name):
    heads, dims, bs = 2, 4, 16
    pool = v2.PhysicalBlockPool(64, bs)
    storage = v2.PagedKVStorage(pool, heads, dims, getattr(v2.DType, name))
    occupied = []

    def until(n):
        while pool.capacity() - pool.available() < n:
            occupied.append(pool.allocate())

    until(10); a = v2.SequenceState(1001, pool); a.append_tokens(14)
    until(32); b = v2.SequenceState(1002, pool); b.append_tokens(11)
    until(59); c = v2.SequenceState(1003, pool); c.append_tokens(1)
    slots = v2.build_slot_mapping([(a, 13), (b, 10), (c, 0)])
    assert slots == [173, 522, 944]
    fill_cache(storage, 0xA5)
    n = len(slots) * heads * dims
    keys = raw(0x1200 + np.arange(n), name)
    values = raw(0x3400 + np.arange(n), name)
    kd, vd = buffer_like(keys), buffer_like(values)
    v2.write_paged_kv(storage, kd.ptr, vd.ptr, slots)
    dt = DTYPES[name][1]
    for i, slot in enumerate(slots):
        for h in range(heads):
            for d in range(dims):
                idx = (i * heads + h) * dims + d
                kb = device.memcpy_d2h(storage.slot_address(v2.KVKind.Key, slot, h, d), keys.itemsize, dt)
                vb = device.memcpy_d2h(storage.slot_address(v2.KVKind.Value, slot, h, d), keys.itemsize, dt)
                assert bits(kb)[0] == bits(keys)[idx] and bits(vb)[0] == bits(values)[idx]
        kn = device.memcpy_d2h(storage.slot_address(v2.KVKind.Key, slot + 1, 1, 3), keys.itemsize, dt)
        vn = device.memcpy_d2h(storage.slot_address(v2.KVKind.Value, slot + 1, 1, 3), keys.itemsize, dt)
        assert bits(kn)[0] == sentinel(name) and bits(vn)[0] == sentinel(name)
    v2.write_paged_kv(storage, 0, 0, [])
    with pytest.raises(ValueError):
        v2.write_paged_kv(storage, 0, vd.ptr, slots)
    with pytest.raises(IndexError):
        v2.write_paged_kv(storage, kd.ptr, vd.ptr, [storage.layout().slot_count()])
    with pytest.raises(ValueError):
        v2.write_paged_kv(storage, kd.ptr, vd.ptr, [173, 173])
    with pytest.raises(ValueError):
        v2.write_paged_kv(storage, keys.ctypes.data, vd.ptr, slots)  # host pointer
    del a, b, c
    for h in occupied:
        pool.free(h)
    assert pool.available() == pool.capacity()


@pytest.mark.parametrize("name", ALL)
def test_read_forty_tokens_across_27_3_91(gpu, v2, name):
    heads, dims, tokens = 2, 3, 40
    elements = tokens * heads * dims
    pool = v2.PhysicalBlockPool(96, 16)
    storage = v2.PagedKVStorage(pool, heads, dims, getattr(v2.DType, name))
    occupied = [pool.allocate() for _ in range(27)]
    request = v2.SequenceState(1001, pool)
    request.append_tokens(16)
    occupied += [pool.allocate() for _ in range(28, 91)]
    pool.free(occupied[3])
    request.append_tokens(16)
    request.append_tokens(8)
    assert v2.build_read_block_table(request) == [27, 3, 91]
    slots = v2.build_slot_mapping([(request, i) for i in range(tokens)])
    keys = raw(0x1000 + np.arange(elements), name)
    values = raw(0x3000 + np.arange(elements), name)
    kin, vin = buffer_like(keys), buffer_like(values)
    v2.write_paged_kv(storage, kin.ptr, vin.ptr, slots)
    kout = device.DeviceBuffer((elements + 1) * keys.itemsize)
    vout = device.DeviceBuffer((elements + 1) * keys.itemsize)
    kout.fill(0xA5)
    vout.fill(0xA5)
    v2.read_paged_kv(storage, request, kout.ptr, vout.ptr)
    dt = DTYPES[name][1]
    ak, av = kout.download(dt), vout.download(dt)
    assert np.array_equal(bits(ak[:elements]), bits(keys)) and np.array_equal(bits(av[:elements]), bits(values))
    assert bits(ak)[elements] == sentinel(name) and bits(av)[elements] == sentinel(name)

    # prefix-shared read without a second write (reference :92-108)
    cache = v2.PrefixCache(pool)
    prompt = list(range(tokens))
    cache.publish_computed_block(request, 0, prompt[:16])
    cache.publish_computed_block(request, 1, prompt[:32])
    shared = v2.SequenceState(1004, pool)
    prompt[32] = 999
    assert cache.attach_cached_prefix(shared, prompt) == 32
    v2.read_paged_kv(storage, shared, kout.ptr, vout.ptr)
    n32 = 32 * heads * dims
    assert np.array_equal(bits(kout.download(dt, n32)), bits(keys[:n32]))
    assert np.array_equal(bits(vout.download(dt, n32)), bits(values[:n32]))

    with pytest.raises(ValueError):
        v2.read_paged_kv(storage, request, 0, vout.ptr)
    with pytest.raises(ValueError):
        v2.read_paged_kv(storage, request, kout.ptr, kout.ptr)
    with pytest.raises(ValueError):
        v2.read_paged_kv(storage, request, keys.ctypes.data, vout.ptr)
    with pytest.raises(ValueError):
        v2.read_paged_kv(storage, request, storage.key_base(), vout.ptr)
    other = v2.SequenceState(1002, v2.PhysicalBlockPool(96, 16))
    other.append_tokens(1)
    with pytest.raises(ValueError):
        v2.read_paged_kv(storage, other, kout.ptr, vout.ptr)
    v2.read_paged_kv(storage, v2.SequenceState(1003, pool), 0, 0)


@pytest.mark.parametrize("name", ALL)
def test_gather_interleaved_requests(gpu, v2, name):
    heads, dims, ept = 2, 3, 6
    pool = v2.PhysicalBlockPool(5, 2)
    storage = v2.PagedKVStorage(pool, heads, dims, getattr(v2.DType, name))
    a, b = v2.SequenceState(101, pool), v2.SequenceState(202, pool)
    a.append_tokens(2); b.append_tokens(2); a.append_tokens(2); b.append_tokens(2); a.append_token()
    assert v2.build_read_block_table(a) == [0, 2, 4] and v2.build_read_block_table(b) == [1, 3]
    writes = [(b, 0), (a, 0), (b, 1), (a, 1), (b, 2), (a, 2), (b, 3), (a, 3), (a, 4)]
    exp = {id(a): (np.zeros(5 * ept, np.int64), np.zeros(5 * ept, np.int64)),
           id(b): (np.zeros(4 * ept, np.int64), np.zeros(4 * ept, np.int64))}
    ik, iv = [], []
    for seq, pos in writes:
        for e in range(ept):
            ident = (100 if seq is a else 200) + pos * ept + e
            ik.append(0x1000 + ident)
            iv.append(0x3000 + ident)
            exp[id(seq)][0][pos * ept + e] = 0x1000 + ident
            exp[id(seq)][1][pos * ept + e] = 0x3000 + ident
    fill_cache(storage, 0xA5)
    kin, vin = buffer_like(raw(ik, name)), buffer_like(raw(iv, name))
    v2.write_paged_kv(storage, kin.ptr, vin.ptr, v2.build_slot_mapping(writes))
    dt = DTYPES[name][1]
    for seq in (a, b):
        ek, ev = exp[id(seq)]
        n = ek.size
        kout = device.DeviceBuffer((n + 1) * np.dtype(dt).itemsize)
        vout = device.DeviceBuffer((n + 1) * np.dtype(dt).itemsize)
        kout.fill(0xA5); vout.fill(0xA5)
        v2.read_paged_kv(storage, seq, kout.ptr, vout.ptr)
        gk, gv = bits(kout.download(dt)), bits(vout.download(dt))
        assert np.array_equal(gk[:n], bits(raw(ek, name))) and np.array_equal(gv[:n], bits(raw(ev, name)))
        assert gk[n] == sentinel(name) and gv[n] == sentinel(name)
    assert pool.available() == 0


def test_storage_roundtrip_and_addresses(gpu, v2):
    pool = v2.PhysicalBlockPool(4, 2)
    storage = v2.PagedKVStorage(pool, 2, 3, v2.DType.Float32)
    layout = storage.layout()
    assert layout.page_bytes() == 48 and layout.cache_bytes() == 192
    assert layout.total_bytes() == 384 and layout.slot_count() == 8
    kb, vb = storage.key_base(), storage.value_base()
    assert vb == kb + layout.cache_bytes()
    request = v2.SequenceState(1001, pool)
    request.append_tokens(5)
    holder = pool.allocate()
    assert pool.id(holder) == 3
    assert storage.page_address(v2.KVKind.Key, holder) == kb + 3 * 48
    assert storage.element_address(v2.KVKind.Value, holder, 1, 1, 2) == vb + 3 * 48 + (6 + 3 + 2) * 4
    assert storage.slot_address(v2.KVKind.Key, 6, 1, 1) == storage.element_address(v2.KVKind.Key, holder, 1, 0, 1)
    keys = (1000 + np.arange(48)).astype(np.uint32)
    values = (10000 + np.arange(48)).astype(np.uint32)
    device.memcpy_h2d(kb, keys)
    device.memcpy_h2d(vb, values)
    slots = v2.build_slot_mapping([(request, 0), (request, 2), (request, 4)])
    assert slots == [0, 2, 4]
    for slot in slots:
        for h in range(2):
            for d in range(3):
                k = device.memcpy_d2h(storage.slot_address(v2.KVKind.Key, slot, h, d), 4, np.uint32)[0]
                assert k == keys[layout.slot_byte_offset(v2.KVKind.Key, slot, h, d) // 4]
    with pytest.raises(IndexError):
        storage.slot_address(v2.KVKind.Key, 8, 0, 0)
    with pytest.raises(IndexError):
        storage.slot_address(v2.KVKind.Key, 0, 2, 0)
    pool.free(holder)
    with pytest.raises(ValueError):
        storage.page_address(v2.KVKind.Key, holder)
    reused = pool.allocate()
    assert reused.id == holder.id and reused.generation != holder.generation
    pool.free(reused)


def _attention_case(v2, name):
    tokens, kv_heads, q_heads, head_size = 10, 2, 4, 4
    kv_elements = tokens * kv_heads * head_size
    pool = v2.PhysicalBlockPool(8, 4)
    storage = v2.PagedKVStorage(pool, kv_heads, head_size, getattr(v2.DType, name))
    occupied = [pool.allocate() for _ in range(5)]
    seq = v2.SequenceState(1001, pool)
    seq.append_tokens(4)
    occupied.append(pool.allocate())
    pool.free(occupied[1])
    seq.append_tokens(4)
    seq.append_tokens(2)
    assert v2.build_read_block_table(seq) == [5, 1, 7]
    i = np.arange(kv_elements)
    key_in = encode(0.125 * ((i * 7 % 17) - 8), name)
    val_in = encode(0.125 * ((i * 11 % 23) - 11), name)
    fill_cache(storage, 0xFF)  # NaN everywhere not written
    kd, vd = buffer_like(key_in), buffer_like(val_in)
    v2.write_paged_kv(storage, kd.ptr, vd.ptr, v2.build_slot_mapping([(seq, t) for t in range(tokens)]))
    return pool, storage, seq, occupied, key_in, val_in, (tokens, kv_heads, q_heads, head_size)


@pytest.mark.parametrize("name", ALL)
def test_paged_attention_matches_gather_plus_reference(gpu, v2, name):
    pool, storage, seq, occupied, key_in, val_in, shape = _attention_case(v2, name)
    tokens, kv_heads, q_heads, head_size = shape
    dt = DTYPES[name][1]
    gk, gv = device.DeviceBuffer(key_in.nbytes), device.DeviceBuffer(val_in.nbytes)
    v2.read_paged_kv(storage, seq, gk.ptr, gv.ptr)
    ck, cv = decode(gk.download(dt), name), decode(gv.download(dt), name)
    assert np.array_equal(ck, decode(key_in, name)) and np.array_equal(cv, decode(val_in, name))
    for q_tokens in (tokens, 3, 1):
        n = q_tokens * q_heads * head_size
        q = (0.125 * ((np.arange(n) * 5 % 19) - 9)).astype(np.float32)
        expected = oracle.reference_attention(q, ck, cv, q_tokens, tokens, q_heads, kv_heads, head_size)
        qd = buffer_like(q)
        od = buffer_like(np.full(n + 1, 12345.0, np.float32))
        v2.paged_attention(storage, seq, qd.ptr, od.ptr, q_tokens, q_heads)
        actual = od.download(np.float32)
        assert np.all(np.isfinite(actual[:n]))
        assert np.abs(actual[:n] - expected).max() < 1e-5
        assert actual[n] == 12345.0
        if q_tokens == 1:
            with pytest.raises(ValueError):
                v2.paged_attention(storage, seq, 0, od.ptr, 1, q_heads)
            with pytest.raises(ValueError):
                v2.paged_attention(storage, seq, qd.ptr, qd.ptr, 1, q_heads)
            with pytest.raises(ValueError):
                v2.paged_attention(storage, seq, q.ctypes.data, od.ptr, 1, q_heads)
            with pytest.raises(ValueError):
                v2.paged_attention(storage, seq, qd.ptr, od.ptr, 1, 3)
            with pytest.raises(ValueError):
                v2.paged_attention(storage, seq, qd.ptr, od.ptr, tokens + 1, q_heads)
    v2.paged_attention(storage, seq, 0, 0, 0, q_heads)
    other = v2.SequenceState(1002, v2.PhysicalBlockPool(8, 4))
    other.append_tokens(1)
    with pytest.raises(ValueError):
        v2.paged_attention(storage, other, 0, 0, 0, q_heads)
    del seq
    for i, h in enumerate(occupied):
        if i != 1:
            pool.free(h)
    assert pool.available() == pool.capacity()


@pytest.mark.parametrize("name", ALL)
def test_paged_attention_batch_variable_lengths(gpu, v2, name):
    kv_heads, q_heads, head_size = 2, 4, 3
    pool = v2.PhysicalBlockPool(16, 4)
    storage = v2.PagedKVStorage(pool, kv_heads, head_size, getattr(v2.DType, name))
    a, b, c = (v2.SequenceState(i, pool) for i in (1, 2, 3))
    a.append_tokens(4); b.append_tokens(4); c.append_tokens(2); a.append_token(); b.append_tokens(5)
    seqs = [a, b, c]
    table = v2.build_batch_block_table(seqs)
    pad = table.invalid_block()
    assert table.sequence_lengths() == [5, 9, 2]
    assert table.block_table() == [0, 3, pad, 1, 4, 5, 2, pad, pad]
    writes = [(s, t) for s in seqs for t in range(s.num_tokens())]
    n_kv = 16 * kv_heads * head_size
    i = np.arange(n_kv)
    keys = encode(0.125 * ((i * 7 % 19) - 9), name)
    values = encode(0.125 * ((i * 11 % 23) - 11), name)
    fill_cache(storage, 0xFF)
    kd, vd = buffer_like(keys), buffer_like(values)
    v2.write_paged_kv(storage, kd.ptr, vd.ptr, v2.build_slot_mapping(writes))
    nq = 3 * q_heads * head_size
    q = (0.125 * ((np.arange(nq) * 5 % 17) - 8)).astype(np.float32)
    qd = buffer_like(q)
    od = buffer_like(np.full(nq + 1, 12345.0, np.float32))
    v2.paged_attention_batch(storage, seqs, qd.ptr, od.ptr, q_heads)
    actual = od.download(np.float32)
    offset = 0
    per = q_heads * head_size
    for r, s in enumerate(seqs):
        L = s.num_tokens()
        k = decode(keys, name)[offset * kv_heads * head_size:(offset + L) * kv_heads * head_size]
        v = decode(values, name)[offset * kv_heads * head_size:(offset + L) * kv_heads * head_size]
        exp = oracle.reference_attention(q[r * per:(r + 1) * per], k, v, 1, L, q_heads, kv_heads, head_size)
        got = actual[r * per:(r + 1) * per]
        assert np.all(np.isfinite(got)) and np.abs(got - exp).max() < 1e-5
        offset += L
    assert actual[nq] == 12345.0
    with pytest.raises(ValueError):
        v2.paged_attention_batch(storage, seqs, 0, od.ptr, q_heads)
    with pytest.raises(ValueError):
        v2.paged_attention_batch(storage, seqs, qd.ptr, qd.ptr, q_heads)
    with pytest.raises(ValueError):
        v2.paged_attention_batch(storage, seqs, q.ctypes.data, od.ptr, q_heads)
    with pytest.raises(ValueError):
        v2.paged_attention_batch(storage, seqs, qd.ptr, od.ptr, 3)
    with pytest.raises(ValueError):
        v2.paged_attention_batch(storage, [a, v2.SequenceState(4, pool)], qd.ptr, od.ptr, q_heads)
    other = v2.SequenceState(5, v2.PhysicalBlockPool(2, 4))
    other.append_token()
    with pytest.raises(ValueError):
        v2.paged_attention_batch(storage, [a, other], qd.ptr, od.ptr, q_heads)
    v2.paged_attention_batch(storage, [], 0, 0, q_heads)
