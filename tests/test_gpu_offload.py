"""GPU <-> CPU chunk transfer of the tiered cache (kvflux::v3).

* The first tests restate the reference's tests/v3_gpu_cpu_migration_test.cpp
  (its fixture: 8 slots of 1 MiB, GpuTier over a v2 pool, CpuTier, NvmeTier,
  PinnedChunkPool; its cases: GPU -> CPU, CPU -> GPU, round trip with LIFO
  page reuse and a new generation, remapping, stale-location rejection, the
  in-flight protocol, several transfers in flight, random bytes). The byte
  patterns are seeded random bytes instead of the reference's xorshift
  stream: any pattern serves, the check is byte equality.
* The batch forms (one kernel for a whole batch, reading and writing the
  pinned slots directly) are checked byte for byte against the same
  directory outcome as single-key transfers, with scattered slots, for the
  pinned pool (one launch) and the pageable heap pool (one copy per chunk),
  and a rejected batch must leave the directory unchanged.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from kvflux_amd import device

pytestmark = pytest.mark.gpu

SLOTS, BYTES = 8, 1 << 20


@pytest.fixture
def v3(gpu):
    import kvflux_amd
    return kvflux_amd.v3


class Fixture:
    def __init__(self, v2, v3, slots=SLOTS, nbytes=BYTES, heap=False):
        self.pool = v2.PhysicalBlockPool(slots, 16)
        self.gpu = v3.GpuTier(self.pool, nbytes)
        self.cpu = v3.CpuTier(slots, nbytes)
        self.nvme = v3.NvmeTier(slots, nbytes)
        self.dir = v3.CacheDirectory(self.gpu, self.cpu, self.nvme)
        self.gpu_store = v3.GpuChunkStore(slots, nbytes)
        self.cpu_pool = v3.HeapChunkPool(slots, nbytes) if heap else v3.PinnedChunkPool(slots, nbytes)
        self.xfer = v3.GpuCpuTransfer(self.dir, self.gpu_store, self.cpu_pool)
        self.nbytes = nbytes
        self.v3 = v3

    def host_write(self, slot, data):
        C.memmove(self.cpu_pool.data(slot), data.ctypes.data, self.nbytes)

    def host_read(self, slot):
        return np.frombuffer(C.string_at(self.cpu_pool.data(slot), self.nbytes), np.uint8)

    def gpu_read(self, loc):
        return device.memcpy_d2h(self.gpu_store.device_ptr(loc), self.nbytes, np.uint8)

    def seed_on_gpu(self, key, data):
        """CPU pattern -> onload -> CPU replica released: only a READY GPU replica."""
        v3 = self.v3
        self.dir.create(key)
        loc = self.dir.place(key, v3.StorageTier.CPU)
        self.host_write(loc.slot, data)
        self.xfer.begin_onload(key)
        self.xfer.finish_onload(key, True)
        assert self.dir.at(key).cpu is None
        assert self.dir.at(key).gpu.state == v3.ChunkState.READY


def make_key(v2, v3, tag):
    return v3.make_cache_key("model-x", 1, v2.DType.Float16, 0, 32, [1, 2, 3, int(tag)])


def pattern(seed, n=BYTES):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8)


def test_gpu_to_cpu(v2, v3):
    f = Fixture(v2, v3)
    key, data = make_key(v2, v3, 1), pattern(0xA17)
    f.seed_on_gpu(key, data)
    f.xfer.begin_offload(key)
    f.xfer.finish_offload(key, False)
    rec = f.dir.at(key)
    assert rec.cpu.state == v3.ChunkState.READY and rec.gpu.state == v3.ChunkState.READY
    assert np.array_equal(f.host_read(rec.cpu.location.slot), data)


def test_cpu_to_gpu(v2, v3):
    f = Fixture(v2, v3)
    key, data = make_key(v2, v3, 2), pattern(0xB22)
    f.dir.create(key)
    loc = f.dir.place(key, v3.StorageTier.CPU)
    f.host_write(loc.slot, data)
    f.xfer.begin_onload(key)
    f.xfer.finish_onload(key, False)
    assert np.array_equal(f.gpu_read(f.dir.at(key).gpu.location), data)


def test_round_trip_reuses_page_with_new_generation(v2, v3):
    f = Fixture(v2, v3)
    key, data = make_key(v2, v3, 3), pattern(0xC33)
    f.seed_on_gpu(key, data)
    before = f.dir.at(key).gpu.location
    f.xfer.begin_offload(key)
    f.xfer.finish_offload(key, True)
    assert f.dir.at(key).gpu is None and f.gpu.allocated_chunks() == 0
    f.xfer.begin_onload(key)
    f.xfer.finish_onload(key, True)
    rec = f.dir.at(key)
    assert rec.cpu is None and rec.gpu.state == v3.ChunkState.READY
    assert rec.gpu.location.slot == before.slot and rec.gpu.location.generation != before.generation
    assert np.array_equal(f.gpu_read(rec.gpu.location), data)


def test_remapping_keeps_bytes(v2, v3):
    f = Fixture(v2, v3)
    a, b = make_key(v2, v3, 4), make_key(v2, v3, 5)
    data_a, data_b = pattern(0xD44), pattern(0xE55)
    f.seed_on_gpu(a, data_a)
    old = f.dir.at(a).gpu.location
    f.xfer.begin_offload(a)
    f.xfer.finish_offload(a, True)
    f.seed_on_gpu(b, data_b)  # B takes A's old page
    assert f.dir.at(b).gpu.location.slot == old.slot
    f.xfer.begin_onload(a)
    f.xfer.finish_onload(a, True)
    assert f.dir.at(a).gpu.location.slot != old.slot
    assert np.array_equal(f.gpu_read(f.dir.at(a).gpu.location), data_a)
    assert np.array_equal(f.gpu_read(f.dir.at(b).gpu.location), data_b)


def test_stale_location_rejected_after_reuse(v2, v3):
    f = Fixture(v2, v3)
    a, b = make_key(v2, v3, 6), make_key(v2, v3, 7)
    f.seed_on_gpu(a, pattern(0xF66))
    stale = f.dir.at(a).gpu.location
    f.xfer.begin_offload(a)
    f.xfer.finish_offload(a, True)
    f.seed_on_gpu(b, pattern(0x077))
    assert f.dir.at(b).gpu.location.slot == stale.slot
    with pytest.raises(ValueError):
        f.gpu.release(stale)
    assert np.array_equal(f.gpu_read(f.dir.at(b).gpu.location), pattern(0x077))


def test_pending_transfer_protocol(v2, v3):
    f = Fixture(v2, v3)
    key = make_key(v2, v3, 8)
    f.seed_on_gpu(key, pattern(0x188))
    f.xfer.begin_offload(key)
    assert f.xfer.has_pending(key)
    rec = f.dir.at(key)
    assert rec.gpu.state == v3.ChunkState.COPYING and rec.cpu.state == v3.ChunkState.COPYING
    assert rec.pin_count == 1
    with pytest.raises(v2.LogicError):
        f.dir.remove(key, v3.StorageTier.GPU)
    with pytest.raises(v2.LogicError):
        f.dir.destroy(key)
    with pytest.raises(v2.LogicError):
        f.xfer.begin_offload(key)
    with pytest.raises(v2.LogicError):
        f.xfer.finish_onload(key, False)  # direction mismatch
    f.xfer.finish_offload(key, True)
    assert not f.xfer.has_pending(key)
    done = f.dir.at(key)
    assert done.gpu is None and done.cpu.state == v3.ChunkState.READY and done.pin_count == 0


def test_several_transfers_in_flight(v2, v3):
    f = Fixture(v2, v3)
    keys = [make_key(v2, v3, 100 + i) for i in range(4)]
    for i, k in enumerate(keys):
        f.seed_on_gpu(k, pattern(0x900 + i))
    for k in keys:
        f.xfer.begin_offload(k)
    for k in keys:
        f.xfer.finish_offload(k, True)
    assert f.gpu.allocated_chunks() == 0 and f.cpu.allocated_chunks() == 4
    for i, k in enumerate(keys):
        assert np.array_equal(f.host_read(f.dir.at(k).cpu.location.slot), pattern(0x900 + i))


def test_random_round_trip(v2, v3):
    f = Fixture(v2, v3)
    key, data = make_key(v2, v3, 9), pattern(0xC0FFEE)
    f.seed_on_gpu(key, data)
    f.xfer.begin_offload(key)
    f.xfer.finish_offload(key, True)
    f.xfer.begin_onload(key)
    f.xfer.finish_onload(key, True)
    assert np.array_equal(f.gpu_read(f.dir.at(key).gpu.location), data)


@pytest.mark.parametrize("heap,nbytes", [(False, 32768), (False, 1000), (True, 32768)])
def test_batch_offload_onload(v2, v3, heap, nbytes):
    """A batch of 24 chunks with scattered slots: one launch (pinned pool) or
    one copy per chunk (heap pool); bytes and directory as single transfers."""
    n = 24
    f = Fixture(v2, v3, slots=48, nbytes=nbytes, heap=heap)
    # scatter the slots: occupy and free every other GPU and CPU slot first
    filler = [make_key(v2, v3, 5000 + i) for i in range(n)]
    for k in filler:
        f.dir.create(k)
        f.dir.place(k, v3.StorageTier.GPU)
        f.dir.place(k, v3.StorageTier.CPU)
    keys = [make_key(v2, v3, 6000 + i) for i in range(n)]
    data = [pattern(700 + i, nbytes) for i in range(n)]
    for k in filler[::2]:
        f.dir.remove(k, v3.StorageTier.GPU)
        f.dir.remove(k, v3.StorageTier.CPU)
    for k, d in zip(keys, data):
        f.dir.create(k)
        loc = f.dir.place(k, v3.StorageTier.CPU)
        f.host_write(loc.slot, d)
    f.xfer.begin_onload_batch(keys)
    assert all(f.xfer.has_pending(k) for k in keys)
    assert all(f.dir.at(k).gpu.state == v3.ChunkState.LOADING for k in keys)
    for k in keys:
        f.xfer.finish_onload(k, True)
    for k, d in zip(keys, data):
        assert f.dir.at(k).cpu is None
        assert np.array_equal(f.gpu_read(f.dir.at(k).gpu.location), d)
    f.xfer.begin_offload_batch(keys)
    for k in keys[::-1]:  # any finishing order
        f.xfer.finish_offload(k, True)
    for k, d in zip(keys, data):
        rec = f.dir.at(k)
        assert rec.gpu is None and rec.cpu.state == v3.ChunkState.READY and rec.pin_count == 0
        assert np.array_equal(f.host_read(rec.cpu.location.slot), d)
    # a rejected batch changes nothing: one key has no CPU replica to onload
    bad = keys[:3] + [filler[1]]
    f.dir.remove(filler[1], v3.StorageTier.CPU)
    def state(k):
        rec = f.dir.at(k)
        return (rec.gpu is None, None if rec.cpu is None else (rec.cpu.location.slot, rec.cpu.state), rec.pin_count)

    states = [state(k) for k in bad]
    with pytest.raises(v2.LogicError):
        f.xfer.begin_onload_batch(bad)
    assert [state(k) for k in bad] == states
    assert not any(f.xfer.has_pending(k) for k in bad)
    with pytest.raises(v2.LogicError):  # duplicate key
        f.xfer.begin_onload_batch([keys[0], keys[0]])
