"""The extension's C++ timing loops over the synchronous API (used by
bench.py): each runs the real call, so its effects must equal one direct
call's, and it returns a positive time per call."""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import buffer_like
from kvflux_amd import device
from oracle import oracle

pytestmark = pytest.mark.gpu


def test_timing_loops_run_the_api(gpu, v2):
    H, D, bs = 2, 128, 16
    pool = v2.PhysicalBlockPool(64, bs)
    storage = v2.PagedKVStorage(pool, H, D, v2.DType.BFloat16)
    seqs = []
    for i, L in enumerate((37, 100)):
        s = v2.SequenceState(i, pool)
        s.append_tokens(L)
        seqs.append(s)
    slots = v2.build_slot_mapping([(seqs[1], t) for t in range(100)])
    kn = oracle.random_elements(0, 100 * H * D, oracle.BF16, 1, 5)
    vn = oracle.random_elements(0, 100 * H * D, oracle.BF16, 1, 6)
    kd, vd = buffer_like(kn), buffer_like(vn)
    assert v2.timing.write_paged_kv(storage, kd.ptr, vd.ptr, slots, 2) > 0
    total = 137
    ko, vo = device.DeviceBuffer(total * H * D * 2), device.DeviceBuffer(total * H * D * 2)
    assert v2.timing.read_paged_kv_batch(storage, seqs, ko.ptr, vo.ptr, 2) > 0
    # the second sequence's rows come back as written
    got_k = device.memcpy_d2h(ko.ptr + 37 * H * D * 2, 100 * H * D * 2, np.uint16)
    assert np.array_equal(got_k, kn)
    q = oracle.random_elements(0, 100 * 8 * D, oracle.F32, 1, 7)
    qd = buffer_like(q)
    od1, od2 = buffer_like(np.zeros(q.size, np.float32)), buffer_like(np.zeros(q.size, np.float32))
    assert v2.timing.paged_attention(storage, [seqs[1]], [qd.ptr], [od1.ptr], 8, v2.AttentionPrecision.Fast, 2) > 0
    v2.paged_attention(storage, seqs[1], qd.ptr, od2.ptr, 100, 8, v2.AttentionPrecision.Fast)
    assert np.array_equal(od1.download(np.float32).view(np.uint32), od2.download(np.float32).view(np.uint32))
    with pytest.raises(ValueError):
        v2.timing.write_paged_kv(storage, kd.ptr, vd.ptr, slots, 0)
