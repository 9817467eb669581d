"""The MFMA attention kernels next to slots that were never written.

The reference's attention test fills the cache with NaN before writing
(tests/paged_attention_test.cu:73-130) so that a kernel touching a slot past a
sequence's length, or a page it does not own, shows up as a non-finite
output. Its shapes (head_size 4) run on the exact kernels; here the same
check runs where the fast kernels load whole 16-token tiles and 64-key tiles,
so the unwritten slots of a sequence's last page are loaded too and must
carry zero weight without their NaN reaching the output:
  * decode batch (block-size-16 kernel, pages of 16/32/64 tokens): 1e-5
    against the oracle's reference attention on the gathered K/V;
  * whole-prompt and suffix prefill (MFMA prefill, AttentionPrecision::Fast):
    2e-2, the bound of the BF16/FP16 MFMA path.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import DTYPES, buffer_like, decode, fill_cache
from kvflux_amd import device
from oracle import oracle

pytestmark = pytest.mark.gpu

LENGTHS = [500, 37, 129, 1]  # none but the last a multiple of the page size
KV_HEADS, Q_HEADS, HEAD = 2, 8, 128


def build(v2, name, bs):
    pool = v2.PhysicalBlockPool(64, bs)
    storage = v2.PagedKVStorage(pool, KV_HEADS, HEAD, getattr(v2.DType, name))
    seqs = [v2.SequenceState(100 + i, pool) for i in range(len(LENGTHS))]
    # Appends in rounds so the sequences' pages interleave in the pool.
    left = list(LENGTHS)
    while any(left):
        for s, n in zip(seqs, left):
            if n:
                s.append_tokens(min(n, bs + 3))
        left = [max(0, n - bs - 3) for n in left]
    assert [s.num_tokens() for s in seqs] == LENGTHS
    fill_cache(storage, 0xFF)  # NaN in every slot not written below
    writes = [(s, t) for s in seqs for t in range(s.num_tokens())]
    n = len(writes) * KV_HEADS * HEAD
    code, dt = DTYPES[name]
    kd, vd = device.DeviceBuffer(n * 2), device.DeviceBuffer(n * 2)
    device.fill_random(kd.ptr, n, code, 1, 11 + bs)
    device.fill_random(vd.ptr, n, code, 1, 12 + bs)
    v2.write_paged_kv(storage, kd.ptr, vd.ptr, v2.build_slot_mapping(writes))
    contiguous = []
    for s in seqs:
        m = s.num_tokens() * KV_HEADS * HEAD
        gk, gv = device.DeviceBuffer(m * 2), device.DeviceBuffer(m * 2)
        v2.read_paged_kv(storage, s, gk.ptr, gv.ptr)
        k, v = decode(gk.download(dt), name), decode(gv.download(dt), name)
        assert np.all(np.isfinite(k)) and np.all(np.isfinite(v))
        contiguous.append((k, v))
    return pool, storage, seqs, contiguous


@pytest.mark.parametrize("name", ["BFloat16", "Float16"])
@pytest.mark.parametrize("bs", [16, 32, 64])
def test_decode_batch_ignores_unwritten_slots(gpu, v2, name, bs):
    pool, storage, seqs, kv = build(v2, name, bs)
    nq = len(seqs) * Q_HEADS * HEAD
    q = oracle.random_elements(0, nq, oracle.F32, 1, 5 + bs)
    qd = buffer_like(q)
    od = buffer_like(np.full(nq + 1, 4321.0, np.float32))
    v2.paged_attention_batch(storage, seqs, qd.ptr, od.ptr, Q_HEADS)
    got = od.download(np.float32)
    assert got[nq] == 4321.0
    assert np.all(np.isfinite(got[:nq]))
    per = Q_HEADS * HEAD
    for r, (s, (k, v)) in enumerate(zip(seqs, kv)):
        exp = oracle.reference_attention(q[r * per:(r + 1) * per], k, v, 1, s.num_tokens(), Q_HEADS, KV_HEADS,
                                         HEAD)
        assert np.abs(got[r * per:(r + 1) * per] - exp).max() < 1e-5, r


@pytest.mark.parametrize("name", ["BFloat16", "Float16"])
@pytest.mark.parametrize("bs", [16, 64])
def test_prefill_ignores_unwritten_slots(gpu, v2, name, bs):
    pool, storage, seqs, kv = build(v2, name, bs)
    for which, q_tokens in ((0, 500), (0, 37), (2, 129), (1, 20)):
        s, (k, v) = seqs[which], kv[which]
        n = q_tokens * Q_HEADS * HEAD
        q = oracle.random_elements(0, n, oracle.F32, 1, 7 * q_tokens + bs)
        qd = buffer_like(q)
        od = buffer_like(np.full(n + 1, 4321.0, np.float32))
        v2.paged_attention(storage, s, qd.ptr, od.ptr, q_tokens, Q_HEADS, v2.AttentionPrecision.Fast)
        got = od.download(np.float32)
        assert got[n] == 4321.0
        assert np.all(np.isfinite(got[:n])), (which, q_tokens)
        exp = oracle.reference_attention(q, k, v, q_tokens, s.num_tokens(), Q_HEADS, KV_HEADS, HEAD)
        assert np.abs(got[:n] - exp).max() < 2e-2, (which, q_tokens)
