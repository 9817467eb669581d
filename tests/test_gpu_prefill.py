"""GPU parity of the MFMA causal prefill kernel (kvflux_paged_prefill).

Two references per case:
  * the CPU reference attention (oracle, a restatement of the reference's
    causal paged attention) at the 2e-2 bound the BF16/FP16 MFMA path is
    specified to;
  * a float64 evaluation of the same arithmetic the kernel performs on its
    inputs -- Q scaled by log2(e)/sqrt(D) and rounded to the cache dtype,
    exact scores, exact softmax -- which leaves only the rounding of the
    softmax weights to the cache dtype, so a misplaced key, dimension or head
    would show up far above its 4e-3 bound.
Caches come from the counter generator (N(0,1) in the cache dtype), pages
from a seeded permutation of the pool.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from gpu_util import buffer_like
from kvflux_amd import capi, device
from oracle import oracle

pytestmark = pytest.mark.gpu

CODES = {"BFloat16": oracle.BF16, "Float16": oracle.F16}


def setup_case(name, blocks, kv_heads, bs, head_size, kv_len, seed):
    code = CODES[name]
    page = kv_heads * bs * head_size
    kc = device.DeviceBuffer(blocks * page * 2)
    vc = device.DeviceBuffer(blocks * page * 2)
    device.fill_random(kc.ptr, blocks * page, code, 1, seed * 3 + 1)
    device.fill_random(vc.ptr, blocks * page, code, 1, seed * 3 + 2)
    npages = (kv_len + bs - 1) // bs
    table = np.random.default_rng(seed).permutation(blocks)[:npages].astype(np.uint64)
    return kc, vc, table


def run_prefill(name, kc, vc, blocks, kv_heads, bs, head_size, table, kv_len, q, q_tokens, q_heads):
    lib = capi.lib()
    td = buffer_like(table)
    qd = buffer_like(q)
    od = buffer_like(np.full(q.size + 4, 777.0, np.float32))
    status = lib.kvflux_paged_prefill(kc.ptr, vc.ptr, blocks, kv_heads, bs, head_size, CODES[name],
                                      td.ptr, len(table), kv_len, q_tokens, q_heads, qd.ptr, od.ptr, None)
    assert status == 0, capi.last_error()
    device.synchronize()
    out = od.download(np.float32)
    assert np.all(out[q.size:] == 777.0)  # nothing written past the output
    return out[:q.size]


def emulate(kc_host, vc_host, name, kv_heads, bs, head_size, table, kv_len, q, q_tokens, q_heads, rows):
    """float64 attention with Q rounded as the kernel rounds it."""
    code = CODES[name]
    G = q_heads // kv_heads
    k = oracle.decode(kc_host, code).reshape(-1, kv_heads, bs, head_size)
    v = oracle.decode(vc_host, code).reshape(-1, kv_heads, bs, head_size)
    t = np.arange(kv_len)
    pages = table[t // bs].astype(np.int64)
    K = k[pages, :, t % bs, :].astype(np.float64)  # [kv_len][H][D]
    V = v[pages, :, t % bs, :].astype(np.float64)
    scale = np.float32(1.4426950408889634 / np.sqrt(head_size))
    qr = q.reshape(q_tokens, q_heads, head_size)
    out = np.zeros((len(rows), q_heads, head_size))
    for i, tok in enumerate(rows):
        last = kv_len - q_tokens + tok
        for hq in range(q_heads):
            scaled = (qr[tok, hq] * scale).astype(np.float32)
            qq = oracle.decode(oracle.encode(scaled, code), code).astype(np.float64)
            s = K[:last + 1, hq // G] @ qq
            w = np.exp2(s - s.max())
            out[i, hq] = (w @ V[:last + 1, hq // G]) / w.sum()
    return out


CASES = [  # name, kv_heads, q_heads, head_size, bs, kv_len, q_tokens
    ("BFloat16", 2, 8, 128, 16, 1000, 1000),
    ("BFloat16", 2, 8, 128, 16, 700, 37),
    ("BFloat16", 1, 8, 128, 32, 333, 333),
    ("Float16", 2, 4, 64, 16, 600, 600),
    ("BFloat16", 4, 4, 64, 64, 300, 300),
    ("Float16", 1, 2, 128, 16, 513, 100),
    # Rows are head-minor (row r: head r % G of token r / G), so any group up
    # to 256 runs in one launch: groups that do not divide the 256 rows of a
    # workgroup (up to G - 1 idle rows), and 10, 11, 12, 32 in one pass.
    ("BFloat16", 2, 6, 128, 16, 500, 500),
    ("Float16", 1, 5, 64, 32, 400, 170),
    ("BFloat16", 2, 12, 64, 16, 300, 300),
    ("BFloat16", 1, 7, 128, 16, 450, 450),
    ("BFloat16", 2, 32, 128, 16, 260, 260),
    ("BFloat16", 1, 10, 128, 16, 129, 40),
    ("BFloat16", 1, 11, 64, 16, 150, 150),
    ("Float16", 1, 12, 128, 64, 333, 333),
    ("BFloat16", 1, 32, 64, 16, 200, 200),
    # head_size 256: 8 row blocks of 16 per workgroup (group 3 leaves 2 rows
    # idle)
    ("BFloat16", 2, 2, 256, 16, 400, 400),
    ("Float16", 1, 3, 256, 32, 300, 120),
    ("BFloat16", 2, 8, 256, 16, 260, 260),
    ("BFloat16", 1, 16, 256, 64, 150, 150),
    # long prompts; the workgroup's page list holds 2048 pages at a time and
    # is restaged at each window boundary
    ("BFloat16", 2, 8, 128, 16, 40000, 64),
    ("Float16", 1, 2, 256, 16, 40000, 40),
    ("BFloat16", 1, 4, 64, 4, 30000, 33),
    ("BFloat16", 1, 4, 64, 1, 20000, 300),
    ("Float16", 1, 2, 256, 4, 40000, 40),
    ("BFloat16", 2, 8, 128, 16, 140000, 16),
    # pages longer than a 64-key tile (a tile is part of one page)
    ("BFloat16", 2, 8, 128, 128, 1000, 1000),
    ("Float16", 1, 4, 64, 256, 700, 300),
    ("BFloat16", 1, 2, 256, 128, 9000, 40),
]


@pytest.mark.parametrize("name,kv_heads,q_heads,head_size,bs,kv_len,q_tokens", CASES)
def test_prefill_matches_reference(gpu, name, kv_heads, q_heads, head_size, bs, kv_len, q_tokens):
    blocks = (kv_len + bs - 1) // bs + 17
    seed = kv_len + q_tokens
    kc, vc, table = setup_case(name, blocks, kv_heads, bs, head_size, kv_len, seed)
    q = oracle.random_elements(0, q_tokens * q_heads * head_size, oracle.F32, 1, seed)
    got = run_prefill(name, kc, vc, blocks, kv_heads, bs, head_size, table, kv_len, q, q_tokens, q_heads)
    assert np.all(np.isfinite(got))
    kh, vh = kc.download(np.uint16), vc.download(np.uint16)
    exp = oracle.paged_attention_causal(kh, vh, kv_heads, bs, head_size, CODES[name], table, kv_len, q,
                                        q_tokens, q_heads, threads=8)
    err = np.abs(got - exp)
    assert err.max() < 2e-2, err.max()
    rows = sorted({0, 1, q_tokens // 2, q_tokens - 2, q_tokens - 1} & set(range(q_tokens)))
    emu = emulate(kh, vh, name, kv_heads, bs, head_size, table, kv_len, q, q_tokens, q_heads, rows)
    sub = got.reshape(q_tokens, q_heads, head_size)[rows]
    assert np.abs(sub - emu).max() < 4e-3


def test_prefill_deterministic_and_unsupported(gpu):
    name, H, Hq, D, bs, L = "BFloat16", 2, 8, 128, 16, 400
    blocks = 40
    kc, vc, table = setup_case(name, blocks, H, bs, D, L, 3)
    q = oracle.random_elements(0, L * Hq * D, oracle.F32, 1, 3)
    a = run_prefill(name, kc, vc, blocks, H, bs, D, table, L, q, L, Hq)
    b = run_prefill(name, kc, vc, blocks, H, bs, D, table, L, q, L, Hq)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    lib = capi.lib()
    td, qd, od = buffer_like(table), buffer_like(q), buffer_like(np.zeros(q.size, np.float32))
    # FP32 caches at head_size 256, head_sizes 96 and 512 and block_size 48
    # are left to the split-K kernels.
    assert lib.kvflux_paged_prefill(kc.ptr, vc.ptr, blocks, H, bs, 256, capi.DTYPE_F32, td.ptr, len(table), L, L,
                                    Hq, qd.ptr, od.ptr, None) == capi.ERR_UNSUPPORTED
    assert lib.kvflux_paged_prefill(kc.ptr, vc.ptr, blocks, H, bs, 96, capi.DTYPE_BF16, td.ptr, len(table), L, L,
                                    Hq, qd.ptr, od.ptr, None) == capi.ERR_UNSUPPORTED
    assert lib.kvflux_paged_prefill(kc.ptr, vc.ptr, blocks, H, bs, 512, capi.DTYPE_BF16, td.ptr, len(table), L, L,
                                    Hq, qd.ptr, od.ptr, None) == capi.ERR_UNSUPPORTED
    assert lib.kvflux_paged_prefill(kc.ptr, vc.ptr, blocks, H, 48, D, capi.DTYPE_BF16, td.ptr, len(table), L, L,
                                    Hq, qd.ptr, od.ptr, None) == capi.ERR_UNSUPPORTED
    # kv_len of 2^31 tokens or more (declined before anything is read)
    assert lib.kvflux_paged_prefill(kc.ptr, vc.ptr, blocks, H, 1, D, capi.DTYPE_BF16, td.ptr, 2**31, 2**31, 1,
                                    Hq, qd.ptr, od.ptr, None) == capi.ERR_UNSUPPORTED
    # table too short for kv_len, more queries than tokens
    assert lib.kvflux_paged_prefill(kc.ptr, vc.ptr, blocks, H, bs, D, capi.DTYPE_BF16, td.ptr, 3, L, L,
                                    Hq, qd.ptr, od.ptr, None) == capi.ERR_INVALID
    assert lib.kvflux_paged_prefill(kc.ptr, vc.ptr, blocks, H, bs, D, capi.DTYPE_BF16, td.ptr, len(table), L,
                                    L + 1, Hq, qd.ptr, od.ptr, None) == capi.ERR_INVALID


@pytest.mark.parametrize("kv_heads,q_heads", [(2, 8), (1, 16), (2, 10)])
def test_prefill_through_cpp_layer(gpu, v2, kv_heads, q_heads):
    """AttentionPrecision::Fast routes a whole-prompt call to the MFMA kernel
    (GQA groups 4, 16 and 5)."""
    pool = v2.PhysicalBlockPool(64, 16)
    storage = v2.PagedKVStorage(pool, kv_heads, 128, v2.DType.BFloat16)
    seq = v2.SequenceState(1, pool)
    seq.append_tokens(500)
    n = storage.layout().cache_bytes() // 2
    device.fill_random(storage.key_base(), n, oracle.BF16, 1, 71)
    device.fill_random(storage.value_base(), n, oracle.BF16, 1, 72)
    q = oracle.random_elements(0, 500 * q_heads * 128, oracle.F32, 1, 73)
    qd, od = buffer_like(q), buffer_like(np.zeros(q.size, np.float32))
    v2.paged_attention(storage, seq, qd.ptr, od.ptr, 500, q_heads, v2.AttentionPrecision.Fast)
    got = od.download(np.float32)
    kh = device.memcpy_d2h(storage.key_base(), storage.layout().cache_bytes(), np.uint16)
    vh = device.memcpy_d2h(storage.value_base(), storage.layout().cache_bytes(), np.uint16)
    table = np.array(v2.build_read_block_table(seq), np.uint64)
    exp = oracle.paged_attention_causal(kh, vh, kv_heads, 16, 128, oracle.BF16, table, 500, q, 500, q_heads,
                                        threads=8)
    assert np.abs(got - exp).max() < 2e-2
    # the same bits as the MFMA kernel called through the C ABI (with the
    # workspace that lets it split the keys, as the C++ layer does)
    td, od2 = buffer_like(table), buffer_like(np.zeros(q.size, np.float32))
    ws = C.c_size_t(0)
    capi.check(capi.lib().kvflux_paged_prefill_workspace_size(kv_heads, 128, 500, 500, q_heads, C.byref(ws)))
    wd = device.DeviceBuffer(max(ws.value, 16))
    assert capi.lib().kvflux_paged_prefill_split(storage.key_base(), storage.value_base(), 64, kv_heads, 16, 128,
                                                 capi.DTYPE_BF16, td.ptr, len(table), 500, 500, q_heads, qd.ptr,
                                                 od2.ptr, wd.ptr, ws.value, None) == 0
    device.synchronize()
    assert np.array_equal(od2.download(np.float32).view(np.uint32), got.view(np.uint32))


def test_precision_routing(gpu, v2):
    """Auto sends calls of 16 or more query tokens to the MFMA prefill (the
    same bits as Fast) and fewer to the exact kernels (the same bits as
    Exact, which is within 1e-5 of the oracle). The reference's own
    six-argument signature (no precision) is Exact at every length."""
    pool = v2.PhysicalBlockPool(64, 16)
    storage = v2.PagedKVStorage(pool, 2, 128, v2.DType.BFloat16)
    seq = v2.SequenceState(1, pool)
    seq.append_tokens(300)
    n = storage.layout().cache_bytes() // 2
    device.fill_random(storage.key_base(), n, oracle.BF16, 1, 81)
    device.fill_random(storage.value_base(), n, oracle.BF16, 1, 82)
    kh = device.memcpy_d2h(storage.key_base(), storage.layout().cache_bytes(), np.uint16)
    vh = device.memcpy_d2h(storage.value_base(), storage.layout().cache_bytes(), np.uint16)
    table = np.array(v2.build_read_block_table(seq), np.uint64)
    P = v2.AttentionPrecision
    for q_tokens in (15, 16):
        q = oracle.random_elements(0, q_tokens * 8 * 128, oracle.F32, 1, 83 + q_tokens)
        qd = buffer_like(q)
        out = {}
        for prec in (P.Auto, P.Fast, P.Exact):
            od = buffer_like(np.zeros(q.size, np.float32))
            v2.paged_attention(storage, seq, qd.ptr, od.ptr, q_tokens, 8, prec)
            out[prec] = od.download(np.float32).view(np.uint32)
        od = buffer_like(np.zeros(q.size, np.float32))
        v2.paged_attention(storage, seq, qd.ptr, od.ptr, q_tokens, 8)  # reference signature
        assert np.array_equal(od.download(np.float32).view(np.uint32), out[P.Exact]), q_tokens
        twin = P.Exact if q_tokens < 16 else P.Fast
        assert np.array_equal(out[P.Auto], out[twin]), q_tokens
        exp = oracle.paged_attention_causal(kh, vh, 2, 16, 128, oracle.BF16, table, 300, q, q_tokens, 8)
        assert np.abs(out[P.Exact].view(np.float32) - exp).max() < 1e-5
        assert np.abs(out[P.Fast].view(np.float32) - exp).max() < 2e-2
    assert not np.array_equal(out[P.Fast], out[P.Exact])  # two different kernels


SPLIT_CASES = [  # name, kv_heads, q_heads, head_size, bs, kv_len, q_tokens
    ("BFloat16", 8, 32, 128, 16, 8192, 64),    # chunked prefill against a long prefix
    ("BFloat16", 2, 8, 128, 16, 5126, 100),    # split 16 starts at key 5120, inside the last
                                               # block's diagonal (rows 5090..5119 see none of it)
    ("Float16", 1, 16, 128, 16, 3000, 40),     # group 16, one token block per workgroup
    ("BFloat16", 2, 20, 64, 32, 4000, 77),     # group 10 in one launch, then one combine
    ("BFloat16", 1, 300, 64, 16, 1000, 3),     # group 300 as 2 x 150 passes, then one combine
    ("BFloat16", 1, 2, 256, 16, 6000, 48),
    ("BFloat16", 1, 4, 128, 1, 20000, 16),     # page-list windows inside splits
    ("BFloat16", 2, 8, 128, 16, 3000, 1),      # one query token (Fast precision sends it here)
    ("Float16", 1, 6, 64, 64, 2500, 2),        # group 6 with two tokens
    ("BFloat16", 2, 8, 128, 128, 6000, 64),    # 128-token pages
    # A split starting one tile before a page-list window boundary (2048
    # pages = 32 tiles at block_size 1, 512 tiles at 16): the window is
    # restaged right after the split's first tile is issued.
    ("BFloat16", 1, 4, 128, 1, 63300, 16),     # 31 tiles per split: split 1 starts at tile 31
    ("BFloat16", 1, 4, 128, 16, 148000, 16),   # 73 tiles per split: split 7 starts at tile 511
]


@pytest.mark.parametrize("name,kv_heads,q_heads,head_size,bs,kv_len,q_tokens", SPLIT_CASES)
def test_prefill_split_keys(gpu, name, kv_heads, q_heads, head_size, bs, kv_len, q_tokens):
    """kvflux_paged_prefill_split: the keys of each (query block, kv head)
    spread over several workgroups and merged by the combine kernel. Matches
    the oracle (2e-2), the float64 emulation (4e-3) and the unsplit kernel."""
    blocks = (kv_len + bs - 1) // bs + 17
    seed = kv_len + 3 * q_tokens
    kc, vc, table = setup_case(name, blocks, kv_heads, bs, head_size, kv_len, seed)
    q = oracle.random_elements(0, q_tokens * q_heads * head_size, oracle.F32, 1, seed)
    lib = capi.lib()
    ws = C.c_size_t(0)
    capi.check(lib.kvflux_paged_prefill_workspace_size(kv_heads, head_size, kv_len, q_tokens, q_heads, C.byref(ws)))
    assert ws.value > 0  # the call splits
    td, qd = buffer_like(table), buffer_like(q)
    wd = device.DeviceBuffer(ws.value)
    od = buffer_like(np.full(q.size + 4, 777.0, np.float32))
    assert lib.kvflux_paged_prefill_split(kc.ptr, vc.ptr, blocks, kv_heads, bs, head_size, CODES[name], td.ptr,
                                          len(table), kv_len, q_tokens, q_heads, qd.ptr, od.ptr, wd.ptr, ws.value,
                                          None) == 0, capi.last_error()
    assert lib.kvflux_paged_prefill_split(kc.ptr, vc.ptr, blocks, kv_heads, bs, head_size, CODES[name], td.ptr,
                                          len(table), kv_len, q_tokens, q_heads, qd.ptr, od.ptr, wd.ptr,
                                          ws.value - 1, None) == capi.ERR_INVALID
    device.synchronize()
    out = od.download(np.float32)
    assert np.all(out[q.size:] == 777.0)
    got = out[:q.size]
    assert np.all(np.isfinite(got))
    kh, vh = kc.download(np.uint16), vc.download(np.uint16)
    exp = oracle.paged_attention_causal(kh, vh, kv_heads, bs, head_size, CODES[name], table, kv_len, q, q_tokens,
                                        q_heads, threads=8)
    assert np.abs(got - exp).max() < 2e-2
    rows = sorted({0, 1, q_tokens // 2, q_tokens - 2, q_tokens - 1} & set(range(q_tokens)))
    emu = emulate(kh, vh, name, kv_heads, bs, head_size, table, kv_len, q, q_tokens, q_heads, rows)
    assert np.abs(got.reshape(q_tokens, q_heads, head_size)[rows] - emu).max() < 4e-3
    whole = run_prefill(name, kc, vc, blocks, kv_heads, bs, head_size, table, kv_len, q, q_tokens, q_heads)
    assert np.abs(got - whole).max() < 4e-3


GAP_CASES = [  # name, kv_heads, q_heads, head_size, bs, kv_len, q_tokens, missing table entries
    ("BFloat16", 2, 8, 128, 4, 500, 500, [3, 40, 124]),
    ("Float16", 1, 8, 64, 8, 333, 120, [0, 20, 41]),
    ("BFloat16", 2, 4, 128, 1, 130, 130, [7, 129]),
    ("BFloat16", 2, 8, 128, 128, 700, 700, [1, 5]),
]


@pytest.mark.parametrize("name,kv_heads,q_heads,head_size,bs,kv_len,q_tokens,missing", GAP_CASES)
def test_prefill_small_pages_and_missing_ids(gpu, name, kv_heads, q_heads, head_size, bs, kv_len, q_tokens,
                                             missing):
    """Block sizes below 16 (a 64-key tile spans 16 to 64 pages) and table
    entries that are not pages of the pool: such a page reads as zeros for K
    and V. The references see the same cache with one all-zero page appended
    and the missing entries pointing at it."""
    blocks = (kv_len + bs - 1) // bs + 17
    seed = kv_len + q_tokens + bs
    kc, vc, table = setup_case(name, blocks, kv_heads, bs, head_size, kv_len, seed)
    table = table.copy()
    table[missing] = 2**64 - 1
    q = oracle.random_elements(0, q_tokens * q_heads * head_size, oracle.F32, 1, seed)
    got = run_prefill(name, kc, vc, blocks, kv_heads, bs, head_size, table, kv_len, q, q_tokens, q_heads)
    assert np.all(np.isfinite(got))
    page = kv_heads * bs * head_size
    kh = np.concatenate([kc.download(np.uint16), np.zeros(page, np.uint16)])
    vh = np.concatenate([vc.download(np.uint16), np.zeros(page, np.uint16)])
    ref_table = table.copy()
    ref_table[missing] = blocks  # the appended zero page
    exp = oracle.paged_attention_causal(kh, vh, kv_heads, bs, head_size, CODES[name], ref_table, kv_len, q,
                                        q_tokens, q_heads, threads=8)
    assert np.abs(got - exp).max() < 2e-2
    rows = sorted({0, 1, q_tokens // 2, q_tokens - 2, q_tokens - 1} & set(range(q_tokens)))
    emu = emulate(kh, vh, name, kv_heads, bs, head_size, ref_table, kv_len, q, q_tokens, q_heads, rows)
    sub = got.reshape(q_tokens, q_heads, head_size)[rows]
    assert np.abs(sub - emu).max() < 4e-3


BATCH_CASES = [  # name, kv_heads, q_heads, head_size, bs, [(kv_len, q_len), ...]
    ("BFloat16", 2, 8, 128, 16, [(700, 700), (1500, 1500), (64, 64), (1000, 37), (2049, 2049)]),
    ("Float16", 1, 5, 64, 4, [(300, 300), (257, 100), (33, 33)]),
    ("BFloat16", 2, 4, 256, 32, [(400, 400), (1200, 800)]),
    ("BFloat16", 1, 12, 128, 1, [(200, 200), (150, 1)]),  # group 12: 21 tokens per workgroup
    ("Float16", 1, 320, 64, 16, [(40, 40), (90, 7)]),     # group 320 as 2 x 160 passes
]


@pytest.mark.parametrize("name,kv_heads,q_heads,head_size,bs,seqs", BATCH_CASES)
def test_prefill_batch_matches_single_calls(gpu, name, kv_heads, q_heads, head_size, bs, seqs):
    """kvflux_paged_prefill_batch: every sequence of the batch, with its own
    table row, length, query count (whole prompts and trailing chunks) and
    query offset, gives the same bits as kvflux_paged_prefill on that
    sequence alone; rows between sequences are untouched; a sampled check
    against the oracle at 2e-2."""
    lib = capi.lib()
    n = len(seqs)
    width = max((kv + bs - 1) // bs for kv, _ in seqs) + 3
    blocks = n * width + 5
    kc, vc, _ = setup_case(name, blocks, kv_heads, bs, head_size, 1, 17 + n)
    rng = np.random.default_rng(23 + n)
    order = rng.permutation(blocks).astype(np.uint64)
    table = np.full((n, width), 2**64 - 1, np.uint64)
    for i, (kv, _) in enumerate(seqs):
        npg = (kv + bs - 1) // bs
        table[i, :npg] = order[i * width:i * width + npg]
    q_lens = np.array([ql for _, ql in seqs], np.uint64)
    kv_lens = np.array([kv for kv, _ in seqs], np.uint64)
    gap = 3  # unused rows between sequences in Q/O
    offsets = np.concatenate([[0], np.cumsum(q_lens + gap)[:-1]]).astype(np.uint64)
    rows_total = int(offsets[-1] + q_lens[-1] + gap)
    row = q_heads * head_size
    q = oracle.random_elements(0, rows_total * row, oracle.F32, 1, 29 + n)
    td, qd = buffer_like(table.reshape(-1)), buffer_like(q)
    kd, ld, od_ = buffer_like(kv_lens), buffer_like(q_lens), buffer_like(offsets)
    out = buffer_like(np.full(rows_total * row, 555.0, np.float32))
    assert lib.kvflux_paged_prefill_batch(kc.ptr, vc.ptr, blocks, kv_heads, bs, head_size, CODES[name], td.ptr,
                                          width, kd.ptr, ld.ptr, od_.ptr, n, int(q_lens.max()), int(kv_lens.max()),
                                          q_heads, qd.ptr, out.ptr, None) == 0, capi.last_error()
    device.synchronize()
    got = out.download(np.float32).reshape(rows_total, row)
    used = np.zeros(rows_total, bool)
    kh, vh = kc.download(np.uint16), vc.download(np.uint16)
    for i, (kv, ql) in enumerate(seqs):
        o0 = int(offsets[i])
        used[o0:o0 + ql] = True
        qi = q.reshape(rows_total, row)[o0:o0 + ql].reshape(-1)
        single = run_prefill(name, kc, vc, blocks, kv_heads, bs, head_size, table[i], kv, qi, ql, q_heads)
        assert np.array_equal(got[o0:o0 + ql].reshape(-1).view(np.uint32), single.view(np.uint32)), i
        pick = sorted({0, ql - 1, ql // 2})
        exp = oracle.paged_attention_rows(kh, vh, kv_heads, bs, head_size, CODES[name], np.tile(table[i], len(pick)),
                                          width, np.array([kv - ql + t + 1 for t in pick], np.uint64),
                                          qi.reshape(ql, row)[pick].reshape(-1), q_heads, threads=8)
        assert np.abs(got[o0:o0 + ql][pick].reshape(-1) - exp).max() < 2e-2
    assert np.all(got[~used] == 555.0)


def random_batch_configs(count, seed):
    """Seeded draws over the prefill's shape space: dtype, head_size, kv
    heads, GQA group, page size and a batch of 1-4 sequences, each a whole
    prompt or a trailing chunk."""
    rng = np.random.default_rng(seed)
    configs = []
    for _ in range(count):
        name = ("BFloat16", "Float16")[int(rng.integers(2))]
        head_size = int(rng.choice([64, 128, 256]))
        kv_heads = int(rng.integers(1, 3))
        group = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 16]))
        bs = int(rng.choice([1, 2, 4, 8, 16, 32, 64, 128, 256]))
        seqs = []
        for _ in range(int(rng.integers(1, 5))):
            kv = int(rng.integers(1, 1501))
            ql = kv if rng.random() < 0.5 else int(rng.integers(1, kv + 1))
            seqs.append((kv, ql))
        configs.append((name, kv_heads, kv_heads * group, head_size, bs, seqs))
    return configs


@pytest.mark.parametrize("case", range(10))
def test_prefill_batch_random_shapes(gpu, case):
    """kvflux_paged_prefill_batch over seeded random shapes: sampled rows of
    every sequence (first, last, middle) against the oracle at 2e-2 and
    against the float64 emulation of the kernel's rounding at 4e-3; rows
    outside the sequences untouched."""
    name, kv_heads, q_heads, head_size, bs, seqs = random_batch_configs(10, 4242)[case]
    lib = capi.lib()
    n = len(seqs)
    width = max((kv + bs - 1) // bs for kv, _ in seqs) + 2
    blocks = n * width + 3
    kc, vc, _ = setup_case(name, blocks, kv_heads, bs, head_size, 1, 90 + case)
    order = np.random.default_rng(91 + case).permutation(blocks).astype(np.uint64)
    table = np.full((n, width), 2**64 - 1, np.uint64)
    for i, (kv, _) in enumerate(seqs):
        npg = (kv + bs - 1) // bs
        table[i, :npg] = order[i * width:i * width + npg]
    q_lens = np.array([ql for _, ql in seqs], np.uint64)
    kv_lens = np.array([kv for kv, _ in seqs], np.uint64)
    offsets = np.concatenate([[0], np.cumsum(q_lens + 1)[:-1]]).astype(np.uint64)
    rows_total = int(offsets[-1] + q_lens[-1] + 1)
    row = q_heads * head_size
    q = oracle.random_elements(0, rows_total * row, oracle.F32, 1, 92 + case)
    td, qd = buffer_like(table.reshape(-1)), buffer_like(q)
    kd, ld, od_ = buffer_like(kv_lens), buffer_like(q_lens), buffer_like(offsets)
    out = buffer_like(np.full(rows_total * row, 555.0, np.float32))
    assert lib.kvflux_paged_prefill_batch(kc.ptr, vc.ptr, blocks, kv_heads, bs, head_size, CODES[name], td.ptr,
                                          width, kd.ptr, ld.ptr, od_.ptr, n, int(q_lens.max()), int(kv_lens.max()),
                                          q_heads, qd.ptr, out.ptr, None) == 0, capi.last_error()
    device.synchronize()
    got = out.download(np.float32).reshape(rows_total, row)
    used = np.zeros(rows_total, bool)
    kh, vh = kc.download(np.uint16), vc.download(np.uint16)
    for i, (kv, ql) in enumerate(seqs):
        o0 = int(offsets[i])
        used[o0:o0 + ql] = True
        qi = q.reshape(rows_total, row)[o0:o0 + ql].reshape(-1)
        pick = sorted({0, ql - 1, ql // 2})
        exp = oracle.paged_attention_rows(kh, vh, kv_heads, bs, head_size, CODES[name], np.tile(table[i], len(pick)),
                                          width, np.array([kv - ql + t + 1 for t in pick], np.uint64),
                                          qi.reshape(ql, row)[pick].reshape(-1), q_heads, threads=8)
        sub = got[o0:o0 + ql][pick]
        assert np.all(np.isfinite(sub))
        assert np.abs(sub.reshape(-1) - exp).max() < 2e-2, (i, kv, ql)
        emu = emulate(kh, vh, name, kv_heads, bs, head_size, table[i], kv, qi, ql, q_heads, pick)
        assert np.abs(sub.reshape(len(pick), q_heads, head_size) - emu).max() < 4e-3, (i, kv, ql)
    assert np.all(got[~used] == 555.0)


EXACT_CASES = [  # name, kv_heads, q_heads, head_size, bs, kv_len, q_tokens
    ("BFloat16", 2, 8, 128, 16, 1000, 1000),
    ("Float16", 2, 8, 128, 16, 700, 37),
    ("BFloat16", 1, 8, 128, 32, 333, 333),
    ("Float16", 2, 4, 64, 16, 600, 600),
    ("BFloat16", 2, 6, 128, 16, 500, 500),      # group 6 (two idle rows of 128)
    ("BFloat16", 2, 32, 128, 16, 260, 260),     # group 16: 8 tokens per workgroup
    ("Float16", 1, 12, 64, 64, 333, 333),       # group 12 (eight idle rows)
    ("BFloat16", 1, 200, 64, 16, 50, 20),       # group 200 as 2 x 100 passes
    ("BFloat16", 1, 4, 64, 1, 3000, 300),       # one-token pages
    ("BFloat16", 2, 8, 128, 128, 1000, 1000),   # pages longer than a tile
    ("BFloat16", 8, 32, 128, 16, 8192, 64),     # chunked prefill: keys split over workgroups
    ("Float16", 1, 4, 128, 16, 40000, 16),      # page-list windows, split keys
]


@pytest.mark.parametrize("name,kv_heads,q_heads,head_size,bs,kv_len,q_tokens", EXACT_CASES)
def test_prefill_exact_matches_reference(gpu, name, kv_heads, q_heads, head_size, bs, kv_len, q_tokens):
    """kvflux_paged_prefill_exact: Q and the weights in three 16-bit parts,
    FP32 row sums; the reference's 1e-5 bound against the oracle (whole
    output), with and without key splits, bit-identical on repeat; head_size
    256 is declined."""
    blocks = (kv_len + bs - 1) // bs + 17
    seed = kv_len + 5 * q_tokens
    kc, vc, table = setup_case(name, blocks, kv_heads, bs, head_size, kv_len, seed)
    q = oracle.random_elements(0, q_tokens * q_heads * head_size, oracle.F32, 1, seed)
    lib = capi.lib()
    ws = C.c_size_t(0)
    capi.check(lib.kvflux_paged_prefill_workspace_size(kv_heads, head_size, kv_len, q_tokens, q_heads, C.byref(ws)))
    td, qd = buffer_like(table), buffer_like(q)
    wd = device.DeviceBuffer(max(ws.value, 256))
    outs = []
    for workspace in (True, False, True):
        od = buffer_like(np.full(q.size + 4, 777.0, np.float32))
        assert lib.kvflux_paged_prefill_exact(kc.ptr, vc.ptr, blocks, kv_heads, bs, head_size, CODES[name], td.ptr,
                                              len(table), kv_len, q_tokens, q_heads, qd.ptr, od.ptr,
                                              wd.ptr if workspace else None, ws.value if workspace else 0,
                                              None) == 0, capi.last_error()
        device.synchronize()
        out = od.download(np.float32)
        assert np.all(out[q.size:] == 777.0)
        outs.append(out[:q.size])
    assert np.array_equal(outs[0].view(np.uint32), outs[2].view(np.uint32))
    kh, vh = kc.download(np.uint16), vc.download(np.uint16)
    exp = oracle.paged_attention_causal(kh, vh, kv_heads, bs, head_size, CODES[name], table, kv_len, q, q_tokens,
                                        q_heads, threads=8)
    for got in outs[:2]:
        assert np.all(np.isfinite(got))
        assert np.abs(got - exp).max() < 1e-5
    assert lib.kvflux_paged_prefill_exact(kc.ptr, vc.ptr, blocks, kv_heads, bs, 256, CODES[name], td.ptr, len(table),
                                          kv_len, q_tokens, q_heads, qd.ptr, qd.ptr, None, 0,
                                          None) == capi.ERR_UNSUPPORTED


F32_CASES = [  # kv_heads, q_heads, head_size, bs, kv_len, q_tokens
    (2, 8, 128, 16, 1000, 1000),
    (2, 8, 128, 16, 700, 37),
    (1, 4, 64, 16, 600, 600),
    (2, 6, 128, 32, 500, 500),      # group 6 (two idle rows of 128)
    (2, 32, 128, 16, 260, 260),     # group 16: 8 tokens per workgroup
    (1, 12, 64, 64, 333, 333),      # group 12 (eight idle rows)
    (1, 136, 64, 16, 60, 17),       # group 136 as 2 x 68 passes
    (1, 4, 64, 1, 3000, 300),       # one-token pages
    (2, 8, 128, 128, 1000, 1000),   # pages longer than a tile
    (1, 2, 128, 2, 40, 40),         # two-token pages, one partial tile
    (8, 32, 128, 16, 8192, 64),     # chunked prefill: keys split over workgroups
    (1, 4, 128, 16, 40000, 16),     # page-list windows, split keys
]


def setup_f32(blocks, kv_heads, bs, head_size, kv_len, seed):
    page = kv_heads * bs * head_size
    kc = device.DeviceBuffer(blocks * page * 4)
    vc = device.DeviceBuffer(blocks * page * 4)
    device.fill_random(kc.ptr, blocks * page, oracle.F32, 1, seed * 3 + 1)
    device.fill_random(vc.ptr, blocks * page, oracle.F32, 1, seed * 3 + 2)
    npages = (kv_len + bs - 1) // bs
    table = np.random.default_rng(seed).permutation(blocks)[:npages].astype(np.uint64)
    return kc, vc, table


@pytest.mark.parametrize("kv_heads,q_heads,head_size,bs,kv_len,q_tokens", F32_CASES)
def test_prefill_f32_matches_reference(gpu, kv_heads, q_heads, head_size, bs, kv_len, q_tokens):
    """FP32 caches on the MFMA prefill (FP32 MFMAs on Q, K, V and the weights
    as they are, FP32 row sums): the whole output within the reference's 1e-5
    of the oracle through all three single-sequence entry points, with and
    without key splits; the split and exact entries give the same bits."""
    blocks = (kv_len + bs - 1) // bs + 17
    seed = kv_len + 7 * q_tokens
    kc, vc, table = setup_f32(blocks, kv_heads, bs, head_size, kv_len, seed)
    q = oracle.random_elements(0, q_tokens * q_heads * head_size, oracle.F32, 1, seed)
    lib = capi.lib()
    ws = C.c_size_t(0)
    capi.check(lib.kvflux_paged_prefill_workspace_size(kv_heads, head_size, kv_len, q_tokens, q_heads, C.byref(ws)))
    td, qd = buffer_like(table), buffer_like(q)
    wd = device.DeviceBuffer(max(ws.value, 256))
    outs = {}
    for entry in ("plain", "split", "exact"):
        od = buffer_like(np.full(q.size + 4, 777.0, np.float32))
        if entry == "plain":
            st = lib.kvflux_paged_prefill(kc.ptr, vc.ptr, blocks, kv_heads, bs, head_size, capi.DTYPE_F32, td.ptr,
                                          len(table), kv_len, q_tokens, q_heads, qd.ptr, od.ptr, None)
        else:
            fn = lib.kvflux_paged_prefill_split if entry == "split" else lib.kvflux_paged_prefill_exact
            st = fn(kc.ptr, vc.ptr, blocks, kv_heads, bs, head_size, capi.DTYPE_F32, td.ptr, len(table), kv_len,
                    q_tokens, q_heads, qd.ptr, od.ptr, wd.ptr, ws.value, None)
        assert st == 0, (entry, capi.last_error())
        device.synchronize()
        out = od.download(np.float32)
        assert np.all(out[q.size:] == 777.0), entry
        outs[entry] = out[:q.size]
    assert np.array_equal(outs["split"].view(np.uint32), outs["exact"].view(np.uint32))
    kh, vh = kc.download(np.float32), vc.download(np.float32)
    exp = oracle.paged_attention_causal(kh, vh, kv_heads, bs, head_size, oracle.F32, table, kv_len, q, q_tokens,
                                        q_heads, threads=8)
    for entry, got in outs.items():
        assert np.all(np.isfinite(got)), entry
        assert np.abs(got - exp).max() < 1e-5, entry


def test_prefill_f32_batch_and_cpp_routing(gpu, v2):
    """kvflux_paged_prefill_batch on an FP32 cache gives each sequence the
    bits of its own kvflux_paged_prefill call; the C++ paged_attention (the
    reference's signature, and Auto) sends a 16-token FP32 call to the MFMA
    prefill (the same bits as the C ABI call with a workspace) and a 15-token
    one to the split-K kernel, both within 1e-5 of the oracle."""
    lib = capi.lib()
    kv_heads, q_heads, head_size, bs = 2, 8, 128, 16
    seqs = [(700, 700), (1500, 64), (33, 33)]
    n = len(seqs)
    width = max((kv + bs - 1) // bs for kv, _ in seqs) + 2
    blocks = n * width + 3
    kc, vc, _ = setup_f32(blocks, kv_heads, bs, head_size, 1, 61)
    order = np.random.default_rng(62).permutation(blocks).astype(np.uint64)
    table = np.full((n, width), 2**64 - 1, np.uint64)
    for i, (kv, _) in enumerate(seqs):
        npg = (kv + bs - 1) // bs
        table[i, :npg] = order[i * width:i * width + npg]
    q_lens = np.array([ql for _, ql in seqs], np.uint64)
    kv_lens = np.array([kv for kv, _ in seqs], np.uint64)
    offsets = np.concatenate([[0], np.cumsum(q_lens + 1)[:-1]]).astype(np.uint64)
    rows_total = int(offsets[-1] + q_lens[-1] + 1)
    row = q_heads * head_size
    q = oracle.random_elements(0, rows_total * row, oracle.F32, 1, 63)
    td, qd = buffer_like(table.reshape(-1)), buffer_like(q)
    kd, ld, od_ = buffer_like(kv_lens), buffer_like(q_lens), buffer_like(offsets)
    out = buffer_like(np.full(rows_total * row, 555.0, np.float32))
    assert lib.kvflux_paged_prefill_batch(kc.ptr, vc.ptr, blocks, kv_heads, bs, head_size, capi.DTYPE_F32, td.ptr,
                                          width, kd.ptr, ld.ptr, od_.ptr, n, int(q_lens.max()), int(kv_lens.max()),
                                          q_heads, qd.ptr, out.ptr, None) == 0, capi.last_error()
    device.synchronize()
    got = out.download(np.float32).reshape(rows_total, row)
    kh, vh = kc.download(np.float32), vc.download(np.float32)
    used = np.zeros(rows_total, bool)
    for i, (kv, ql) in enumerate(seqs):
        o0 = int(offsets[i])
        used[o0:o0 + ql] = True
        qi = q.reshape(rows_total, row)[o0:o0 + ql].reshape(-1)
        sd, so = buffer_like(table[i]), buffer_like(np.zeros(qi.size, np.float32))
        qs = buffer_like(qi)
        assert lib.kvflux_paged_prefill(kc.ptr, vc.ptr, blocks, kv_heads, bs, head_size, capi.DTYPE_F32, sd.ptr,
                                        width, kv, ql, q_heads, qs.ptr, so.ptr, None) == 0, capi.last_error()
        device.synchronize()
        assert np.array_equal(got[o0:o0 + ql].reshape(-1).view(np.uint32), so.download(np.float32).view(np.uint32))
        exp = oracle.paged_attention_causal(kh, vh, kv_heads, bs, head_size, oracle.F32, table[i], kv, qi, ql,
                                            q_heads, threads=8)
        assert np.abs(got[o0:o0 + ql].reshape(-1) - exp).max() < 1e-5, i
    assert np.all(got[~used] == 555.0)

    pool = v2.PhysicalBlockPool(64, 16)
    storage = v2.PagedKVStorage(pool, 2, 128, v2.DType.Float32)
    seq = v2.SequenceState(1, pool)
    seq.append_tokens(300)
    count = storage.layout().cache_bytes() // 4
    device.fill_random(storage.key_base(), count, oracle.F32, 1, 64)
    device.fill_random(storage.value_base(), count, oracle.F32, 1, 65)
    kh = device.memcpy_d2h(storage.key_base(), storage.layout().cache_bytes(), np.float32)
    vh = device.memcpy_d2h(storage.value_base(), storage.layout().cache_bytes(), np.float32)
    rtable = np.array(v2.build_read_block_table(seq), np.uint64)
    P = v2.AttentionPrecision
    for q_tokens in (15, 16):
        q = oracle.random_elements(0, q_tokens * 8 * 128, oracle.F32, 1, 66 + q_tokens)
        qd = buffer_like(q)
        res = {}
        for prec in (None, P.Auto, P.Fast):
            od = buffer_like(np.zeros(q.size, np.float32))
            if prec is None:
                v2.paged_attention(storage, seq, qd.ptr, od.ptr, q_tokens, 8)
            else:
                v2.paged_attention(storage, seq, qd.ptr, od.ptr, q_tokens, 8, prec)
            res[prec] = od.download(np.float32)
        assert np.array_equal(res[None].view(np.uint32), res[P.Auto].view(np.uint32)), q_tokens
        exp = oracle.paged_attention_causal(kh, vh, 2, 16, 128, oracle.F32, rtable, 300, q, q_tokens, 8)
        assert np.abs(res[None] - exp).max() < 1e-5, q_tokens
        assert np.abs(res[P.Fast] - exp).max() < 1e-5, q_tokens
        ws = C.c_size_t(0)
        capi.check(lib.kvflux_paged_prefill_workspace_size(2, 128, 300, q_tokens, 8, C.byref(ws)))
        wd = device.DeviceBuffer(max(ws.value, 256))
        td, od = buffer_like(rtable), buffer_like(np.zeros(q.size, np.float32))
        assert lib.kvflux_paged_prefill_exact(storage.key_base(), storage.value_base(), 64, 2, 16, 128,
                                              capi.DTYPE_F32, td.ptr, len(rtable), 300, q_tokens, 8, qd.ptr, od.ptr,
                                              wd.ptr, ws.value, None) == 0
        device.synchronize()
        same = np.array_equal(od.download(np.float32).view(np.uint32), res[None].view(np.uint32))
        assert same == (q_tokens >= 16), q_tokens


@pytest.mark.parametrize("name", ["BFloat16", "Float32"])
def test_exact_prefill_workspace_for_awkward_group(gpu, name):
    """kvflux_paged_prefill_workspace_size serves the exact and FP32-cache
    variants too. With 131 query heads on one kv head (a group whose largest
    divisor up to 128 is 1), 64 query tokens and 32768 keys, the exact
    kernels hold fewer rows per workgroup than the rounded one and plan more
    key splits; a workspace of exactly the reported size must be enough, and
    sampled rows stay within 1e-5 of the oracle."""
    kv_heads, q_heads, head_size, bs, kv, ql = 1, 131, 64, 16, 32768, 64
    blocks = kv // bs + 3
    code = {"BFloat16": oracle.BF16, "Float32": oracle.F32}[name]
    abi = {"BFloat16": capi.DTYPE_BF16, "Float32": capi.DTYPE_F32}[name]
    elems = blocks * kv_heads * bs * head_size
    kc = device.DeviceBuffer(elems * (4 if name == "Float32" else 2))
    vc = device.DeviceBuffer(elems * (4 if name == "Float32" else 2))
    device.fill_random(kc.ptr, elems, abi, 1, 77)
    device.fill_random(vc.ptr, elems, abi, 1, 78)
    table = np.random.default_rng(78).permutation(blocks)[:kv // bs].astype(np.uint64)
    q = oracle.random_elements(0, ql * q_heads * head_size, oracle.F32, 1, 79)
    ws = C.c_size_t(0)
    capi.call("kvflux_paged_prefill_workspace_size", kv_heads, head_size, kv, ql, q_heads, C.byref(ws))
    assert ws.value > 0
    wd = device.DeviceBuffer(ws.value)
    td, qd = buffer_like(table), buffer_like(q)
    out = buffer_like(np.zeros(q.size, np.float32))
    assert capi.lib().kvflux_paged_prefill_exact(kc.ptr, vc.ptr, blocks, kv_heads, bs, head_size, abi, td.ptr,
                                                 len(table), kv, ql, q_heads, qd.ptr, out.ptr, wd.ptr, ws.value,
                                                 None) == 0, capi.last_error()
    device.synchronize()
    got = out.download(np.float32).reshape(ql, q_heads * head_size)
    kh = kc.download(np.float32 if name == "Float32" else np.uint16)
    vh = vc.download(np.float32 if name == "Float32" else np.uint16)
    pick = [0, 31, 63]
    exp = oracle.paged_attention_rows(kh, vh, kv_heads, bs, head_size, code, np.tile(table, len(pick)),
                                      len(table), np.array([kv - ql + t + 1 for t in pick], np.uint64),
                                      q.reshape(ql, -1)[pick].reshape(-1), q_heads, threads=8)
    assert np.abs(got[pick].reshape(-1) - exp).max() < 1e-5
