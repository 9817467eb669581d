"""Pins the CPU oracle before it is trusted as the GPU checker.

* reference_attention: the reference's closed-form known answers
  (tests/reference_attention_test.cpp:28-80), bit-exact agreement with the
  reference's own compiled function on the golden fixtures, and with the
  compiled reference on fresh random inputs where oracle/_ref is built;
  plus invariants a dropped term or swapped index would break.
* write/gather: against an independent numpy restatement of the layout.
* conversions and the counter-based generator: against numpy float16, an
  exact rational rounding of BF16, and distribution moments.
"""
from __future__ import annotations

import math
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle

GOLDEN = Path(__file__).resolve().parent / "golden" / "attention_golden.npz"


def attn(q, k, v, shape):
    q_tokens, kv_tokens, q_heads, kv_heads, head_size = shape
    return oracle.reference_attention(np.asarray(q, np.float32), np.asarray(k, np.float32),
                                      np.asarray(v, np.float32), q_tokens, kv_tokens, q_heads,
                                      kv_heads, head_size)


def test_reference_attention_known_answers():
    causal = attn([0, 0, 0], [0, 0, 0], [2, 4, 8], (3, 3, 1, 1, 1))
    assert np.allclose(causal, [2.0, 3.0, 14.0 / 3.0], atol=1e-6)
    decode = attn([2, 0, 0, 0], [0, 0, 0, 0, 1, 0, 0, 0], [0, 0, 0, 0, 10, 0, 0, 0], (1, 2, 1, 1, 4))
    assert abs(decode[0] - 10 * math.e / (1 + math.e)) < 1e-6 and abs(decode[1]) < 1e-6
    suffix = attn([0, 0], [0, 0, 0, 0], [1, 2, 3, 4], (2, 4, 1, 1, 1))
    assert np.allclose(suffix, [2.0, 2.5], atol=1e-6)
    grouped = attn([0, 0, 0, 0], [0, 0, 0, 0], [1, 10, 3, 30], (1, 2, 4, 2, 1))
    assert grouped.tolist() == [2, 2, 20, 20]
    stable = attn([1e20], [1e20, 1e20], [2, 4], (1, 2, 1, 1, 1))
    assert abs(stable[0] - 3.0) < 1e-6
    assert attn([], [], [], (0, 0, 1, 1, 1)).size == 0


def test_reference_attention_rejects_bad_inputs():
    with pytest.raises(ValueError):
        attn([1], [1], [1], (2, 1, 1, 1, 1))
    with pytest.raises(ValueError):
        attn([1], [1], [1], (1, 1, 1, 0, 1))
    with pytest.raises(ValueError):
        attn([float("nan")], [1], [1], (1, 1, 1, 1, 1))
    with pytest.raises(OverflowError):
        oracle.reference_attention(np.zeros(1, np.float32), np.zeros(1, np.float32),
                                   np.zeros(1, np.float32), 1, 1, 2**64 - 1, 1, 2)


def golden_cases():
    data = np.load(GOLDEN, allow_pickle=False)
    names = sorted({k.split("/")[0] for k in data.files})
    out = []
    for name in names:
        for key in data.files:
            if key.startswith(name + "/o"):
                out.append((name, int(key.split("/o")[1])))
    return out


@pytest.mark.parametrize("name,q_tokens", golden_cases())
def test_oracle_bit_exact_on_golden_vectors(name, q_tokens):
    data = np.load(GOLDEN, allow_pickle=False)
    kv_tokens, kv_heads, q_heads, head_size, dtype = (int(x) for x in data[f"{name}/shape"])
    k = oracle.decode(data[f"{name}/k_bits"], dtype)
    v = oracle.decode(data[f"{name}/v_bits"], dtype)
    out = oracle.reference_attention(data[f"{name}/q{q_tokens}"], k, v, q_tokens, kv_tokens,
                                     q_heads, kv_heads, head_size)
    expected = data[f"{name}/o{q_tokens}"]
    assert np.array_equal(out.view(np.uint32), expected.view(np.uint32))


@pytest.mark.skipif(not oracle.ref_available(), reason="reference CPU library not built here")
@pytest.mark.parametrize("seed", range(6))
def test_oracle_matches_compiled_reference_on_random_inputs(seed):
    rng = np.random.default_rng(seed)
    kv_heads = int(rng.integers(1, 4))
    q_heads = kv_heads * int(rng.choice([1, 2, 4]))
    head_size = int(rng.choice([1, 3, 4, 16, 64]))
    kv_tokens = int(rng.integers(1, 70))
    q_tokens = int(rng.integers(0, kv_tokens + 1))
    q = rng.standard_normal(q_tokens * q_heads * head_size).astype(np.float32)
    k = rng.standard_normal(kv_tokens * kv_heads * head_size).astype(np.float32)
    v = rng.standard_normal(kv_tokens * kv_heads * head_size).astype(np.float32)
    ours = oracle.reference_attention(q, k, v, q_tokens, kv_tokens, q_heads, kv_heads, head_size)
    status, theirs = oracle.ref_reference_attention(q, k, v, q_tokens, kv_tokens, q_heads,
                                                    kv_heads, head_size)
    assert status == 0
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))


def test_attention_invariants():
    rng = np.random.default_rng(7)
    T, H, G, D = 23, 2, 3, 8
    q = rng.standard_normal(T * H * G * D).astype(np.float32)
    k = rng.standard_normal(T * H * D).astype(np.float32)
    # identical V rows -> every output equals that row
    row = rng.standard_normal(D).astype(np.float32)
    v = np.tile(row, T * H)
    out = attn(q, k, v, (T, T, H * G, H, D)).reshape(T, H * G, D)
    assert np.allclose(out, row, atol=1e-6)
    # first query sees only token 0: output = v[0] of its kv head
    v = rng.standard_normal(T * H * D).astype(np.float32)
    out = attn(q, k, v, (T, T, H * G, H, D)).reshape(T, H * G, D)
    vv = v.reshape(T, H, D)
    for h in range(H * G):
        assert np.allclose(out[0, h], vv[0, h // G], atol=1e-6)
    # GQA == MHA with the kv heads repeated
    k_rep = np.repeat(k.reshape(T, H, D), G, axis=1).reshape(-1)
    v_rep = np.repeat(vv, G, axis=1).reshape(-1)
    mha = attn(q, k_rep, v_rep, (T, T, H * G, H * G, D))
    assert np.array_equal(mha, out.reshape(-1))
    # brute-force softmax in float64 for the last query
    qq = q.reshape(T, H * G, D)
    kk = k.reshape(T, H, D).astype(np.float64)
    for h in range(H * G):
        s = kk[:, h // G] @ qq[-1, h].astype(np.float64) / math.sqrt(D)
        p = np.exp(s - s.max())
        p /= p.sum()
        assert np.allclose(out[-1, h], p @ vv[:, h // G].astype(np.float64), atol=1e-6)


def numpy_scatter(kc, vc, H, bs, D, kn, vn, slots):
    kc = kc.reshape(-1, H, bs, D).copy()
    vc = vc.reshape(-1, H, bs, D).copy()
    kn = kn.reshape(-1, H, D)
    vn = vn.reshape(-1, H, D)
    for n, slot in enumerate(slots):
        kc[slot // bs, :, slot % bs, :] = kn[n]
        vc[slot // bs, :, slot % bs, :] = vn[n]
    return kc.reshape(-1), vc.reshape(-1)


@pytest.mark.parametrize("dtype", [oracle.F16, oracle.BF16, oracle.F32])
def test_write_and_gather_oracle_against_numpy_layout(dtype):
    rng = np.random.default_rng(dtype)
    blocks, H, bs, D = 12, 3, 4, 5
    npt = oracle.np_dtype(dtype)
    kc = rng.integers(0, 2**16, blocks * H * bs * D).astype(npt)
    vc = rng.integers(0, 2**16, blocks * H * bs * D).astype(npt)
    slots = rng.permutation(blocks * bs)[:17].astype(np.uint64)
    kn = rng.integers(0, 2**16, 17 * H * D).astype(npt)
    vn = rng.integers(0, 2**16, 17 * H * D).astype(npt)
    ek, ev = numpy_scatter(kc, vc, H, bs, D, kn, vn, slots)
    oracle.write_paged_kv(kc, vc, H, bs, D, dtype, kn, vn, slots)
    assert np.array_equal(kc, ek) and np.array_equal(vc, ev)
    table = rng.permutation(blocks)[:5].astype(np.uint64)
    tokens = 18
    gk, gv = oracle.gather_paged_kv(kc, vc, H, bs, D, dtype, table, tokens)
    kk = kc.reshape(blocks, H, bs, D)
    expect = np.stack([kk[table[t // bs], :, t % bs, :] for t in range(tokens)]).reshape(-1)
    assert np.array_equal(gk, expect)


def exact_bf16(x: np.float32) -> int:
    """Round-to-nearest-even of an FP32 value to BF16 using exact rationals."""
    f = Fraction(float(x))
    if f == 0:
        return int(np.float32(x).view(np.uint32)) >> 16
    sign = 0x8000 if f < 0 else 0
    a = abs(f)
    e = math.floor(math.log2(a))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    unit = Fraction(2) ** (e - 7)
    q = a / unit
    n = math.floor(q)
    rem = q - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    val = np.float32(float(n * unit))
    return sign | (int(val.view(np.uint32)) >> 16)


def test_bf16_and_f16_rounding():
    rng = np.random.default_rng(3)
    xs = np.concatenate([
        rng.standard_normal(3000).astype(np.float32),
        (rng.standard_normal(500) * 1e-6).astype(np.float32),
        np.array([1.00390625, 1.01171875, -2.0078125, 65504.0, 6.1e-5, 3e-8, 2.0**-25], np.float32),
    ])
    lib = oracle.lib()
    for x in xs:
        assert lib.oracle_f32_to_bf16(float(x)) == exact_bf16(x)
        assert lib.oracle_f32_to_f16(float(x)) == int(np.float16(x).view(np.uint16))
    # the vectorised encoder agrees with the scalar ones
    assert np.array_equal(oracle.encode(xs, oracle.BF16), [exact_bf16(x) for x in xs])
    assert np.array_equal(oracle.encode(xs, oracle.F16), [lib.oracle_f32_to_f16(float(x)) for x in xs])
    halves = np.arange(2**16, dtype=np.uint32).astype(np.uint16)
    finite = halves[~np.isnan(halves.view(np.float16))]
    for h in finite[::61]:
        assert lib.oracle_f16_to_f32(int(h)) == float(np.uint16(h).view(np.float16))


def test_counter_generator_properties():
    u = oracle.random_elements(0, 200000, oracle.F32, 0, 5)
    assert u.min() >= -1.0 and u.max() < 1.0 and abs(u.mean()) < 0.01
    assert np.all(np.mod(u.astype(np.float64) * 2**23, 1.0) == 0)  # 2^-23 grid
    n = oracle.random_elements(0, 200000, oracle.F32, 1, 6)
    assert abs(n.mean()) < 0.01 and abs(n.std() - 1.0) < 0.01 and np.abs(n).max() <= 6.0
    # element i depends only on (seed, i)
    part = oracle.random_elements(1234, 10, oracle.F32, 1, 6)
    assert np.array_equal(part, n[1234:1244])
    b = oracle.random_elements(0, 1000, oracle.BF16, 1, 6)
    assert np.array_equal(b, np.array([exact_bf16(x) for x in n[:1000]], np.uint16))


def _fragmented_case(dtype, kv_heads, block_size, head_size, pages, seed):
    """A cache of `pages` pages filled with random elements of `dtype`
    (NaN-free), and a seeded permutation to draw non-contiguous tables from."""
    rng = np.random.default_rng(seed)
    n = pages * kv_heads * block_size * head_size
    k = oracle.random_elements(0, n, dtype, 0, seed * 10 + 1)
    v = oracle.random_elements(0, n, dtype, 0, seed * 10 + 2)
    return k, v, rng.permutation(pages).astype(np.uint64), rng


PAGED_CASES = [  # dtype, kv_heads, q_heads, block_size, head_size
    (oracle.F32, 2, 4, 16, 64),
    (oracle.BF16, 2, 8, 3, 32),
    (oracle.F16, 1, 3, 1, 5),
    (oracle.BF16, 4, 4, 7, 16),
]


@pytest.mark.parametrize("dtype,kv_heads,q_heads,block_size,head_size", PAGED_CASES)
def test_paged_oracle_is_gather_then_reference_attention(dtype, kv_heads, q_heads, block_size, head_size):
    """The paged oracle functions the GPU parity tests check against,
    oracle_paged_attention_rows and oracle_paged_attention_causal, against
    the two-path composition of the reference's own attention test
    (tests/paged_attention_test.cu:86-110): gather each sequence's pages to
    contiguous K/V, then the pinned reference_attention. Fragmented random
    tables, tail pages of every fill, lengths 1 and a page multiple;
    bit-exact, on one thread and on four."""
    pages = 96
    k, v, order, rng = _fragmented_case(dtype, kv_heads, block_size, head_size, pages, head_size + block_size)
    width = pages // 4
    lens = np.array([1, block_size, block_size * 3 + 1, width * block_size, 37, 2 * block_size - 1], np.uint64)
    lens = np.minimum(lens, width * block_size)
    tables = np.stack([order[(7 * r) % (pages - width):][:width] for r in range(len(lens))])
    rows = len(lens)
    q = oracle.random_elements(0, rows * q_heads * head_size, oracle.F32, 0, 99 + head_size)
    expected = np.empty(rows * q_heads * head_size, np.float32)
    for r in range(rows):
        L = int(lens[r])
        kg, vg = oracle.gather_paged_kv(k, v, kv_heads, block_size, head_size, dtype, tables[r], L)
        qr = q[r * q_heads * head_size:(r + 1) * q_heads * head_size]
        expected[r * q_heads * head_size:(r + 1) * q_heads * head_size] = oracle.reference_attention(
            qr, oracle.decode(kg, dtype), oracle.decode(vg, dtype), 1, L, q_heads, kv_heads, head_size)
    for threads in (1, 4):
        got = oracle.paged_attention_rows(k, v, kv_heads, block_size, head_size, dtype, tables.reshape(-1), width,
                                          lens, q, q_heads, threads=threads)
        assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))
    # causal trailing queries of one sequence
    kv_len = int(width * block_size - block_size // 2)
    tq = min(9, kv_len)
    qc = oracle.random_elements(0, tq * q_heads * head_size, oracle.F32, 0, 7 + head_size)
    kg, vg = oracle.gather_paged_kv(k, v, kv_heads, block_size, head_size, dtype, tables[2], kv_len)
    exp_c = oracle.reference_attention(qc, oracle.decode(kg, dtype), oracle.decode(vg, dtype), tq, kv_len, q_heads,
                                       kv_heads, head_size)
    for threads in (1, 4):
        got_c = oracle.paged_attention_causal(k, v, kv_heads, block_size, head_size, dtype, tables[2], kv_len, qc, tq,
                                              q_heads, threads=threads)
        assert np.array_equal(got_c.view(np.uint32), exp_c.view(np.uint32))
    # a plausible indexing mistake (a row reading its neighbour's table) is caught
    wrong = oracle.paged_attention_rows(k, v, kv_heads, block_size, head_size, dtype, tables[::-1].reshape(-1), width,
                                        lens, q, q_heads)
    assert not np.array_equal(wrong.view(np.uint32), expected.view(np.uint32))
