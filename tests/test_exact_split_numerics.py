"""CPU emulation of the exact attention kernels' FP16 weight path.

The exact kernels (prefill.hip PfF16Exact, attention.hip on FP16 caches) feed
the softmax weights to FP16 MFMAs as three FP16 parts and divide by an FP32
row sum. This emulates that path in numpy on a peaked row (one sink key,
32767 keys 25-26 log2 units below it) to show why the kernels scale the
weights by 2^15 before the split and keep a compensated row sum; the GPU
tests in test_gpu_exact_f16.py check the kernels themselves on such rows.
"""
from __future__ import annotations

import numpy as np


def split3_f16(x):
    """x as the sum of three FP16 parts, each the rounded remainder."""
    parts, r = [], x.astype(np.float32)
    for _ in range(3):
        h = r.astype(np.float16)
        parts.append(h.astype(np.float64))
        r = (r - h.astype(np.float32)).astype(np.float32)
    return parts[0] + parts[1] + parts[2]


def test_f16_weight_split_emulation():
    """CPU emulation of the exact kernels' weight path on the peaked row (one
    sink key with V = -1, 32767 keys 25-26 log2 units below with V ~ 1 +
    0.5 N(0,1), so their share of the row, about 7e-4, moves O): O = sum(w_i
    v_i) / l with the weights w_i entering as three FP16 parts and l their
    FP32 row sum. Splitting the raw weights (<= 1) loses the small ones
    (FP16 stops at 2^-24) and misses 1e-5; splitting 2^15 times the weights
    and dividing by 2^15 meets it, as long as l keeps the rounding error of
    each addition (a plain FP32 running sum of 1 + many 2^-25 terms drops
    them the same way every time)."""
    rng = np.random.default_rng(5)
    n = 32768
    logw = -rng.uniform(25.0, 26.0, n)
    logw[0] = 0.0
    w = np.exp2(logw).astype(np.float32)
    v = 1.0 + 0.5 * rng.standard_normal(n)
    v[0] = -1.0
    exact = (np.exp2(logw) * v).sum() / np.exp2(logw).sum()

    def fp32_sum(terms, compensated):
        hi, lo = np.float32(0), np.float32(0)
        for t in terms.astype(np.float32).reshape(-1, 8).sum(1, dtype=np.float32):  # 8 weights per step
            s = np.float32(hi + t)
            if compensated:
                bp = np.float32(s - hi)
                lo = np.float32(lo + np.float32(np.float32(hi - np.float32(s - bp)) + np.float32(t - bp)))
            hi = s
        return float(hi) + float(lo)

    l_comp = fp32_sum(w, True)
    unscaled = (split3_f16(w) * v).sum() / l_comp
    scaled = (split3_f16(w * np.float32(32768.0)) * v).sum() / 32768.0 / l_comp
    plain_sum = (split3_f16(w * np.float32(32768.0)) * v).sum() / 32768.0 / fp32_sum(w, False)
    assert abs(unscaled - exact) > 1e-5
    assert abs(plain_sum - exact) > 1e-5
    assert abs(scaled - exact) < 1e-6
