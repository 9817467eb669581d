"""Writes the golden fixtures of tests/golden/ from the reference's own CPU
library (oracle/_ref/libkvflux_ref.so, built by `make -C oracle ref` from the
reference sources). Run in the build container, where the reference checkout
exists:

    make -C oracle ref && python tests/golden/gen_golden.py

Fixtures (numpy .npz, no pickles):
  attention_golden.npz   reference_attention outputs for seeded inputs:
                         the 40-token FP32 correctness case (H=2, Hq=4,
                         D=64, uniform[-1,1]) at Tq = 1, 7, 40, and
                         BF16/FP16-decoded K/V cases (GQA 4 and 1).
  trace_golden.npz       control-plane op traces and the reference's
                         results (page ids, slots, tables, errors).
Inputs are stored next to the outputs, so the fixtures do not depend on the
generator staying the same.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

from oracle import oracle  # noqa: E402
import trace_ops  # noqa: E402

OUT = Path(__file__).resolve().parent

# (name, kv_tokens, kv_heads, q_heads, head_size, kv dtype, distribution, seed, q_tokens list)
ATTENTION_CASES = [
    ("cfg1_fp32", 40, 2, 4, 64, oracle.F32, 0, 1, (1, 7, 40)),
    ("bf16_gqa4", 300, 2, 8, 128, oracle.BF16, 1, 2, (1, 5)),
    ("f16_mha", 100, 4, 4, 64, oracle.F16, 1, 3, (1, 3)),
    ("bf16_d32_g2", 77, 3, 6, 32, oracle.BF16, 0, 4, (1, 77)),
]

TRACE_CASES = [  # (seed, capacity, block_size, steps)
    (11, 16, 4, 400),
    (12, 64, 16, 600),
    (13, 8, 2, 300),
    (14, 200, 16, 800),
]
# Prefix-sharing churn (trace_ops.churn_trace): small pools, long traces, so
# idle published pages are held, released and evicted thousands of times.
CHURN_CASES = [  # (seed, capacity, block_size, steps)
    (21, 6, 2, 4000),
    (22, 12, 4, 6000),
    (23, 24, 1, 6000),
]


def attention_fixture() -> dict:
    data = {}
    for name, kv_tokens, kv_heads, q_heads, head_size, dtype, dist, seed, q_list in ATTENTION_CASES:
        n_kv = kv_tokens * kv_heads * head_size
        k_bits = oracle.random_elements(0, n_kv, dtype, dist, seed * 1000 + 1)
        v_bits = oracle.random_elements(0, n_kv, dtype, dist, seed * 1000 + 2)
        k = oracle.decode(k_bits, dtype).astype(np.float32)
        v = oracle.decode(v_bits, dtype).astype(np.float32)
        data[f"{name}/shape"] = np.array([kv_tokens, kv_heads, q_heads, head_size, dtype], np.int64)
        data[f"{name}/k_bits"] = k_bits
        data[f"{name}/v_bits"] = v_bits
        for q_tokens in q_list:
            q = oracle.random_elements(0, q_tokens * q_heads * head_size, oracle.F32, dist,
                                       seed * 1000 + 3 + q_tokens)
            status, out = oracle.ref_reference_attention(q, k, v, q_tokens, kv_tokens, q_heads,
                                                         kv_heads, head_size)
            assert status == 0, (name, q_tokens, status)
            data[f"{name}/q{q_tokens}"] = q
            data[f"{name}/o{q_tokens}"] = out
    return data


def trace_fixture() -> dict:
    data = {}
    for seed, capacity, block_size, steps in TRACE_CASES:
        ops = trace_ops.random_trace(seed, capacity, block_size, steps)
        results = oracle.ref_run_trace(capacity, block_size, ops)
        data[f"t{seed}/config"] = np.array([capacity, block_size], np.int64)
        data[f"t{seed}/ops"] = ops
        data[f"t{seed}/results"] = results
    for seed, capacity, block_size, steps in CHURN_CASES:
        ops = trace_ops.churn_trace(seed, capacity, block_size, steps)
        results = oracle.ref_run_trace(capacity, block_size, ops)
        data[f"c{seed}/config"] = np.array([capacity, block_size], np.int64)
        data[f"c{seed}/ops"] = ops
        data[f"c{seed}/results"] = results
    return data


def main() -> None:
    if not oracle.ref_available():
        raise SystemExit("oracle/_ref/libkvflux_ref.so missing: run `make -C oracle ref`")
    np.savez_compressed(OUT / "attention_golden.npz", **attention_fixture())
    np.savez_compressed(OUT / "trace_golden.npz", **trace_fixture())
    for f in ("attention_golden.npz", "trace_golden.npz"):
        print(f, (OUT / f).stat().st_size, "bytes")


if __name__ == "__main__":
    main()
