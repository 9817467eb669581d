"""Control-plane parity with the reference on recorded op traces.

tests/golden/trace_golden.npz holds seeded op sequences and the results the
reference's own CPU library produced for them (tests/golden/gen_golden.py):
page ids, slot numbers, read and batch tables, reference counts, prefix
sharing and the exception class of every failing op. The same ops replayed
on this repository's implementation must produce the same results.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import trace_ops

GOLDEN = Path(__file__).resolve().parent / "golden" / "trace_golden.npz"


def _cases():
    data = np.load(GOLDEN, allow_pickle=False)
    seeds = sorted({k.split("/")[0] for k in data.files})
    return [(s, data) for s in seeds]


@pytest.mark.parametrize("seed", [s for s, _ in _cases()])
def test_trace_matches_reference(v2, seed):
    data = np.load(GOLDEN, allow_pickle=False)
    capacity, block_size = (int(x) for x in data[f"{seed}/config"])
    expected = data[f"{seed}/results"]
    actual = trace_ops.replay(v2, capacity, block_size, data[f"{seed}/ops"])
    assert len(actual) == len(expected)
    mismatch = np.nonzero(actual != expected)[0]
    assert mismatch.size == 0, f"first mismatch at result {mismatch[:1]}"
    # The traces exercise failures too, not only the happy path.
    assert (expected == -4).any() or (expected == -1).any()
