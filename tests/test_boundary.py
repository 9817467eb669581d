"""The drop-in boundary, checked on the CPU (no GPU calls):

* every entry point declared in include/kvflux_hip.h is exported by the
  built libkvflux_hip.so and has a ctypes signature in kvflux_amd/capi.py;
* the product (package sources, host C++ layer, HIP kernels, built
  libraries) neither imports nor links the oracle;
* kvflux::v2::reference_attention (the API's host reference function) is
  bit-identical to the oracle and to the compiled reference on random inputs,
  and the reference's own CPU tests pass against this repository's headers
  and libkvflux.so (built from /root/reference where that checkout exists).
"""
from __future__ import annotations

import ctypes as C
import os
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from kvflux_amd import capi
from oracle import oracle

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "kvflux_hip.h"
REFERENCE = Path("/root/reference")


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(kvflux_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_entry_point_is_exported():
    names = declared_functions()
    assert "kvflux_write_paged_kv" in names and "kvflux_paged_prefill" in names
    lib = C.CDLL(str(capi.LIB_PATH))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(capi.EXPORTS) == names  # the Python binding covers exactly the header


def test_product_does_not_use_the_oracle():
    product = [p for p in (ROOT / "kvflux_amd").rglob("*")
               if p.suffix in {".py", ".cpp", ".h", ".hip"} and "_build" not in p.parts]
    product += list((ROOT / "include").rglob("*.h"))
    for path in product:
        text = path.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle\b", text, re.M), path
        assert "liboracle" not in text and "oracle/" not in text, path
    for lib in (ROOT / "kvflux_amd" / "lib").glob("*.so"):
        needed = subprocess.run(["readelf", "-d", str(lib)], capture_output=True, text=True).stdout
        assert "oracle" not in needed and "kvflux_ref" not in needed, lib


def _random_case(rng):
    kv_heads = int(rng.integers(1, 4))
    q_heads = kv_heads * int(rng.choice([1, 2, 4]))
    head_size = int(rng.choice([1, 4, 16, 64]))
    kv_tokens = int(rng.integers(1, 60))
    q_tokens = int(rng.integers(0, kv_tokens + 1))
    q = rng.standard_normal(q_tokens * q_heads * head_size).astype(np.float32)
    k = rng.standard_normal(kv_tokens * kv_heads * head_size).astype(np.float32)
    v = rng.standard_normal(kv_tokens * kv_heads * head_size).astype(np.float32)
    return q, k, v, (q_tokens, kv_tokens, q_heads, kv_heads, head_size)


@pytest.mark.parametrize("seed", range(5))
def test_api_reference_attention_bit_exact(v2, seed):
    q, k, v, shape = _random_case(np.random.default_rng(100 + seed))
    ours = np.array(v2.reference_attention(q.tolist(), k.tolist(), v.tolist(), v2.AttentionShape(*shape)),
                    np.float32)
    expected = oracle.reference_attention(q, k, v, *shape)
    assert np.array_equal(ours.view(np.uint32), expected.view(np.uint32))
    if oracle.ref_available():
        status, theirs = oracle.ref_reference_attention(q, k, v, *shape)
        assert status == 0
        assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))


def test_api_reference_attention_errors(v2):
    with pytest.raises(ValueError):
        v2.reference_attention([1.0], [1.0], [1.0], v2.AttentionShape(2, 1, 1, 1, 1))
    with pytest.raises(ValueError):
        v2.reference_attention([float("nan")], [1.0], [1.0], v2.AttentionShape(1, 1, 1, 1, 1))
    with pytest.raises(OverflowError):
        v2.reference_attention([], [], [], v2.AttentionShape(1, 1, 2**64 - 1, 1, 2))
    assert v2.reference_attention([], [], [], v2.AttentionShape(0, 0, 1, 1, 1)) == []


@pytest.mark.skipif(not (REFERENCE / "tests").is_dir(), reason="reference checkout not present")
def test_reference_cpu_tests_pass_against_this_api():
    build = subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "compat"], capture_output=True, text=True,
                           timeout=600)
    assert build.returncode == 0, build.stdout + build.stderr
    binaries = sorted((ROOT / "oracle" / "_ref" / "compat").iterdir())
    assert len(binaries) >= 13
    for exe in binaries:
        run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120,
                             env={**os.environ, "LD_LIBRARY_PATH": str(ROOT / "kvflux_amd" / "lib")})
        assert run.returncode == 0, (exe.name, run.stdout, run.stderr)
