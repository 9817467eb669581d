"""ctypes wrapper of the CPU oracle (liboracle.so) and of the reference's own
CPU library (oracle/_ref/libkvflux_ref.so, present only where it was built).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's CPU-baseline leg, as the checker. The product never imports it.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libkvflux_ref.so"

F16, BF16, F32 = 0, 1, 2
OK, INVALID, RANGE, OVERFLOW = 0, 1, 2, 3

_vp, _sz, _u64, _i32 = C.c_void_p, C.c_size_t, C.c_uint64, C.c_int
_lib = None
_ref = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        h = C.CDLL(str(LIB_PATH))
        h.oracle_bf16_to_f32.restype = C.c_float
        h.oracle_bf16_to_f32.argtypes = [C.c_uint16]
        h.oracle_f16_to_f32.restype = C.c_float
        h.oracle_f16_to_f32.argtypes = [C.c_uint16]
        h.oracle_f32_to_bf16.restype = C.c_uint16
        h.oracle_f32_to_bf16.argtypes = [C.c_float]
        h.oracle_f32_to_f16.restype = C.c_uint16
        h.oracle_f32_to_f16.argtypes = [C.c_float]
        h.oracle_random_value.restype = C.c_float
        h.oracle_random_value.argtypes = [_u64, _u64, _i32]
        h.oracle_fill_random.restype = None
        h.oracle_fill_random.argtypes = [_vp, _u64, _u64, _i32, _i32, _u64]
        h.oracle_write_paged_kv.restype = None
        h.oracle_write_paged_kv.argtypes = [_vp, _vp, _sz, _sz, _sz, _i32, _vp, _vp, _vp, _sz]
        h.oracle_gather_paged_kv.restype = None
        h.oracle_gather_paged_kv.argtypes = [_vp, _vp, _sz, _sz, _sz, _i32, _vp, _sz, _vp, _vp]
        h.oracle_reference_attention.restype = _i32
        h.oracle_reference_attention.argtypes = [_vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _vp]
        h.oracle_paged_attention_rows.restype = _i32
        h.oracle_paged_attention_rows.argtypes = [_vp, _vp, _sz, _sz, _sz, _i32, _vp, _sz, _vp,
                                                  _sz, _sz, _vp, _vp, _i32]
        h.oracle_paged_attention_causal.restype = _i32
        h.oracle_paged_attention_causal.argtypes = [_vp, _vp, _sz, _sz, _sz, _i32, _vp, _sz, _sz,
                                                    _sz, _vp, _vp, _i32]
        _lib = h
    return _lib


def ref_available() -> bool:
    return REF_PATH.exists()


def ref() -> C.CDLL:
    global _ref
    if _ref is None:
        h = C.CDLL(str(REF_PATH))
        h.ref_reference_attention.restype = _i32
        h.ref_reference_attention.argtypes = [_vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _sz, _sz,
                                              _sz, _vp]
        h.ref_run_trace.restype = C.c_long
        h.ref_run_trace.argtypes = [_sz, _sz, _vp, _sz, _vp, _sz]
        _ref = h
    return _ref


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


# ------------------------------------------------------------- conversions
def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def decode(bits: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == F32:
        return np.asarray(bits).view(np.float32)
    return bf16_to_f32(bits) if dtype == BF16 else f16_to_f32(bits)


def encode(values: np.ndarray, dtype: int) -> np.ndarray:
    """FP32 values -> storage bits of `dtype`, rounding to nearest even (the
    vectorised form of oracle_f32_to_bf16 / oracle_f32_to_f16)."""
    values = np.asarray(values, dtype=np.float32)
    if dtype == F32:
        return values.copy()
    if dtype == F16:
        return values.astype(np.float16).view(np.uint16)
    u = values.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(values)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)


def np_dtype(dtype: int):
    return np.float32 if dtype == F32 else np.uint16


def random_elements(first: int, count: int, dtype: int, distribution: int, seed: int) -> np.ndarray:
    out = np.empty(count, dtype=np_dtype(dtype))
    lib().oracle_fill_random(_p(out), first, count, dtype, distribution, seed & (2**64 - 1))
    return out


# ------------------------------------------------------------- data path
def write_paged_kv(key_cache, value_cache, heads, block_size, head_size, dtype, key_new,
                   value_new, slots) -> None:
    slots = np.ascontiguousarray(slots, dtype=np.uint64)
    lib().oracle_write_paged_kv(_p(key_cache), _p(value_cache), heads, block_size, head_size,
                                dtype, _p(key_new), _p(value_new), _p(slots), len(slots))


def gather_paged_kv(key_cache, value_cache, heads, block_size, head_size, dtype, table, tokens):
    table = np.ascontiguousarray(table, dtype=np.uint64)
    n = tokens * heads * head_size
    k = np.empty(n, dtype=np_dtype(dtype))
    v = np.empty(n, dtype=np_dtype(dtype))
    lib().oracle_gather_paged_kv(_p(key_cache), _p(value_cache), heads, block_size, head_size,
                                 dtype, _p(table), tokens, _p(k), _p(v))
    return k, v


def reference_attention(q, k, v, q_tokens, kv_tokens, q_heads, kv_heads, head_size) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    n = q_tokens * q_heads * head_size
    # An overflowing shape is rejected by the C code before it writes.
    out = np.empty(max(n, 1) if n < 2**40 else 1, dtype=np.float32)
    status = lib().oracle_reference_attention(_p(q), _p(k), _p(v), q_tokens, kv_tokens, q_heads,
                                              kv_heads, head_size, _p(out))
    if status == INVALID:
        raise ValueError("invalid reference attention input")
    if status == OVERFLOW:
        raise OverflowError("reference attention size overflow")
    return out[: q_tokens * q_heads * head_size]


def paged_attention_rows(key_cache, value_cache, kv_heads, block_size, head_size, dtype, tables,
                         table_stride, lens, q, q_heads, threads=1) -> np.ndarray:
    tables = np.ascontiguousarray(tables, dtype=np.uint64)
    lens = np.ascontiguousarray(lens, dtype=np.uint64)
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.zeros(len(lens) * q_heads * head_size, dtype=np.float32)
    status = lib().oracle_paged_attention_rows(_p(key_cache), _p(value_cache), kv_heads,
                                               block_size, head_size, dtype, _p(tables),
                                               table_stride, _p(lens), len(lens), q_heads, _p(q),
                                               _p(out), threads)
    if status != OK:
        raise RuntimeError(f"oracle paged attention failed ({status})")
    return out


def paged_attention_causal(key_cache, value_cache, kv_heads, block_size, head_size, dtype, table,
                           kv_len, q, q_tokens, q_heads, threads=1) -> np.ndarray:
    table = np.ascontiguousarray(table, dtype=np.uint64)
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.zeros(q_tokens * q_heads * head_size, dtype=np.float32)
    status = lib().oracle_paged_attention_causal(_p(key_cache), _p(value_cache), kv_heads,
                                                 block_size, head_size, dtype, _p(table), kv_len,
                                                 q_tokens, q_heads, _p(q), _p(out), threads)
    if status != OK:
        raise RuntimeError(f"oracle causal attention failed ({status})")
    return out


# ------------------------------------------------------------- reference lib
def ref_reference_attention(q, k, v, q_tokens, kv_tokens, q_heads, kv_heads, head_size):
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty(max(q_tokens * q_heads * head_size, 1), dtype=np.float32)
    status = ref().ref_reference_attention(_p(q), q.size, _p(k), k.size, _p(v), v.size, q_tokens,
                                           kv_tokens, q_heads, kv_heads, head_size, _p(out))
    return status, out[: q_tokens * q_heads * head_size]


def ref_run_trace(capacity: int, block_size: int, ops: np.ndarray, out_cap: int = 1 << 20):
    ops = np.ascontiguousarray(ops, dtype=np.int64)
    out = np.empty(out_cap, dtype=np.int64)
    n = ref().ref_run_trace(capacity, block_size, _p(ops), len(ops) // 3, _p(out), out_cap)
    if n < 0:
        raise RuntimeError("trace output overflow")
    return out[:n]
