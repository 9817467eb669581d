"""Helpers shared by the GPU tests: device buffers via the C ABI and
conversions between numpy arrays and the cache dtypes."""
from __future__ import annotations

import numpy as np

from kvflux_amd import device
from oracle import oracle

DTYPES = {  # v2.DType name -> (oracle dtype code, numpy storage type)
    "Float16": (oracle.F16, np.uint16),
    "BFloat16": (oracle.BF16, np.uint16),
    "Float32": (oracle.F32, np.float32),
}


def encode(values: np.ndarray, name: str) -> np.ndarray:
    """FP32 values -> storage bits of `name` (round to nearest even)."""
    values = np.asarray(values, np.float32)
    if name == "Float32":
        return values.copy()
    if name == "Float16":
        return values.astype(np.float16).view(np.uint16)
    lib = oracle.lib()
    return np.array([lib.oracle_f32_to_bf16(float(x)) for x in values], np.uint16)


def decode(bits: np.ndarray, name: str) -> np.ndarray:
    return oracle.decode(bits, DTYPES[name][0])


def raw(values: np.ndarray, name: str) -> np.ndarray:
    """Integer patterns (as the reference's raw-bit tests use) in storage type."""
    if name == "Float32":
        return np.asarray(values, np.uint32).view(np.float32)
    return np.asarray(values, np.uint16)


def buffer_like(array: np.ndarray, extra_elements: int = 0, fill: int | None = None):
    buf = device.DeviceBuffer(array.nbytes + extra_elements * array.itemsize)
    if fill is not None:
        buf.fill(fill)
    buf.upload(array)
    return buf


def read_cache(storage, name: str) -> tuple[np.ndarray, np.ndarray]:
    """Downloads the whole K and V arena of a (small) storage."""
    layout = storage.layout()
    dt = DTYPES[name][1]
    k = device.memcpy_d2h(storage.key_base(), layout.cache_bytes(), dt)
    v = device.memcpy_d2h(storage.value_base(), layout.cache_bytes(), dt)
    return k, v


def fill_cache(storage, byte: int) -> None:
    layout = storage.layout()
    from kvflux_amd import capi
    import ctypes as C
    capi.call("kvflux_fill_bytes", C.c_void_p(storage.key_base()), byte, layout.total_bytes(),
              C.c_void_p(0))
    device.synchronize()
