"""ctypes view of the C ABI in include/kvflux_hip.h (libkvflux_hip.so).

Every function declared in the header is bound here with its exact
signature; `EXPORTS` lists them so tests can check the library exports the
whole boundary. Importing this module loads the library but makes no GPU
call.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "lib"
LIB_PATH = LIB_DIR / "libkvflux_hip.so"

OK, ERR_INVALID, ERR_RANGE, ERR_OVERFLOW, ERR_RUNTIME, ERR_UNSUPPORTED = range(6)
DTYPE_F16, DTYPE_BF16, DTYPE_F32 = 0, 1, 2
DIST_UNIFORM, DIST_NORMAL = 0, 1

_vp, _u64, _sz, _i32 = C.c_void_p, C.c_uint64, C.c_size_t, C.c_int
_pu64 = C.POINTER(C.c_uint64)
_pf = C.POINTER(C.c_float)

# name -> (restype, argtypes)
SIGNATURES = {
    "kvflux_last_error": (C.c_char_p, []),
    "kvflux_abi_version": (_i32, []),
    "kvflux_device_count": (_i32, [C.POINTER(C.c_int)]),
    "kvflux_get_device": (_i32, [C.POINTER(C.c_int)]),
    "kvflux_set_device": (_i32, [_i32]),
    "kvflux_device_malloc": (_i32, [C.POINTER(_vp), _sz]),
    "kvflux_device_free": (_i32, [_vp]),
    "kvflux_host_malloc_pinned": (_i32, [C.POINTER(_vp), _sz]),
    "kvflux_host_free_pinned": (_i32, [_vp]),
    "kvflux_host_device_pointer": (_i32, [_vp, C.POINTER(_vp)]),
    "kvflux_pointer_device": (_i32, [_vp, C.POINTER(C.c_int)]),
    "kvflux_memcpy_async": (_i32, [_vp, _vp, _sz, _vp]),
    "kvflux_memcpy": (_i32, [_vp, _vp, _sz]),
    "kvflux_fill_bytes": (_i32, [_vp, _i32, _sz, _vp]),
    "kvflux_stream_create": (_i32, [C.POINTER(_vp)]),
    "kvflux_stream_destroy": (_i32, [_vp]),
    "kvflux_stream_synchronize": (_i32, [_vp]),
    "kvflux_device_synchronize": (_i32, []),
    "kvflux_event_create": (_i32, [C.POINTER(_vp)]),
    "kvflux_event_destroy": (_i32, [_vp]),
    "kvflux_event_record": (_i32, [_vp, _vp]),
    "kvflux_event_elapsed_ms": (_i32, [C.POINTER(C.c_float), _vp, _vp]),
    "kvflux_event_synchronize": (_i32, [_vp]),
    "kvflux_event_query": (_i32, [_vp, C.POINTER(C.c_int)]),
    "kvflux_stream_wait_event": (_i32, [_vp, _vp]),
    "kvflux_write_paged_kv": (_i32, [_vp, _vp, _u64, _u64, _u64, _u64, _i32, _vp, _vp, _vp,
                                     _u64, _vp]),
    "kvflux_gather_paged_kv": (_i32, [_vp, _vp, _u64, _u64, _u64, _u64, _i32, _vp, _u64, _vp,
                                      _vp, _u64, _u64, _vp, _vp, _vp]),
    "kvflux_gather_paged_kv_live": (_i32, [_vp, _vp, _u64, _u64, _u64, _u64, _i32, _vp, _u64, _vp,
                                           _vp, _vp, _u64, _u64, _vp, _vp, _vp]),
    "kvflux_paged_attention_workspace_size": (_i32, [_u64, _u64, _u64, _u64, _u64, _u64,
                                                     C.POINTER(C.c_size_t)]),
    "kvflux_paged_attention": (_i32, [_vp, _vp, _u64, _u64, _u64, _u64, _i32, _vp, _u64, _vp,
                                      _u64, _u64, _u64, _vp, _vp, _vp, _sz, _vp]),
    "kvflux_paged_attention_noalloc": (_i32, [_vp, _vp, _u64, _u64, _u64, _u64, _i32, _vp, _u64, _vp,
                                              _u64, _u64, _u64, _vp, _vp, _vp]),
    "kvflux_paged_prefill": (_i32, [_vp, _vp, _u64, _u64, _u64, _u64, _i32, _vp, _u64, _u64,
                                    _u64, _u64, _vp, _vp, _vp]),
    "kvflux_paged_prefill_workspace_size": (_i32, [_u64, _u64, _u64, _u64, _u64, C.POINTER(_sz)]),
    "kvflux_paged_prefill_split": (_i32, [_vp, _vp, _u64, _u64, _u64, _u64, _i32, _vp, _u64, _u64,
                                          _u64, _u64, _vp, _vp, _vp, _u64, _vp]),
    "kvflux_paged_prefill_exact": (_i32, [_vp, _vp, _u64, _u64, _u64, _u64, _i32, _vp, _u64, _u64,
                                          _u64, _u64, _vp, _vp, _vp, _u64, _vp]),
    "kvflux_paged_prefill_batch": (_i32, [_vp, _vp, _u64, _u64, _u64, _u64, _i32, _vp, _u64, _vp, _vp, _vp,
                                          _u64, _u64, _u64, _u64, _vp, _vp, _vp]),
    "kvflux_copy_pages": (_i32, [_vp, _vp, _u64, _u64, _vp, _u64, _vp]),
    "kvflux_table_apply": (_i32, [_vp, _u64, _vp, _u64, _vp, _u64, _vp]),
    "kvflux_write_paged_kv_tail": (_i32, [_vp, _vp, _u64, _u64, _u64, _u64, _i32, _vp, _vp, _vp,
                                          _u64, _vp, _u64, _vp]),
    "kvflux_copy_chunks": (_i32, [_vp, _u64, _u64, _vp]),
    "kvflux_copy_page_list": (_i32, [_vp, _vp, _u64, _u64, _vp, _u64, _vp]),
    "kvflux_bandwidth_probe": (_i32, [_i32, _vp, _vp, _u64, C.c_uint32, C.c_uint32, C.c_uint32, _i32, _vp]),
    "kvflux_bandwidth_probe_pages": (_i32, [_vp, _vp, _u64, _u64, _vp, _u64, C.c_uint32, C.c_uint32, _i32, _vp,
                                            _vp]),
    "kvflux_fill_random": (_i32, [_vp, _u64, _i32, _i32, _u64, _vp]),
    "kvflux_compare_bytes": (_i32, [_vp, _vp, _u64, _pu64]),
}
EXPORTS = tuple(SIGNATURES)

_lib = None


def lib() -> C.CDLL:
    """Loads libkvflux_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        handle = C.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


class KvfluxError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[status {status}] {message}")
        self.status = status


def check(status: int) -> None:
    if status != OK:
        raise KvfluxError(status, lib().kvflux_last_error().decode())


def last_error() -> str:
    return lib().kvflux_last_error().decode()


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))


def device_count() -> int:
    n = C.c_int(0)
    call("kvflux_device_count", C.byref(n))
    return n.value
