"""MI355X (gfx950) paged-KV data path with the kvflux::v2 API.

`kvflux_amd.v2` is the Python binding of the C++17 layer (same class and
function names as kvflux::v2), `kvflux_amd.v3` that of the tiered cache
(kvflux::v3); `kvflux_amd.capi` is the raw C ABI of
libkvflux_hip.so; `kvflux_amd.device` holds device buffers, streams and
events made through that ABI. Nothing here falls back to a CPU path: if the
native libraries are missing, importing `v2` raises.
"""
from __future__ import annotations

import importlib


def _load_v2():
    try:
        return importlib.import_module("kvflux_amd._kvflux")
    except ImportError as e:  # pragma: no cover - exercised when unbuilt
        raise ImportError("kvflux_amd native extension is not built; run __graft_entry__.build()") from e


def __getattr__(name):
    if name == "v2":
        mod = _load_v2()
        globals()["v2"] = mod
        return mod
    if name == "v3":  # tiered cache (GPU <-> CPU chunk transfer), kvflux::v3
        mod = _load_v2().v3
        globals()["v3"] = mod
        return mod
    raise AttributeError(name)
