"""The byte kernels behind kvflux_fill_bytes and kvflux_compare_bytes (test
and benchmark support; the benchmark also uses them as its write-only and
read-only bandwidth probes): exact results on sizes that end inside a
32 KiB chunk, inside a 16-byte vector and on a single byte."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from kvflux_amd import capi, device

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [1, 15, 16, 4097, 32768, 3 * 32768 + 16 * 5 + 7, (1 << 23) + 48])
def test_fill_and_compare_exact(gpu, nbytes):
    pad = 64
    buf = device.DeviceBuffer(nbytes + pad)
    buf.fill(0x11)
    capi.call("kvflux_fill_bytes", C.c_void_p(buf.ptr), 0xA7, nbytes, None)
    device.synchronize()
    got = buf.download(np.uint8)
    assert np.all(got[:nbytes] == 0xA7) and np.all(got[nbytes:] == 0x11)
    other = device.DeviceBuffer(nbytes + pad)
    other.upload(got)
    assert device.compare_bytes(buf.ptr, other.ptr, nbytes) == 0
    # plant differences: first byte, last byte and (when present) one in a whole chunk
    flips = sorted({0, nbytes - 1, min(nbytes - 1, 40000)})
    changed = got.copy()
    changed[flips] ^= 0x5A
    other.upload(changed)
    assert device.compare_bytes(buf.ptr, other.ptr, nbytes) == len(flips)
    assert device.compare_bytes(buf.ptr, other.ptr, nbytes + pad) == len(flips)
