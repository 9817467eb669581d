"""Write and gather over a sweep of row shapes, through the C ABI.

The write and gather kernels pick their vector width from the row size
(head_size x element bytes) and their per-wavefront layout from the page
size, so each shape below exercises a different combination: 2-, 4-, 8- and
16-byte vectors, rows shorter than one vector per lane, pages of 1 to 64
tokens, one to eight kv heads, all three dtypes. Each case is bit-exact
against the oracle (a restatement of paged_kv_write.cu:62-83 and
paged_kv_read.cu:67-87):
  * write: the whole K and V arenas after scattering N tokens into a cache
    pre-filled with random bytes (slots past the arena are skipped, so every
    byte the oracle does not write must be unchanged), N = 0, 1 and odd;
  * gather: several sequences of ragged lengths (0, 1, a partial tail page)
    in one launch, with a guard region after the output left untouched,
    through both launches (the table-only 2D grid and the live-page grid
    driven by the scan of the page counts).
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import buffer_like
from kvflux_amd import capi, device
from oracle import oracle

pytestmark = pytest.mark.gpu

CODES = {"Float16": oracle.F16, "BFloat16": oracle.BF16, "Float32": oracle.F32}
ABI = {"Float16": capi.DTYPE_F16, "BFloat16": capi.DTYPE_BF16, "Float32": capi.DTYPE_F32}

SHAPES = [  # dtype, kv_heads, head_size, block_size
    ("Float16", 1, 1, 1),
    ("BFloat16", 3, 3, 16),
    ("Float32", 2, 3, 8),
    ("Float16", 2, 4, 16),
    ("Float32", 1, 5, 32),
    ("BFloat16", 8, 8, 16),
    ("Float16", 2, 40, 4),
    ("BFloat16", 8, 64, 16),
    ("Float32", 4, 64, 16),
    ("Float16", 3, 80, 32),
    ("BFloat16", 2, 96, 64),
    ("BFloat16", 8, 128, 16),
    ("Float16", 8, 128, 1),
    ("Float32", 8, 128, 16),
    ("BFloat16", 2, 256, 16),
    ("Float32", 1, 256, 2),
    ("BFloat16", 4, 512, 8),
]


def random_bytes(n, seed):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8)


@pytest.mark.parametrize("name,kv_heads,head_size,bs", SHAPES)
def test_write_shapes(gpu, name, kv_heads, head_size, bs):
    code, dt = CODES[name], ABI[name]
    e = 4 if name == "Float32" else 2
    blocks = 37
    slot_count = blocks * bs
    arena = blocks * kv_heads * bs * head_size * e
    seed = kv_heads * 1000 + head_size * 10 + bs
    k_host, v_host = random_bytes(arena, seed), random_bytes(arena, seed + 1)
    kc, vc = buffer_like(k_host), buffer_like(v_host)
    lib = capi.lib()
    rng = np.random.default_rng(seed)
    for n in (0, 1, min(slot_count, 77)):
        slots = rng.permutation(slot_count)[:n].astype(np.uint64)
        if n > 1:
            slots[rng.integers(0, n)] = slot_count + 5  # past the arena: skipped
        row = kv_heads * head_size * e
        kn, vn = random_bytes(max(n, 1) * row, seed + 2 + n), random_bytes(max(n, 1) * row, seed + 3 + n)
        knd, vnd, sd = buffer_like(kn), buffer_like(vn), buffer_like(slots if n else np.zeros(1, np.uint64))
        status = lib.kvflux_write_paged_kv(kc.ptr, vc.ptr, blocks, kv_heads, bs, head_size, dt, knd.ptr, vnd.ptr,
                                           sd.ptr, n, None)
        assert status == 0, capi.last_error()
        device.synchronize()
        keep = slots < slot_count
        oracle.write_paged_kv(k_host, v_host, kv_heads, bs, head_size, code,
                              kn[:n * row].reshape(n, row)[keep].copy(), vn[:n * row].reshape(n, row)[keep].copy(),
                              slots[keep])
        assert np.array_equal(kc.download(np.uint8), k_host), n
        assert np.array_equal(vc.download(np.uint8), v_host), n


@pytest.mark.parametrize("entry", ["table", "live"])
@pytest.mark.parametrize("name,kv_heads,head_size,bs", SHAPES)
def test_gather_shapes(gpu, name, kv_heads, head_size, bs, entry):
    code, dt = CODES[name], ABI[name]
    e = 4 if name == "Float32" else 2
    blocks = 64
    arena = blocks * kv_heads * bs * head_size * e
    seed = kv_heads * 2000 + head_size * 10 + bs
    k_host, v_host = random_bytes(arena, seed), random_bytes(arena, seed + 1)
    kc, vc = buffer_like(k_host), buffer_like(v_host)
    rng = np.random.default_rng(seed)
    lens = [0, 1, bs, 3 * bs - 1 if bs > 1 else 3, min(blocks // 4, 9) * bs + bs // 2]
    width = max((n + bs - 1) // bs for n in lens)
    perm = rng.permutation(blocks)
    table = np.full((len(lens), width), 2**64 - 1, np.uint64)
    used = 0
    for i, n in enumerate(lens):
        pages = (n + bs - 1) // bs
        table[i, :pages] = perm[used:used + pages]
        used += pages
    assert used <= blocks
    offsets = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.uint64)
    total = int(sum(lens))
    row = kv_heads * head_size * e
    guard = 64
    ko = buffer_like(np.full(total * row + guard, 0xA5, np.uint8))
    vo = buffer_like(np.full(total * row + guard, 0xA5, np.uint8))
    td, ld, od = buffer_like(table.reshape(-1)), buffer_like(np.array(lens, np.uint64)), buffer_like(offsets)
    if entry == "table":
        status = capi.lib().kvflux_gather_paged_kv(kc.ptr, vc.ptr, blocks, kv_heads, bs, head_size, dt, td.ptr,
                                                   width, ld.ptr, od.ptr, len(lens), max(lens), ko.ptr, vo.ptr, None)
    else:  # one workgroup per live page, from the exclusive scan of the page counts
        counts = np.array([(n + bs - 1) // bs for n in lens], np.uint64)
        starts = buffer_like(np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.uint64))
        status = capi.lib().kvflux_gather_paged_kv_live(kc.ptr, vc.ptr, blocks, kv_heads, bs, head_size, dt, td.ptr,
                                                        width, ld.ptr, od.ptr, starts.ptr, len(lens),
                                                        int(counts.sum()), ko.ptr, vo.ptr, None)
    assert status == 0, capi.last_error()
    device.synchronize()
    kg, vg = ko.download(np.uint8), vo.download(np.uint8)
    assert np.all(kg[total * row:] == 0xA5) and np.all(vg[total * row:] == 0xA5)
    for i, n in enumerate(lens):
        ek, ev = oracle.gather_paged_kv(k_host, v_host, kv_heads, bs, head_size, code, table[i], n)
        o = int(offsets[i]) * row
        assert np.array_equal(kg[o:o + n * row], ek.view(np.uint8)), i
        assert np.array_equal(vg[o:o + n * row], ev.view(np.uint8)), i
