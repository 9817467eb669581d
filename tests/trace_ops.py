"""Control-plane trace language shared by tests/golden/gen_golden.py (which
runs it on the reference's CPU library through oracle/ref_shim.cpp) and the
CPU tests (which replay it on kvflux_amd.v2). Op codes and result encoding
are defined in oracle/ref_shim.cpp."""
from __future__ import annotations

import random

import numpy as np

ALLOC, FREE, RETAIN, NEW_SEQ, APPEND, APPEND_ONE, FORK, DROP, SLOT, TABLE, AVAILABLE, REFS, \
    APPEND_COW, BATCH, PUBLISH, ATTACH, ID = range(17)


def random_trace(seed: int, capacity: int, block_size: int, steps: int) -> np.ndarray:
    """A seeded op sequence that mostly stays valid but also provokes errors
    (capacity exhaustion, stale handles, out-of-range positions)."""
    rng = random.Random(seed)
    ops = []
    handles = 0
    seqs = []  # indices of live sequences (as the interpreter numbers them)
    nseq = 0
    tokens = {}
    for _ in range(steps):
        r = rng.random()
        if r < 0.08 or not seqs:
            ops.append((NEW_SEQ, 0, 0)); seqs.append(nseq); tokens[nseq] = 0; nseq += 1
        elif r < 0.30:
            s = rng.choice(seqs); n = rng.choice([0, 1, 3, block_size - 1, block_size, 2 * block_size + 5])
            ops.append((APPEND, s, n))
        elif r < 0.42:
            ops.append((APPEND_ONE, rng.choice(seqs), 0))
        elif r < 0.47:
            ops.append((FORK, rng.choice(seqs), 0)); seqs.append(nseq); nseq += 1
        elif r < 0.52:
            ops.append((APPEND_COW, rng.choice(seqs), 0))
        elif r < 0.57 and len(seqs) > 1:
            s = rng.choice(seqs); seqs.remove(s); ops.append((DROP, s, 0))
        elif r < 0.65:
            ops.append((SLOT, rng.choice(seqs), rng.randrange(0, 4 * block_size)))
        elif r < 0.72:
            ops.append((TABLE, rng.choice(seqs), 0))
        elif r < 0.76:
            ops.append((ALLOC, 0, 0)); handles += 1
        elif r < 0.80 and handles:
            ops.append((FREE, rng.randrange(handles), 0))
        elif r < 0.82 and handles:
            ops.append((RETAIN, rng.randrange(handles), 0))
        elif r < 0.84 and handles:
            ops.append((ID, rng.randrange(handles), 0))
        elif r < 0.88:
            ops.append((AVAILABLE, 0, 0))
        elif r < 0.91:
            ops.append((REFS, rng.choice(seqs), rng.randrange(0, 3)))
        elif r < 0.94:
            ops.append((BATCH, rng.randrange(1, 5), 0))
        elif r < 0.97:
            ops.append((PUBLISH, rng.choice(seqs), rng.randrange(0, 3)))
        else:
            ops.append((ATTACH, rng.choice(seqs), rng.randrange(0, 4 * block_size)))
    return np.asarray(ops, dtype=np.int64).reshape(-1)


def churn_trace(seed: int, capacity: int, block_size: int, steps: int) -> np.ndarray:
    """A seeded op sequence heavy on prefix sharing: blocks are published,
    their sequences dropped (the pages go idle), re-attached by new
    sequences (idle pages held again) and evicted by allocations under
    capacity pressure, thousands of times over a small pool."""
    rng = random.Random(seed)
    ops = []
    seqs = []
    nseq = 0
    for _ in range(steps):
        r = rng.random()
        if r < 0.14 or not seqs:
            ops.append((NEW_SEQ, 0, 0)); seqs.append(nseq); nseq += 1
            if rng.random() < 0.7:  # attach a cached prefix to the new, empty sequence
                ops.append((ATTACH, nseq - 1, rng.choice([block_size, 2 * block_size, 3 * block_size,
                                                          4 * block_size + 1])))
        elif r < 0.34:
            s = rng.choice(seqs)
            ops.append((APPEND, s, rng.choice([1, block_size - 1, block_size, 2 * block_size])))
        elif r < 0.52:
            ops.append((PUBLISH, rng.choice(seqs), rng.randrange(0, 4)))
        elif r < 0.70 and len(seqs) > 1:
            s = rng.choice(seqs); seqs.remove(s); ops.append((DROP, s, 0))
        elif r < 0.76:
            ops.append((AVAILABLE, 0, 0))
        elif r < 0.84:
            ops.append((TABLE, rng.choice(seqs), 0))
        elif r < 0.90:
            ops.append((APPEND_ONE, rng.choice(seqs), 0))
        elif r < 0.93:
            ops.append((FORK, rng.choice(seqs), 0)); seqs.append(nseq); nseq += 1
        elif r < 0.97:
            ops.append((REFS, rng.choice(seqs), rng.randrange(0, 4)))
        else:
            ops.append((APPEND_COW, rng.choice(seqs), 0))
        if len(seqs) > 8:  # keep the live set small so the pool churns
            s = seqs.pop(0); ops.append((DROP, s, 0))
    return np.asarray(ops, dtype=np.int64).reshape(-1)


def _status(exc: BaseException, v2) -> int:
    if isinstance(exc, v2.CapacityError):
        return -4
    if isinstance(exc, ValueError):
        return -1
    if isinstance(exc, IndexError):
        return -2
    if isinstance(exc, OverflowError):
        return -3
    if isinstance(exc, v2.LogicError):
        return -5
    return -9


def replay(v2, capacity: int, block_size: int, ops: np.ndarray) -> np.ndarray:
    """Runs a trace on this repository's implementation (kvflux_amd.v2)."""
    pool = v2.PhysicalBlockPool(capacity, block_size)
    handles, seqs, out = [], [], []

    def seq(i):
        if i < 0 or i >= len(seqs) or seqs[i] is None:
            raise RuntimeError("bad trace sequence index")
        return seqs[i]

    def prefix(n):
        return list(range(n))

    def step(code, a, b):
        # Locals die when this returns, so a dropped sequence is released at
        # once, as in the C++ interpreter.
        if code == ALLOC:
            handles.append(pool.allocate())
            return [handles[-1].id]
        if code == FREE:
            pool.free(handles[a]); return [0]
        if code == RETAIN:
            pool.retain(handles[a]); return [0]
        if code == NEW_SEQ:
            seqs.append(v2.SequenceState(len(seqs), pool)); return [len(seqs) - 1]
        if code == APPEND:
            seq(a).append_tokens(b); return [0]
        if code == APPEND_ONE:
            loc = seq(a).append_token(); return [loc.physical_block * (1 << 20) + loc.offset_in_block]
        if code == FORK:
            seqs.append(seq(a).fork_shared(len(seqs))); return [len(seqs) - 1]
        if code == DROP:
            seqs[a] = None; return [0]
        if code == SLOT:
            return [v2.build_slot_mapping([(seq(a), b)])[0]]
        if code == TABLE:
            t = v2.build_read_block_table(seq(a)); return [len(t), *t]
        if code == AVAILABLE:
            return [pool.available()]
        if code == REFS:
            return [seq(a).block_table().ref_count(b)]
        if code == APPEND_COW:
            loc = seq(a).append_token_with_copy(lambda src, dst: None)
            return [loc.physical_block * (1 << 20) + loc.offset_in_block]
        if code == BATCH:
            t = v2.build_batch_block_table([s for s in seqs if s is not None][-a:] if a else [])
            return [t.max_blocks_per_sequence(), *t.sequence_lengths(),
                    *(x if x < 2**63 else x - 2**64 for x in t.block_table())]
        if code == PUBLISH:
            v2.PrefixCache(pool).publish_computed_block(seq(a), b, prefix((b + 1) * block_size))
            return [0]
        if code == ATTACH:
            return [v2.PrefixCache(pool).attach_cached_prefix(seq(a), prefix(b))]
        if code == ID:
            return [pool.id(handles[a])]
        return [-99]

    for code, a, b in np.asarray(ops).reshape(-1, 3).tolist():
        try:
            out.extend(step(code, a, b))
        except Exception as exc:  # noqa: BLE001 - every failure is encoded
            out.append(_status(exc, v2))
    # Drop sequences before the pool goes away.
    seqs.clear()
    return np.asarray(out, dtype=np.int64)
