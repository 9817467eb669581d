"""Benchmark of the paged-KV data path on one MI355X.

Prints ONE JSON line (stdout). Progress goes to stderr.

Headline (`value`): batch GQA decode PagedAttention, B=128 rows with
seq_len ~ U[1024, 32768], 32 query / 8 KV heads, head_size 128,
block_size 16, BF16 K/V ~ N(0,1), FP32 Q ~ N(0,1), a 2048-token prefix
shared by every row through the same physical pages, the other pages drawn
from a seeded permutation of a 2^18-page pool. `value` is HBM throughput in
TB/s over the UNIQUE bytes the step must read (shared prefix pages once) plus
Q, O and the tables; logical bytes are reported next to it.

Also measured in the same run (sub-objects of the JSON line):
  decode_contiguous: the same decode launch on a contiguous layout (same
           lengths and shared prefix, each row's own pages consecutive):
           `frag_over_contig` is the fragmented batch's rate over it
  decode_read_ceiling: every unique page of the batch (K and V) read once,
           in the order the rows meet them, by a kernel that only reads
           (kvflux_bandwidth_probe_pages, best of six launch shapes), and the
           decode's rate over it
  write  : slot-mapped KV write, 4096 tokens x 8 heads x 128, BF16, 65536-page
           pool. Headline HBM-cold (16 rotated input/slot sets on distinct
           pages, 537 MB); `warm` repeats one set (Infinity Cache), and
           `contiguous` writes into an unfragmented pool
  gather : BlockTable gather, 64 sequences with L ~ U[512, 8192], H=8, D=128,
           FP16 and BF16, odd pages of a full 65536-page pool: the live-page
           launch (the C++ API's), the table launch, and two ceilings timed
           beside them: a plain streaming copy of the same byte count and a
           copy of the same source pages into a contiguous buffer
  prefill: causal paged prefill on MFMA, 8 sequences x 4096 tokens written
           through slot_mapping into random pages, 32 q / 8 kv heads, D=128,
           BF16; TFLOP/s and MFMA utilisation against 2.5 PFLOP/s dense BF16
  cow    : batched copy-on-write page copy, 4096 pairs of 32 KiB K and V
           pages, HBM-cold (8 rotated pair sets covering the pool), with one
           repeated set and contiguous pairs beside it
  decode_step: whole decode steps on the decode batch through the C++ API
           (device batch table) against the reference API's composition
  offload: GPU <-> CPU chunk transfer (tiered cache), per-chunk DMA against
           one kernel per batch, and overlap with the decode kernel; the host
           time of the begin calls beside each rate
  gather_BFloat16.cpu_baseline : the CPU oracle's gather (one thread) on 16
           of the 64 sequences, pages in a shuffled host cache, in the GPU
           figure's bytes.
  prefill.cpu_baseline : the oracle calls that check the prefill's 128
           sampled rows, timed (8 threads).
  cpu_baseline : the CPU oracle (gather + double-precision attention, one
           thread) on a bounded sample of the decode rows, timed here; the
           same rows on all cores of the process's CPU share (at most 16) in
           `all_cores`, and the CPU model.
  write, gather and prefill also report the synchronous C++ API time
  (`api_us` / `api_ms`: validation, metadata upload, launch, synchronisation),
  timed in C++ by the extension's `timing` module.

roofline.traffic is the HBM traffic of one decode call measured with
rocprofv3 FETCH_SIZE / WRITE_SIZE and scaled by what the same counters read
for a copy of known size (`python bench.py --calibrate-copy`); it is read
from profiles/decode_bs16_traffic.txt when that summary is present.

`--only LEG` runs one leg alone (write, gather, prefill, cow, ceilings, or
cow_placement: the copy-on-write pairs placed seven ways, to locate the cost
of random placement) and prints its JSON object.

Every timed region launches through the C ABI on a dedicated stream with all
inputs and metadata already resident in HBM; HIP events on that stream give
the average kernel time per launch.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBPS = 8000.0
PEAK_BF16_TFLOPS = 2500.0  # dense MFMA
PEAK_FP32_MFMA_TFLOPS = 157.3  # dense FP32 MFMA
TRAFFIC_SUMMARY = ROOT / "profiles" / "decode_bs16_traffic.txt"
PREFILL_COUNTERS = ROOT / "profiles" / "prefill_counters.txt"
METRIC = "decode paged-attn HBM TB/s (% of peak) + KV write/gather GB/s, 1 GPU"


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def fragment_pool(pool, order: np.ndarray) -> None:
    """Allocates every page, then frees `order` reversed so that subsequent
    allocations return the pages in `order` (LIFO free list)."""
    holders = [pool.allocate() for _ in range(pool.capacity())]
    for idx in order[::-1]:
        pool.free(holders[int(idx)])
    keep = np.ones(pool.capacity(), bool)
    keep[order] = False
    return [holders[i] for i in np.nonzero(keep)[0]]


def time_launches(launch, stream, warmup: int, steps: int) -> float:
    """Average milliseconds per launch measured with HIP events on `stream`."""
    from kvflux_amd import device
    for _ in range(warmup):
        launch()
    device.synchronize(stream)
    start, stop = device.Event(), device.Event()
    start.record(stream)
    for _ in range(steps):
        launch()
    stop.record(stream)
    return start.elapsed_ms(stop) / steps


# --------------------------------------------------------------------- decode
def bench_decode(v2, args, stream):
    from kvflux_amd import capi, device
    from oracle import oracle

    B, H, Hq, D, bs, prefix = 128, 8, 32, 128, args.block_size, 2048
    rng = np.random.default_rng(args.seed)
    lens = rng.integers(1024, 32768 + 1, B)
    pool = v2.PhysicalBlockPool((1 << 22) // bs, bs)  # 2^22 tokens of room
    storage = v2.PagedKVStorage(pool, H, D, v2.DType.BFloat16)
    fragment_pool(pool, rng.permutation(pool.capacity()))
    cache = v2.PrefixCache(pool)
    base = v2.SequenceState(10**9, pool)
    base.append_tokens(prefix)
    tokens = list(range(prefix))
    for blk in range(prefix // bs):
        cache.publish_computed_block(base, blk, tokens[: (blk + 1) * bs])
    seqs = []
    for i, L in enumerate(lens.tolist()):
        s = v2.SequenceState(i, pool)
        shared = cache.attach_cached_prefix(s, tokens[: min(L, prefix)])
        s.append_tokens(L - shared)
        seqs.append(s)
    table = v2.build_batch_block_table(seqs)
    flat = np.array(table.block_table(), np.uint64)
    width = table.max_blocks_per_sequence()
    n_elems = storage.layout().cache_bytes() // 2
    device.fill_random(storage.key_base(), n_elems, capi.DTYPE_BF16, 1, args.seed + 1)
    device.fill_random(storage.value_base(), n_elems, capi.DTYPE_BF16, 1, args.seed + 2)
    q = device.DeviceBuffer(B * Hq * D * 4)
    o = device.DeviceBuffer(B * Hq * D * 4)
    device.fill_random(q.ptr, B * Hq * D, capi.DTYPE_F32, 1, args.seed + 3)
    td = device.to_device(flat)
    ld = device.to_device(lens.astype(np.uint64))
    ws = C.c_size_t(0)
    capi.call("kvflux_paged_attention_workspace_size", B, int(lens.max()), H, Hq, bs, D, C.byref(ws))
    wd = device.DeviceBuffer(ws.value)
    wd.fill(0)
    device.synchronize()
    lib = capi.lib()
    kb, vb, max_len = storage.key_base(), storage.value_base(), int(lens.max())

    def launch():
        capi.check(lib.kvflux_paged_attention(kb, vb, pool.capacity(), H, bs, D, capi.DTYPE_BF16,
                                              td.ptr, width, ld.ptr, max_len, B, Hq, q.ptr, o.ptr,
                                              wd.ptr, ws.value, stream))

    ms = time_launches(launch, stream, args.warmup, args.steps)
    out = o.download(np.float32)
    mat = flat.reshape(B, width)

    # The same launch on a contiguous layout: the shared prefix on pages
    # 0..127, each row's own pages consecutive after it (same lengths, same
    # sharing, same bytes), for the fragmentation's cost.
    prefix_pages = [int(base.physical_block_id(b)) for b in range(prefix // bs)]
    ident = np.full_like(mat, 2**64 - 1)
    nxt = prefix // bs
    for r in range(B):
        for blk in range((int(lens[r]) + bs - 1) // bs):
            if blk < len(prefix_pages) and int(mat[r, blk]) == prefix_pages[blk]:
                ident[r, blk] = blk
            else:
                ident[r, blk] = nxt
                nxt += 1
    assert nxt <= pool.capacity()
    tcd = device.to_device(ident.reshape(-1))
    device.synchronize()

    def launch_contig():
        capi.check(lib.kvflux_paged_attention(kb, vb, pool.capacity(), H, bs, D, capi.DTYPE_BF16,
                                              tcd.ptr, width, ld.ptr, max_len, B, Hq, q.ptr, o.ptr,
                                              wd.ptr, ws.value, stream))

    ms_contig = time_launches(launch_contig, stream, args.warmup, args.steps)
    del tcd

    # Read ceiling of the same pages: every unique page of the batch (K and
    # V, whole pages) read once in the order the rows meet them, by a kernel
    # that only reads (kvflux_bandwidth_probe_pages), best of six shapes.
    order, seen_pages = [], set()
    for r in range(B):
        for blk in range((int(lens[r]) + bs - 1) // bs):
            page = int(mat[r, blk])
            if page not in seen_pages:
                seen_pages.add(page)
                order.append(page)
    pl = device.to_device(np.array(order, np.uint64))
    sink = device.DeviceBuffer(1024 * 16)
    page_bytes_all = H * bs * D * 2
    ceiling = None
    for threads in (256, 512, 1024):
        for vpt in (1, 2):
            def probe(t=threads, v=vpt):
                capi.check(lib.kvflux_bandwidth_probe_pages(kb, vb, pool.capacity(), page_bytes_all, pl.ptr,
                                                            len(order), t, v, 1, sink.ptr, stream))
            pms = time_launches(probe, stream, 2, 10)
            if ceiling is None or pms < ceiling[0]:
                ceiling = (pms, threads, vpt)
    read_bytes = 2 * len(order) * page_bytes_all
    del pl, sink

    # Bytes: every (page, kv head) row read once, counted by unique page.
    tok_per_page = {}
    for r in range(B):
        L = int(lens[r])
        for blk in range((L + bs - 1) // bs):
            page = int(mat[r, blk])
            tok_per_page[page] = max(tok_per_page.get(page, 0), min(bs, L - blk * bs))
    kv_token_bytes = H * D * 2 * 2  # K and V, BF16, all kv heads
    io_bytes = 2 * B * Hq * D * 4 + flat.nbytes + lens.size * 8
    unique_bytes = sum(tok_per_page.values()) * kv_token_bytes + io_bytes
    logical_bytes = int(lens.sum()) * kv_token_bytes + io_bytes
    flops = 4 * Hq * D * int(lens.sum())

    # CPU oracle on a bounded sample of rows (copied to a compact host cache).
    sample_rows = list(range(args.cpu_rows))
    qh = q.download(np.float32).reshape(B, Hq * D)
    page_bytes = H * bs * D * 2
    err = 0.0
    cpu_s = 0.0
    cpu_bytes = 0
    compact = []
    for r in sample_rows:
        L = int(lens[r])
        npg = (L + bs - 1) // bs
        pages = mat[r, :npg]
        kc = np.empty(npg * page_bytes // 2, np.uint16)
        vc = np.empty_like(kc)
        for j, pg in enumerate(pages.tolist()):
            kc[j * page_bytes // 2:(j + 1) * page_bytes // 2] = device.memcpy_d2h(kb + pg * page_bytes, page_bytes, np.uint16)
            vc[j * page_bytes // 2:(j + 1) * page_bytes // 2] = device.memcpy_d2h(vb + pg * page_bytes, page_bytes, np.uint16)
        local = np.arange(npg, dtype=np.uint64)
        t0 = time.perf_counter()
        ref = oracle.paged_attention_rows(kc, vc, H, bs, D, oracle.BF16, local, npg,
                                          np.array([L], np.uint64), qh[r], Hq, threads=1)
        cpu_s += time.perf_counter() - t0
        cpu_bytes += L * kv_token_bytes
        err = max(err, float(np.abs(ref - out[r * Hq * D:(r + 1) * Hq * D]).max()))
        compact.append((kc, vc, local, npg, L, r))
    # The same rows on all cores of this process's CPU share (at most 16, the
    # share of one GPU): the oracle splits each row's query heads over threads.
    threads = min(16, len(os.sched_getaffinity(0)))
    cpu_mt_s = 0.0
    for kc, vc, local, npg, L, r in compact:
        t0 = time.perf_counter()
        oracle.paged_attention_rows(kc, vc, H, bs, D, oracle.BF16, local, npg, np.array([L], np.uint64), qh[r], Hq,
                                    threads=threads)
        cpu_mt_s += time.perf_counter() - t0
    del compact
    step = None if args.skip_aux else bench_decode_step(v2, args, storage, seqs, width, ms)
    offload = None if args.skip_aux else bench_offload(v2, args, launch, stream, ms)
    del seqs, base
    return {
        "decode_step": step,
        "offload": offload,
        "ms": ms,
        "ms_contiguous": ms_contig,
        "read_ceiling": {"ms": ceiling[0], "TBps": read_bytes / (ceiling[0] * 1e-3) / 1e12, "bytes": read_bytes,
                         "pages": len(order),
                         "kernel": f"kvflux_bandwidth_probe_pages, {ceiling[1]} threads x {ceiling[2]} vectors, "
                                   "non-temporal (best of 256/512/1024 x 1/2)"},
        "unique_bytes": unique_bytes,
        "logical_bytes": logical_bytes,
        "flops": flops,
        "sum_len": int(lens.sum()),
        "max_abs_err": err,
        "cpu": None if not sample_rows else
               {"value": cpu_bytes / cpu_s / 1e12, "unit": "TB/s", "cores": 1, "kind": "port",
                "seconds": cpu_s, "cpu_model": cpu_model(),
                "all_cores": {"value": cpu_bytes / cpu_mt_s / 1e12, "cores": threads, "seconds": cpu_mt_s},
                "sample": f"{len(sample_rows)} decode rows (L={[int(lens[r]) for r in sample_rows]}, "
                          "32 q heads each): page gather + double-precision softmax attention, 1 thread"},
    }


def bench_decode_step(v2, args, storage, seqs, width, kernel_ms):
    """Whole decode steps on the same batch through the C++ API (synchronous):
    decode_step (device table, batched copy-on-write, tail-slot write, batch
    attention, one sync) against the reference API's composition of the same
    step (append_token_cow per row, slot mapping + write_paged_kv, host batch
    table + paged_attention_batch). Both include host work and every sync."""
    from kvflux_amd import capi, device

    B, H, Hq, D = len(seqs), 8, 32, 128
    kn, vn = device.DeviceBuffer(B * H * D * 2), device.DeviceBuffer(B * H * D * 2)
    device.fill_random(kn.ptr, B * H * D, capi.DTYPE_BF16, 1, args.seed + 5)
    device.fill_random(vn.ptr, B * H * D, capi.DTYPE_BF16, 1, args.seed + 6)
    q, o = device.DeviceBuffer(B * Hq * D * 4), device.DeviceBuffer(B * Hq * D * 4)
    device.fill_random(q.ptr, B * Hq * D, capi.DTYPE_F32, 1, args.seed + 7)
    table = v2.DeviceBatchTable(storage, seqs, width + 64)
    steps = 10

    def run_device(n):
        t0 = time.perf_counter()
        for _ in range(n):
            v2.decode_step(storage, table, kn.ptr, vn.ptr, q.ptr, o.ptr, Hq)
        return (time.perf_counter() - t0) / n * 1e3

    def run_composed(n):
        t0 = time.perf_counter()
        for _ in range(n):
            for s in seqs:
                v2.append_token_cow(storage, s)
            v2.write_paged_kv(storage, kn.ptr, vn.ptr,
                              v2.build_slot_mapping([(s, s.num_tokens() - 1) for s in seqs]))
            v2.paged_attention_batch(storage, seqs, q.ptr, o.ptr, Hq)
        return (time.perf_counter() - t0) / n * 1e3

    run_device(2)
    dev_ms = run_device(steps)
    run_composed(2)
    comp_ms = run_composed(steps)
    max_blocks = max(s.num_allocated_blocks() for s in seqs)
    return {
        "rows": B,
        "ms": dev_ms,
        "composed_reference_api_ms": comp_ms,
        "attention_kernel_ms": kernel_ms,
        "host_to_device_bytes_per_step": B * 32,
        "composed_host_to_device_bytes_per_step": B * 8 + B * max_blocks * 8 + B * 8,
        "note": "synchronous C++ API, host work included; steps append one token per row",
    }


# --------------------------------------------------------------------- offload
def bench_offload(v2, args, decode_launch, stream, decode_ms):
    """GPU <-> CPU chunk transfer of the tiered cache (kvflux::v3): 4096 chunks
    of 64 KiB (256 MiB) with scattered pinned host slots, moved
    * one DMA copy per chunk (the reference's GpuCpuTransfer, one
      cudaMemcpyAsync per begin_offload / begin_onload), and
    * one kernel per batch (begin_offload_batch / begin_onload_batch).
    Rates are bytes over the transfer stream's own event time. Each offload
    is repeated while decode steps run on the compute stream, to see how
    much the two slow each other."""
    import kvflux_amd
    from kvflux_amd import device

    v3 = kvflux_amd.v3
    N, CB = 4096, 65536
    pool = v2.PhysicalBlockPool(N, 16)
    gpu, cpu, nvme = v3.GpuTier(pool, CB), v3.CpuTier(N, CB), v3.NvmeTier(1, CB)
    directory = v3.CacheDirectory(gpu, cpu, nvme)
    store, host = v3.GpuChunkStore(N, CB), v3.PinnedChunkPool(N, CB)
    xfer = v3.GpuCpuTransfer(directory, store, host)
    keys = [v3.make_cache_key("bench", 1, v2.DType.BFloat16, 0, 1, [i]) for i in range(N)]
    rng = np.random.default_rng(args.seed + 50)
    for k in keys:
        directory.create(k)
    # scatter the host slots: take them in a random order
    order = rng.permutation(N)
    for i in order:
        directory.place(keys[int(i)], v3.StorageTier.CPU)
    for k in keys:
        directory.place(k, v3.StorageTier.GPU)
        directory.remove(k, v3.StorageTier.CPU)
    base = store.device_ptr(v3.TierLocation(0, 0))  # slot 0: the start of the store
    device.fill_random(base, N * CB // 2, 1, 0, args.seed + 51)
    device.synchronize()
    total = N * CB

    xs = xfer.stream()

    def move(batch, to_host, release=True, during=None):
        """One direction for every key; returns the transfer stream's time (ms)
        from the first copy to the last, and the decode time per step (ms)
        when `during` launches decode steps meanwhile."""
        e0, e1 = device.Event(), device.Event()
        e0.record(xs)
        t0 = time.perf_counter()
        if batch:
            (xfer.begin_offload_batch if to_host else xfer.begin_onload_batch)(keys)
        else:
            for k in keys:
                (xfer.begin_offload if to_host else xfer.begin_onload)(k)
        host_ms = (time.perf_counter() - t0) * 1e3
        e1.record(xs)
        dec = during() if during else None
        for k in keys:
            (xfer.finish_offload if to_host else xfer.finish_onload)(k, release)
        return e0.elapsed_ms(e1), dec, host_ms

    def decode_steps(n=10):
        start, stop = device.Event(), device.Event()
        start.record(stream)
        for _ in range(n):
            decode_launch()
        stop.record(stream)
        return start.elapsed_ms(stop) / n

    res = {"chunks": N, "chunk_bytes": CB, "bytes": total, "decode_ms_alone": decode_ms}
    first = device.memcpy_d2h(store.device_ptr(directory.at(keys[0]).gpu.location), CB, np.uint8)
    for batch in (False, True):
        move(batch, True), move(batch, False)  # warm
        off, _, off_host = move(batch, True)
        on, _, on_host = move(batch, False)
        # the offload again, this time under decode steps on the compute stream
        off_during, dec, _ = move(batch, True, release=False, during=decode_steps)
        for k in keys:  # back to GPU-only
            directory.remove(k, v3.StorageTier.CPU)
        res["batch_kernel" if batch else "dma_per_chunk"] = {
            "offload_GBps": total / off / 1e6, "onload_GBps": total / on / 1e6,
            "offload_GBps_during_decode": total / off_during / 1e6, "decode_ms_during_offload": dec,
            # host time of the begin call(s): key checks, directory updates, enqueueing
            "offload_begin_host_ms": off_host, "onload_begin_host_ms": on_host}
    again = device.memcpy_d2h(store.device_ptr(directory.at(keys[0]).gpu.location), CB, np.uint8)
    res["round_trip_identical"] = bool(np.array_equal(first, again))
    return res


# --------------------------------------------------------------------- copy-on-write
def bench_cow(v2, args, stream):
    """Batched page copy (copy-on-write) kernel: 4096 (source, destination)
    pairs of 32 KiB pages (8 kv heads x 16 tokens x 128, BF16) in a
    65536-page pool; K and V pages both copied (0.537 GB moved per launch).

    The headline is HBM-cold: the launches rotate over 8 pair sets that
    together touch every page of the pool once (8 x 0.537 GB per cycle, far
    past the 256 MB Infinity Cache). `warm` repeats one set; `contiguous`
    copies pages i -> 4096 + i (same
    byte count, consecutive pages), so `frag_over_contig` is the random
    placement's cost."""
    from kvflux_amd import capi, device

    P, H, D, bs, SETS = 4096, 8, 128, 16, 8
    rng = np.random.default_rng(args.seed + 40)
    pool = v2.PhysicalBlockPool(65536, bs)
    storage = v2.PagedKVStorage(pool, H, D, v2.DType.BFloat16)
    n = storage.layout().cache_bytes() // 2
    device.fill_random(storage.key_base(), n, capi.DTYPE_BF16, 1, args.seed + 41)
    device.fill_random(storage.value_base(), n, capi.DTYPE_BF16, 1, args.seed + 42)
    order = rng.permutation(65536)
    sets = []
    for j in range(SETS):
        src, dst = order[2 * j * P:(2 * j + 1) * P], order[(2 * j + 1) * P:(2 * j + 2) * P]
        sets.append((src, dst, device.to_device(np.stack([src, dst], 1).astype(np.uint64).reshape(-1))))
    contig = np.stack([np.arange(P), P + np.arange(P)], 1).astype(np.uint64).reshape(-1)
    cd = device.to_device(contig)
    lib = capi.lib()
    kb, vb = storage.key_base(), storage.value_base()
    page_bytes = storage.layout().page_bytes()
    cycle = [0]

    def launch_cold():
        pd = sets[cycle[0] % SETS][2]
        cycle[0] += 1
        capi.check(lib.kvflux_copy_pages(kb, vb, 65536, page_bytes, pd.ptr, P, stream))

    def launch_warm():
        capi.check(lib.kvflux_copy_pages(kb, vb, 65536, page_bytes, sets[0][2].ptr, P, stream))

    def launch_contig():
        capi.check(lib.kvflux_copy_pages(kb, vb, 65536, page_bytes, cd.ptr, P, stream))

    ms = time_launches(launch_cold, stream, SETS, SETS * max(4, args.steps // 4))
    ms_warm = time_launches(launch_warm, stream, args.warmup, max(args.steps, 50))
    ms_contig = time_launches(launch_contig, stream, args.warmup, max(args.steps, 50))
    launch_warm()  # the checked set copied last
    device.synchronize(stream)
    src, dst, _ = sets[0]
    mism = 0
    for i in range(0, P, P // 64):  # sampled pairs, bit-exact
        for base in (kb, vb):
            a = device.memcpy_d2h(base + int(src[i]) * page_bytes, page_bytes, np.uint8)
            b = device.memcpy_d2h(base + int(dst[i]) * page_bytes, page_bytes, np.uint8)
            mism += int((a != b).sum())
    bytes_step = 2 * 2 * P * page_bytes
    gbps = bytes_step / (ms * 1e-3) / 1e9
    return {"kernel_us": ms * 1e3, "GBps": gbps, "pct_of_peak": round(100 * gbps / PEAK_HBM_GBPS, 2),
            "bytes": bytes_step, "basis": "HBM-cold: 8 rotated pair sets covering the 65536-page pool",
            "pairs": P, "page_bytes": page_bytes, "pairs_checked": 64, "mismatched_bytes": mism,
            "warm": {"kernel_us": ms_warm * 1e3, "GBps": bytes_step / (ms_warm * 1e-3) / 1e9,
                     "note": "one pair set repeated (non-temporal stores: no faster than cold)"},
            "contiguous": {"kernel_us": ms_contig * 1e3, "GBps": bytes_step / (ms_contig * 1e-3) / 1e9},
            "frag_over_contig": round(ms_contig / ms, 4)}


def bench_cow_placement(v2, args, stream):
    """Where copy-on-write's random-placement cost comes from: the same 4096
    pairs of 32 KiB pages (K and V, 0.537 GB moved) placed eight ways in the
    65536-page pool, each launched 50 times back to back on one pair set.
    Separates the order of the pairs, the spread of the pages (a 256 MiB
    region against the whole 2 GiB cache) and random sources against random
    destinations."""
    from kvflux_amd import capi, device

    P, H, D, bs, N = 4096, 8, 128, 16, 65536
    pool = v2.PhysicalBlockPool(N, bs)
    storage = v2.PagedKVStorage(pool, H, D, v2.DType.BFloat16)
    n = storage.layout().cache_bytes() // 2
    device.fill_random(storage.key_base(), n, capi.DTYPE_BF16, 1, args.seed + 41)
    device.fill_random(storage.value_base(), n, capi.DTYPE_BF16, 1, args.seed + 42)
    kb, vb = storage.key_base(), storage.value_base()
    page_bytes = storage.layout().page_bytes()
    lib = capi.lib()
    rng = np.random.default_rng(args.seed + 43)
    order = rng.permutation(N)
    src, dst = order[:P], order[P:2 * P]
    by_src, by_dst = np.argsort(src, kind="stable"), np.argsort(dst, kind="stable")
    local = rng.permutation(2 * P)
    cases = {
        "random": (src, dst),
        "random_sorted_by_source": (src[by_src], dst[by_src]),
        "random_sorted_by_destination": (src[by_dst], dst[by_dst]),
        "random_within_8192_pages": (local[:P], local[P:]),
        "consecutive_sources_random_destinations": (np.arange(P), P + rng.permutation(N - P)[:P]),
        "random_sources_consecutive_destinations": (P + rng.permutation(N - P)[:P], np.arange(P)),
        "consecutive": (np.arange(P), P + np.arange(P)),
    }
    res = {"pairs": P, "page_bytes": page_bytes, "bytes": 2 * 2 * P * page_bytes, "kernel_us": {}}
    for name, (s_, d_) in cases.items():
        s_, d_ = np.asarray(s_, np.uint64), np.asarray(d_, np.uint64)
        if len(set(s_.tolist()) | set(d_.tolist())) != 2 * P or max(s_.max(), d_.max()) >= N:
            raise RuntimeError(f"cow placement case {name}: pages not distinct or out of the pool")
        pd = device.to_device(np.stack([s_, d_], 1).reshape(-1))
        ms = time_launches(lambda: capi.check(lib.kvflux_copy_pages(kb, vb, N, page_bytes, pd.ptr, P, stream)),
                           stream, args.warmup, 50)
        res["kernel_us"][name] = round(ms * 1e3, 2)
    return res


# --------------------------------------------------------------------- write
def bench_write(v2, args, stream):
    """KV write, 4096 tokens x 8 heads x 128 BF16 into a 65536-page pool.

    The headline figure (`kernel_us`, `GBps`, `pct_of_peak`) is HBM-cold: the
    launches rotate over 16 distinct (K_new, V_new, slots) sets on distinct
    pages, 537 MB in all, more than the 256 MB Infinity Cache. `warm` repeats
    one step's inputs and slots (its inputs and pages stay in that cache), and
    `contiguous` is the cold write into an unfragmented pool (consecutive
    pages), so `frag_over_contig` is the fragmentation's cost."""
    from kvflux_amd import capi, device
    from oracle import oracle

    N_SEQ, NEW, H, D, bs = 256, 16, 8, 128, 16
    rng = np.random.default_rng(args.seed + 10)
    pool = v2.PhysicalBlockPool(65536, bs)
    storage = v2.PagedKVStorage(pool, H, D, v2.DType.BFloat16)
    fragment_pool(pool, rng.permutation(pool.capacity()))
    prefix_lens = rng.integers(0, 2048, N_SEQ)
    seqs = []
    writes = []
    for i, L0 in enumerate(prefix_lens.tolist()):
        s = v2.SequenceState(i, pool)
        s.append_tokens(L0 + NEW)
        seqs.append(s)
        writes += [(s, L0 + j) for j in range(NEW)]
    slots = np.array(v2.build_slot_mapping(writes), np.uint64)
    N = slots.size
    n = N * H * D
    kn, vn = device.DeviceBuffer(n * 2), device.DeviceBuffer(n * 2)
    device.fill_random(kn.ptr, n, capi.DTYPE_BF16, 1, args.seed + 11)
    device.fill_random(vn.ptr, n, capi.DTYPE_BF16, 1, args.seed + 12)
    lib = capi.lib()
    capi.call("kvflux_fill_bytes", C.c_void_p(storage.key_base()), 0xA5, storage.layout().total_bytes(), None)
    sd = device.to_device(slots)
    device.synchronize()
    kb, vb = storage.key_base(), storage.value_base()

    def launch():
        capi.check(lib.kvflux_write_paged_kv(kb, vb, pool.capacity(), H, bs, D, capi.DTYPE_BF16,
                                             kn.ptr, vn.ptr, sd.ptr, N, stream))

    warm_ms = time_launches(launch, stream, args.warmup, max(args.steps, 50))
    # Full synchronous C++ API call (host validation + upload + kernel + sync).
    slot_list = slots.tolist()
    for _ in range(3):
        v2.write_paged_kv(storage, kn.ptr, vn.ptr, slot_list)
    # The synchronous C++ API, timed in C++ (the Python binding would add the
    # conversion of 4096 slots from a Python list to every call).
    api_us = v2.timing.write_paged_kv(storage, kn.ptr, vn.ptr, slot_list, 50) * 1e6

    # Bit-exact check of every touched page (and its untouched slots).
    page_elems = H * bs * D
    pages = np.unique(slots // bs)
    remap = {int(p): j for j, p in enumerate(pages.tolist())}
    host_k = np.full(pages.size * page_elems, 0xA5A5, np.uint16)
    host_v = host_k.copy()
    oracle.write_paged_kv(host_k, host_v, H, bs, D, oracle.BF16, kn.download(np.uint16),
                          vn.download(np.uint16),
                          np.array([remap[int(s // bs)] * bs + int(s % bs) for s in slots], np.uint64))
    mism = 0
    for j, pg in enumerate(pages.tolist()):
        gk = device.memcpy_d2h(kb + pg * page_elems * 2, page_elems * 2, np.uint16)
        gv = device.memcpy_d2h(vb + pg * page_elems * 2, page_elems * 2, np.uint16)
        mism += int((gk != host_k[j * page_elems:(j + 1) * page_elems]).sum())
        mism += int((gv != host_v[j * page_elems:(j + 1) * page_elems]).sum())
    bytes_step = 2 * 2 * N * H * D * 2 + N * 8
    cold = bench_write_cold(v2, args, stream, pool, storage, rng)
    del seqs
    # The same cold write into an unfragmented pool: pages handed out in order.
    pool_c = v2.PhysicalBlockPool(65536, bs)
    storage_c = v2.PagedKVStorage(pool_c, H, D, v2.DType.BFloat16)
    contig = bench_write_cold(v2, args, stream, pool_c, storage_c, np.random.default_rng(args.seed + 13))
    del storage_c, pool_c
    warm = {"kernel_us": warm_ms * 1e3, "GBps": bytes_step / (warm_ms * 1e-3) / 1e9,
            "pct_of_peak": round(100 * bytes_step / (warm_ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 2),
            "note": "one step's inputs and slots repeated: inputs and written pages stay in the Infinity Cache"}
    return {"kernel_us": cold["kernel_us"], "GBps": cold["GBps"], "pct_of_peak": cold["pct_of_peak"],
            "bytes": bytes_step, "basis": "HBM-cold: 16 rotated input/slot sets on distinct pages (537 MB)",
            "sets": cold["sets"], "working_set_bytes": cold["working_set_bytes"],
            "sets_checked": cold["sets_checked"], "mismatched_elements_cold": cold["mismatched_elements"],
            "api_us": api_us, "tokens": N, "pages_checked": int(pages.size), "mismatched_elements": mism,
            "warm": warm,
            "contiguous": {"kernel_us": contig["kernel_us"], "GBps": contig["GBps"],
                           "mismatched_elements": contig["mismatched_elements"]},
            "frag_over_contig": round(contig["kernel_us"] / cold["kernel_us"], 4)}


def bench_write_cold(v2, args, stream, pool, storage, rng, sets: int = 16):
    """The write with its working set rotated through `sets` distinct
    (K_new, V_new, slots) triples, 16 x 33.6 MB = 537 MB in all: more than
    the 256 MB Infinity Cache, so every launch reads inputs and writes pages
    that no earlier launch of the cycle touched. Each set is 256 sequences of
    16 new tokens at a prefix length ~ U[0, 64) (uniform in-page offsets),
    on pages no other set uses, in the pool's allocation order."""
    from kvflux_amd import capi, device
    from oracle import oracle

    N_SEQ, NEW, H, D, bs = 256, 16, 8, 128, 16
    n = N_SEQ * NEW * H * D
    lib = capi.lib()
    kb, vb = storage.key_base(), storage.value_base()
    bufs, seqs = [], []
    for j in range(sets):
        writes = []
        for i, L0 in enumerate(rng.integers(0, 64, N_SEQ).tolist()):
            s = v2.SequenceState(10**6 + j * N_SEQ + i, pool)
            s.append_tokens(L0 + NEW)
            seqs.append(s)
            writes += [(s, L0 + t) for t in range(NEW)]
        slots = np.array(v2.build_slot_mapping(writes), np.uint64)
        kn, vn = device.DeviceBuffer(n * 2), device.DeviceBuffer(n * 2)
        device.fill_random(kn.ptr, n, capi.DTYPE_BF16, 1, args.seed + 100 + 2 * j)
        device.fill_random(vn.ptr, n, capi.DTYPE_BF16, 1, args.seed + 101 + 2 * j)
        bufs.append((kn, vn, device.to_device(slots), slots))
    device.synchronize()
    cycle = [0]

    def launch():
        kn, vn, sd, _ = bufs[cycle[0] % sets]
        cycle[0] += 1
        capi.check(lib.kvflux_write_paged_kv(kb, vb, pool.capacity(), H, bs, D, capi.DTYPE_BF16,
                                             kn.ptr, vn.ptr, sd.ptr, N_SEQ * NEW, stream))

    ms = time_launches(launch, stream, sets, sets * max(4, args.steps // 4))
    # Every set's pages hold that set's rows: check two sets bit-exactly.
    page_elems = H * bs * D
    mism = 0
    for j in (0, sets - 1):
        kn, vn, _, slots = bufs[j]
        pages = np.unique(slots // bs)
        remap = {int(p): i for i, p in enumerate(pages.tolist())}
        local = np.array([remap[int(s // bs)] * bs + int(s % bs) for s in slots], np.uint64)
        host_k = np.concatenate([device.memcpy_d2h(kb + int(p) * page_elems * 2, page_elems * 2, np.uint16)
                                 for p in pages])
        host_v = np.concatenate([device.memcpy_d2h(vb + int(p) * page_elems * 2, page_elems * 2, np.uint16)
                                 for p in pages])
        exp_k, exp_v = host_k.copy(), host_v.copy()
        oracle.write_paged_kv(exp_k, exp_v, H, bs, D, oracle.BF16, kn.download(np.uint16), vn.download(np.uint16),
                              local)
        mism += int((exp_k != host_k).sum() + (exp_v != host_v).sum())
    del seqs
    bytes_step = 2 * 2 * N_SEQ * NEW * H * D * 2 + N_SEQ * NEW * 8
    return {"kernel_us": ms * 1e3, "GBps": bytes_step / (ms * 1e-3) / 1e9, "sets": sets,
            "working_set_bytes": sets * bytes_step, "sets_checked": 2, "mismatched_elements": mism,
            "pct_of_peak": round(100 * bytes_step / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 2)}


# --------------------------------------------------------------------- gather
def bench_gather(v2, args, stream, dtype_name: str):
    from kvflux_amd import capi, device
    from oracle import oracle

    S, H, D, bs = 64, 8, 128, 16
    code = capi.DTYPE_F16 if dtype_name == "Float16" else capi.DTYPE_BF16
    rng = np.random.default_rng(args.seed + 20)
    lens = rng.integers(512, 8192 + 1, S)
    pool = v2.PhysicalBlockPool(65536, bs)
    storage = v2.PagedKVStorage(pool, H, D, getattr(v2.DType, dtype_name))
    odd = np.arange(1, pool.capacity(), 2)
    fragment_pool(pool, rng.permutation(odd))
    seqs = []
    for i, L in enumerate(lens.tolist()):
        s = v2.SequenceState(i, pool)
        s.append_tokens(L)
        seqs.append(s)
    t = v2.build_batch_block_table(seqs)
    flat = np.array(t.block_table(), np.uint64)
    width = t.max_blocks_per_sequence()
    assert all(int(p) % 2 == 1 for p in flat if p < 2**63)
    n_elems = storage.layout().cache_bytes() // 2
    device.fill_random(storage.key_base(), n_elems, code, 1, args.seed + 21)
    device.fill_random(storage.value_base(), n_elems, code, 1, args.seed + 22)
    total = int(lens.sum())
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.uint64)
    out_bytes = total * H * D * 2
    ko, vo = device.DeviceBuffer(out_bytes), device.DeviceBuffer(out_bytes)
    td, ld, od = device.to_device(flat), device.to_device(lens.astype(np.uint64)), device.to_device(offs)
    device.synchronize()
    lib = capi.lib()
    kb, vb = storage.key_base(), storage.value_base()
    max_len = int(lens.max())
    counts = (lens + bs - 1) // bs
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.uint64)
    sd = device.to_device(starts)
    pages = int(counts.sum())
    device.synchronize()

    def launch():  # one workgroup per live page (the C++ API's launch)
        capi.check(lib.kvflux_gather_paged_kv_live(kb, vb, pool.capacity(), H, bs, D, code, td.ptr, width, ld.ptr,
                                                   od.ptr, sd.ptr, S, pages, ko.ptr, vo.ptr, stream))

    def launch_table():  # table-only form: (logical page x part, sequence) grid
        capi.check(lib.kvflux_gather_paged_kv(kb, vb, pool.capacity(), H, bs, D, code, td.ptr, width,
                                              ld.ptr, od.ptr, S, max_len, ko.ptr, vo.ptr, stream))

    ms_table = time_launches(launch_table, stream, args.warmup, args.steps)
    ms = time_launches(launch, stream, args.warmup, args.steps)
    # Ceilings in the same run. (1) A plain streaming copy of the same byte
    # count (no page table, contiguous, the probe's best shape: one 16-byte
    # vector per thread, 512 threads, one-shot grid, non-temporal), K and V.
    # (2) An independent copy of the same fragmented source pages into a
    # contiguous buffer (kvflux_copy_page_list, no transposition), K and V.
    out_bytes = total * H * D * 2
    cbytes = out_bytes // 8192 * 8192

    def plain_copy():
        capi.check(lib.kvflux_bandwidth_probe(0, ko.ptr, kb, cbytes, 512, 1, 0, 1, stream))
        capi.check(lib.kvflux_bandwidth_probe(0, vo.ptr, vb, cbytes, 512, 1, 0, 1, stream))

    page_bytes = H * bs * D * 2
    list_dev = device.to_device(np.concatenate([flat.reshape(S, width)[r, :int(counts[r])] for r in range(S)]))
    stage_k, stage_v = device.DeviceBuffer(pages * page_bytes), device.DeviceBuffer(pages * page_bytes)

    def page_copy():
        capi.check(lib.kvflux_copy_page_list(stage_k.ptr, kb, pool.capacity(), page_bytes, list_dev.ptr, pages,
                                             stream))
        capi.check(lib.kvflux_copy_page_list(stage_v.ptr, vb, pool.capacity(), page_bytes, list_dev.ptr, pages,
                                             stream))

    ms_copy = time_launches(plain_copy, stream, args.warmup, args.steps)
    ms_pages = time_launches(page_copy, stream, args.warmup, args.steps)
    del stage_k, stage_v
    launch()
    device.synchronize(stream)
    # The synchronous C++ API on the same batch (validation, metadata upload,
    # one launch, stream synchronisation).
    v2.read_paged_kv_batch(storage, seqs, ko.ptr, vo.ptr)
    api_us = v2.timing.read_paged_kv_batch(storage, seqs, ko.ptr, vo.ptr, 10) * 1e6
    # Bit-exact check of a few sequences against the oracle gather.
    page_elems = H * bs * D
    mism = 0
    mat = flat.reshape(S, width)
    for r in (0, S // 2, S - 1):
        L = int(lens[r])
        npg = (L + bs - 1) // bs
        kc = np.concatenate([device.memcpy_d2h(kb + int(p) * page_elems * 2, page_elems * 2, np.uint16)
                             for p in mat[r, :npg]])
        vc = np.concatenate([device.memcpy_d2h(vb + int(p) * page_elems * 2, page_elems * 2, np.uint16)
                             for p in mat[r, :npg]])
        ek, ev = oracle.gather_paged_kv(kc, vc, H, bs, D, code, np.arange(npg, dtype=np.uint64), L)
        gk = device.memcpy_d2h(ko.ptr + int(offs[r]) * H * D * 2, L * H * D * 2, np.uint16)
        gv = device.memcpy_d2h(vo.ptr + int(offs[r]) * H * D * 2, L * H * D * 2, np.uint16)
        mism += int((gk != ek).sum() + (gv != ev).sum())
    bytes_step = 8192 * total + 8 * pages
    gbps = bytes_step / (ms * 1e-3) / 1e9
    copy_gbps = 4 * cbytes / (ms_copy * 1e-3) / 1e9
    pages_gbps = 4 * pages * page_bytes / (ms_pages * 1e-3) / 1e9
    out = {"dtype": dtype_name, "kernel_us": ms * 1e3, "GBps": gbps, "bytes": bytes_step,
           "kernel": "paged_kv_gather_live_kernel (kvflux_gather_paged_kv_live: one workgroup per live page)",
           "table_launch": {"kernel_us": ms_table * 1e3, "GBps": bytes_step / (ms_table * 1e-3) / 1e9,
                            "kernel": "paged_kv_gather_kernel (kvflux_gather_paged_kv)"},
           "ceilings": {"plain_copy_same_bytes": {"kernel_us": ms_copy * 1e3, "GBps": copy_gbps,
                                                  "bytes": 4 * cbytes,
                                                  "kernel": "kvflux_bandwidth_probe copy, 512 threads x 1 vector, "
                                                            "one-shot grid, non-temporal (K and V)"},
                        "page_copy_same_source_pages": {"kernel_us": ms_pages * 1e3, "GBps": pages_gbps,
                                                        "bytes": 4 * pages * page_bytes,
                                                        "kernel": "kvflux_copy_page_list (K and V)"},
                        "frac_of_plain_copy": round(gbps / copy_gbps, 4),
                        "frac_of_page_copy": round(gbps / pages_gbps, 4)},
           "api_us": api_us, "tokens": total, "pages": pages, "mismatched_elements_sampled": mism}
    if dtype_name == "BFloat16":
        out["cpu_baseline"] = cpu_gather_baseline(kb, vb, mat, lens, H, bs, D, code, rng)
    del seqs
    return out


def cpu_gather_baseline(kb, vb, mat, lens, H, bs, D, code, rng, sample_rows=16):
    """The CPU oracle's gather (one thread) on a bounded sample of the
    gather batch: the sampled sequences' pages copied to a host cache in a
    shuffled order (so the CPU reads scattered pages too), then every
    sampled sequence gathered; throughput in the GPU figure's bytes."""
    from kvflux_amd import device
    from oracle import oracle

    rows = sorted(rng.choice(len(lens), sample_rows, replace=False).tolist())
    page_elems = H * bs * D
    npgs = [(int(lens[r]) + bs - 1) // bs for r in rows]
    order = rng.permutation(sum(npgs))
    kc = np.empty(sum(npgs) * page_elems, np.uint16)
    vc = np.empty_like(kc)
    tables, slot = [], 0
    for r, npg in zip(rows, npgs):
        t = order[slot:slot + npg].astype(np.uint64)
        for j, dst in enumerate(t.tolist()):
            src = int(mat[r, j]) * page_elems * 2
            kc[dst * page_elems:(dst + 1) * page_elems] = device.memcpy_d2h(kb + src, page_elems * 2, np.uint16)
            vc[dst * page_elems:(dst + 1) * page_elems] = device.memcpy_d2h(vb + src, page_elems * 2, np.uint16)
        tables.append(t)
        slot += npg
    reps = 0
    t0 = time.perf_counter()
    while reps < 3 or time.perf_counter() - t0 < 2.0:  # about 2 s of gathering
        for r, t in zip(rows, tables):
            oracle.gather_paged_kv(kc, vc, H, bs, D, code, t, int(lens[r]))
        reps += 1
    sec = (time.perf_counter() - t0) / reps
    tokens = int(sum(int(lens[r]) for r in rows))
    moved = 8192 * tokens + 8 * sum(npgs)
    return {"value": moved / sec / 1e9, "unit": "GB/s", "cores": 1, "kind": "port", "seconds": sec,
            "repetitions": reps,
            "sample": f"{sample_rows} of the 64 sequences ({tokens} tokens, {moved / 1e9:.3f} GB moved), pages "
                      "in a shuffled host cache, one thread, averaged over the repetitions"}


# --------------------------------------------------------------------- prefill
def bench_prefill(v2, args, stream):
    from kvflux_amd import capi, device
    from oracle import oracle

    S, T, H, Hq, D, bs = 8, 4096, 8, 32, 128, 16
    rng = np.random.default_rng(args.seed + 30)
    pool = v2.PhysicalBlockPool(S * T // bs + 256, bs)
    storage = v2.PagedKVStorage(pool, H, D, v2.DType.BFloat16)
    fragment_pool(pool, rng.permutation(pool.capacity()))
    seqs, tables, qs = [], [], []
    kn, vn = device.DeviceBuffer(T * H * D * 2), device.DeviceBuffer(T * H * D * 2)
    for i in range(S):
        s = v2.SequenceState(i, pool)
        s.append_tokens(T)
        seqs.append(s)
        device.fill_random(kn.ptr, T * H * D, capi.DTYPE_BF16, 1, args.seed + 31 + 2 * i)
        device.fill_random(vn.ptr, T * H * D, capi.DTYPE_BF16, 1, args.seed + 32 + 2 * i)
        v2.write_paged_kv(storage, kn.ptr, vn.ptr, v2.build_slot_mapping([(s, t) for t in range(T)]))
        tables.append(device.to_device(np.array(v2.build_read_block_table(s), np.uint64)))
        q = device.DeviceBuffer(T * Hq * D * 4)
        device.fill_random(q.ptr, T * Hq * D, capi.DTYPE_F32, 1, args.seed + 50 + i)
        qs.append(q)
    out = device.DeviceBuffer(S * T * Hq * D * 4)
    lib = capi.lib()
    kb, vb = storage.key_base(), storage.value_base()
    npages = T // bs
    # One batch launch over the 8 sequences: Q of all sequences in one
    # buffer, their tables as the rows of one batch table.
    q_all = device.DeviceBuffer(S * T * Hq * D * 4)
    for i in range(S):
        capi.call("kvflux_memcpy_async", C.c_void_p(q_all.ptr + i * T * Hq * D * 4), C.c_void_p(qs[i].ptr),
                  T * Hq * D * 4, None)
    batch_table = device.to_device(np.concatenate([np.array(v2.build_read_block_table(s), np.uint64) for s in seqs]))
    kv_lens = device.to_device(np.full(S, T, np.uint64))
    q_offs = device.to_device((np.arange(S) * T).astype(np.uint64))
    device.synchronize()

    def launch():
        capi.check(lib.kvflux_paged_prefill_batch(kb, vb, pool.capacity(), H, bs, D, capi.DTYPE_BF16, batch_table.ptr,
                                                  npages, kv_lens.ptr, kv_lens.ptr, q_offs.ptr, S, T, T, Hq,
                                                  q_all.ptr, out.ptr, stream))

    def per_sequence():
        for i in range(S):
            capi.check(lib.kvflux_paged_prefill(kb, vb, pool.capacity(), H, bs, D, capi.DTYPE_BF16, tables[i].ptr,
                                                npages, T, T, Hq, qs[i].ptr, out.ptr + i * T * Hq * D * 4, stream))

    # The reference's arithmetic contract (1e-5): the exact variant, one
    # launch per sequence, into its own output.
    out_exact = device.DeviceBuffer(S * T * Hq * D * 4)

    def per_sequence_exact():
        for i in range(S):
            capi.check(lib.kvflux_paged_prefill_exact(kb, vb, pool.capacity(), H, bs, D, capi.DTYPE_BF16,
                                                      tables[i].ptr, npages, T, T, Hq, qs[i].ptr,
                                                      out_exact.ptr + i * T * Hq * D * 4, None, 0, stream))

    # FP32 caches holding the same values (BF16 widened exactly), one batch
    # launch on FP32 MFMAs; the same oracle rows apply.
    cache_bytes = storage.layout().cache_bytes()
    k32 = device.to_device((device.memcpy_d2h(kb, cache_bytes, np.uint16).astype(np.uint32) << 16).view(np.float32))
    v32 = device.to_device((device.memcpy_d2h(vb, cache_bytes, np.uint16).astype(np.uint32) << 16).view(np.float32))
    out_f32 = device.DeviceBuffer(S * T * Hq * D * 4)

    def launch_f32():
        capi.check(lib.kvflux_paged_prefill_batch(k32.ptr, v32.ptr, pool.capacity(), H, bs, D, capi.DTYPE_F32,
                                                  batch_table.ptr, npages, kv_lens.ptr, kv_lens.ptr, q_offs.ptr, S, T,
                                                  T, Hq, q_all.ptr, out_f32.ptr, stream))

    per_seq_ms = time_launches(per_sequence, stream, max(1, args.warmup // 2), max(3, args.steps // 4))
    exact_ms = time_launches(per_sequence_exact, stream, 1, max(3, args.steps // 4))
    f32_ms = time_launches(launch_f32, stream, 1, max(3, args.steps // 4))
    ms = time_launches(launch, stream, max(1, args.warmup // 2), max(3, args.steps // 4))
    # The synchronous C++ API (paged_attention with AttentionPrecision::Fast,
    # one call per sequence) on the same inputs.
    api_ms = v2.timing.paged_attention(storage, seqs, [qs[i].ptr for i in range(S)],
                                       [out.ptr + i * T * Hq * D * 4 for i in range(S)], Hq,
                                       v2.AttentionPrecision.Fast, 3) * 1e3
    flops = S * T * (T + 1) / 2 * Hq * D * 4
    # 16 rows of every sequence (first and last tokens, tile and page
    # boundaries, a seeded sample) against the CPU reference.
    page_bytes = H * bs * D * 2
    err = 0.0
    err_exact = 0.0
    err_f32 = 0.0
    checked = 0
    cpu_s, cpu_flops = 0.0, 0.0
    local = np.arange(npages, dtype=np.uint64)
    for i in range(S):
        ids = device.memcpy_d2h(tables[i].ptr, npages * 8, np.uint64)
        kc = np.concatenate([device.memcpy_d2h(kb + int(p) * page_bytes, page_bytes, np.uint16) for p in ids])
        vc = np.concatenate([device.memcpy_d2h(vb + int(p) * page_bytes, page_bytes, np.uint16) for p in ids])
        rows = sorted({0, 63, 64, 1000, 2047, 2048, 4094, 4095} | set(rng.integers(0, T, 8).tolist()))
        qall = device.memcpy_d2h(qs[i].ptr, T * Hq * D * 4, np.float32).reshape(T, Hq * D)
        oall = device.memcpy_d2h(out.ptr + i * T * Hq * D * 4, T * Hq * D * 4, np.float32).reshape(T, Hq * D)
        t0 = time.perf_counter()
        ref = oracle.paged_attention_rows(kc, vc, H, bs, D, oracle.BF16, np.tile(local, len(rows)), npages,
                                          np.array([t + 1 for t in rows], np.uint64), qall[rows].reshape(-1), Hq,
                                          threads=8)
        cpu_s += time.perf_counter() - t0
        cpu_flops += sum(4.0 * Hq * D * (t + 1) for t in rows)
        err = max(err, float(np.abs(oall[rows].reshape(-1) - ref).max()))
        oex = device.memcpy_d2h(out_exact.ptr + i * T * Hq * D * 4, T * Hq * D * 4, np.float32).reshape(T, Hq * D)
        err_exact = max(err_exact, float(np.abs(oex[rows].reshape(-1) - ref).max()))
        of32 = device.memcpy_d2h(out_f32.ptr + i * T * Hq * D * 4, T * Hq * D * 4, np.float32).reshape(T, Hq * D)
        err_f32 = max(err_f32, float(np.abs(of32[rows].reshape(-1) - ref).max()))
        checked += len(rows)
    del seqs
    tflops = flops / (ms * 1e-3) / 1e12
    return {"workload": "8 x 4096-token causal prefill, 32 q / 8 kv heads, D=128, BF16 KV, block_size 16",
            "kernel": "paged_prefill_kernel<bf16,128> (group 4), one batch launch (kvflux_paged_prefill_batch)",
            "ms": ms, "ms_one_launch_per_sequence": per_seq_ms, "api_ms": api_ms, "TFLOPs": tflops,
            "mfma_util_pct": 100.0 * tflops / PEAK_BF16_TFLOPS, "flops": flops,
            # Counter-derived: busy cycles at the clock the part ran (about
            # 2.05 GHz under this load), so above the FLOP share of the 2.4 GHz
            # spec peak above.
            "mfma_busy_pct": read_prefill_busy(), "mfma_busy_source": "profiles/prefill_counters.txt",
            "max_abs_err_vs_oracle": err, "rows_checked": checked, "tolerance": 2e-2,
            # The exact variant (kvflux_paged_prefill_exact: Q and weights as
            # three 16-bit parts), one launch per sequence, at the
            # reference's 1e-5 bound on the same checked rows.
            "exact": {"ms": exact_ms, "TFLOPs": flops / (exact_ms * 1e-3) / 1e12,
                      "max_abs_err_vs_oracle": err_exact, "tolerance": 1e-5},
            # FP32 caches (the same values): one batch launch on
            # v_mfma_f32_16x16x4_f32, against the FP32 MFMA peak.
            "f32": {"kernel": "paged_prefill_kernel<f32,128> (group 4), one batch launch", "ms": f32_ms,
                    "TFLOPs": flops / (f32_ms * 1e-3) / 1e12,
                    "frac_of_fp32_mfma_peak": flops / (f32_ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS,
                    "max_abs_err_vs_oracle": err_f32, "tolerance": 1e-5},
            # The checked rows' oracle calls, timed: causal attention of each
            # row in double precision after a page gather, on 8 threads.
            "cpu_baseline": {"value": cpu_flops / cpu_s / 1e12, "unit": "TFLOP/s", "cores": 8, "kind": "port",
                             "seconds": cpu_s,
                             "sample": f"{checked} rows (16 of each sequence, all 32 query heads): page gather + "
                                       "double-precision causal attention per row"}}


def bench_ceilings(v2, args, stream):
    """HBM ceilings of this part, with no page table: kvflux_bandwidth_probe
    (plain streaming copy, write-only, read-only over one contiguous 1 GiB
    range) swept over threads per workgroup {256, 512, 1024}, 16-byte vectors
    per thread {1, 2, 4, 8}, grid {one workgroup per step, 1024, 4096
    walking the steps} and plain / non-temporal accesses; the runtime's
    device copy beside it; and a cold copy of the KV write's bytes (16
    rotated sets of 16 MiB -> 16 MiB, 537 MB in all, one launch per set).
    `best` holds the fastest shape of each operation."""
    from kvflux_amd import capi, device

    lib = capi.lib()
    n = 1 << 30
    a, b = device.DeviceBuffer(n), device.DeviceBuffer(n)
    device.fill_random(a.ptr, n // 2, capi.DTYPE_BF16, 0, 7)
    b.fill(0)
    device.synchronize()
    rows, best = [], {}
    for op, name in ((0, "copy"), (1, "write"), (2, "read")):
        for threads in (256, 512, 1024):
            for vpt in (1, 2, 4, 8):
                for grid in (0, 1024, 4096):
                    for nt in (0, 1):
                        def run(op=op, threads=threads, vpt=vpt, grid=grid, nt=nt):
                            capi.check(lib.kvflux_bandwidth_probe(op, b.ptr, a.ptr, n, threads, vpt, grid, nt, stream))
                        ms = time_launches(run, stream, 2, max(5, args.steps // 4))
                        moved = 2 * n if op == 0 else n
                        gbps = moved / (ms * 1e-3) / 1e9
                        rows.append([name, threads, vpt, grid, nt, round(ms * 1e3, 2), round(gbps, 1)])
                        if name not in best or gbps > best[name]["GBps"]:
                            best[name] = {"GBps": round(gbps, 1), "us": round(ms * 1e3, 2), "threads": threads,
                                          "vectors_per_thread": vpt, "grid": grid, "nontemporal": nt,
                                          "bytes": moved, "pct_of_peak": round(100 * gbps / PEAK_HBM_GBPS, 2)}
    log(f"ceilings best {best}")

    def d2d():
        capi.call("kvflux_memcpy_async", C.c_void_p(b.ptr), C.c_void_p(a.ptr), n, C.c_void_p(stream))

    ms = time_launches(d2d, stream, args.warmup, args.steps)
    runtime_copy = {"us": round(ms * 1e3, 2), "GBps": round(2 * n / (ms * 1e-3) / 1e9, 1), "bytes": 2 * n}
    del a, b
    # The KV write's bytes (4096 tokens x 8 heads x 128 BF16, K and V: 16 MiB
    # read, 16 MiB written), cold: 16 rotated source/destination pairs.
    sets, m = 16, 16 << 20
    bufs = [(device.DeviceBuffer(m), device.DeviceBuffer(m)) for _ in range(sets)]
    for j, (src, _) in enumerate(bufs):
        device.fill_random(src.ptr, m // 2, capi.DTYPE_BF16, 0, 100 + j)
    device.synchronize()
    cold = {}
    for threads, vpt, nt in ((512, 1, 1), (256, 4, 1), (1024, 1, 1), (512, 2, 0)):
        cycle = [0]

        def small(threads=threads, vpt=vpt, nt=nt):
            src, dst = bufs[cycle[0] % sets]
            cycle[0] += 1
            capi.check(lib.kvflux_bandwidth_probe(0, dst.ptr, src.ptr, m, threads, vpt, 0, nt, stream))

        ms = time_launches(small, stream, sets, sets * max(4, args.steps // 4))
        cold[f"{threads}x{vpt}{' nt' if nt else ''}"] = {"us": round(ms * 1e3, 3),
                                                         "GBps": round(2 * m / (ms * 1e-3) / 1e9, 1)}
    del bufs
    top = max(cold.values(), key=lambda v: v["GBps"])
    return {"best": best, "runtime_copy": runtime_copy,
            "write_sized_copy_cold": {"shapes": cold, "best_GBps": top["GBps"], "best_us": top["us"],
                                      "bytes": 2 * m, "sets": sets},
            "sweep_columns": ["op", "threads", "vectors_per_thread", "grid", "nontemporal", "us", "GBps"],
            "sweep": rows}


def calibrate_copy(args) -> int:
    """A plain 1 GiB device-to-device copy (the runtime's copy kernel), run
    under rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE to scale those counters."""
    from kvflux_amd import capi, device
    capi.call("kvflux_set_device", 0)
    n = 1 << 30
    a, b = device.DeviceBuffer(n), device.DeviceBuffer(n)
    a.fill(1)
    b.fill(0)
    device.synchronize()
    for _ in range(5):
        capi.call("kvflux_memcpy_async", C.c_void_p(b.ptr), C.c_void_p(a.ptr), n, None)
    device.synchronize()
    print(json.dumps({"calibration": "device copy", "bytes_read_per_dispatch": n, "bytes_written_per_dispatch": n}))
    return 0


def read_prefill_busy():
    """MFMA-busy share of the batch prefill launch (rocprofv3 MfmaUtil:
    SQ_VALU_MFMA_BUSY_CYCLES over GPU-active cycles x SIMDs) from the
    committed counter summary, or None."""
    if not PREFILL_COUNTERS.exists():
        return None
    for line in PREFILL_COUNTERS.read_text().splitlines():
        if line.startswith("batch_MfmaUtil_pct:"):
            try:
                return float(line.split(":", 1)[1].split()[0])
            except (ValueError, IndexError):
                return None
    return None


def read_traffic():
    """HBM bytes per decode call from the committed rocprofv3 summary, or None."""
    if not TRAFFIC_SUMMARY.exists():
        return None
    vals = {}
    for line in TRAFFIC_SUMMARY.read_text().splitlines():
        if ":" in line and not line.startswith("#"):
            k, v = line.split(":", 1)
            try:
                vals[k.strip()] = float(v.split()[0])
            except (ValueError, IndexError):
                pass
    need = ("decode_fetch_kib_per_call", "decode_write_kib_per_call", "copy_fetch_kib_per_gib", "copy_write_kib_per_gib")
    if not all(k in vals for k in need):
        return None
    fetch = vals["decode_fetch_kib_per_call"] * (1 << 30) / vals["copy_fetch_kib_per_gib"]
    write = vals["decode_write_kib_per_call"] * (1 << 30) / vals["copy_write_kib_per_gib"]
    return int(fetch + write)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--seed", type=int, default=2024)
    ap.add_argument("--cpu-rows", type=int, default=24, help="decode rows timed on the CPU oracle")
    ap.add_argument("--skip-aux", action="store_true", help="decode only")
    ap.add_argument("--block-size", type=int, default=16, help="page size of the decode batch (16 is the benchmark)")
    ap.add_argument("--only", choices=("write", "gather", "prefill", "cow", "cow_placement", "ceilings"),
                    help="run one auxiliary leg alone and print its JSON object (for profiling runs)")
    ap.add_argument("--calibrate-copy", action="store_true", help="1 GiB device copy for counter scaling")
    args = ap.parse_args()
    if args.calibrate_copy:
        return calibrate_copy(args)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}); run with --gpus 1.", file=sys.stderr)
        return 2
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py runs as a single process on one GPU", file=sys.stderr)
        return 2

    import kvflux_amd
    from kvflux_amd import capi, device

    v2 = kvflux_amd.v2
    if capi.device_count() < 1:
        print("no GPU visible", file=sys.stderr)
        return 1
    capi.call("kvflux_set_device", 0)
    stream = device.Stream()

    if args.only:
        legs = {"write": lambda: bench_write(v2, args, stream.handle),
                "gather": lambda: bench_gather(v2, args, stream.handle, "BFloat16"),
                "prefill": lambda: bench_prefill(v2, args, stream.handle),
                "cow": lambda: bench_cow(v2, args, stream.handle),
                "cow_placement": lambda: bench_cow_placement(v2, args, stream.handle),
                "ceilings": lambda: bench_ceilings(v2, args, stream.handle)}
        log(f"{args.only} ...")
        print(json.dumps({args.only: legs[args.only]()}))
        return 0

    log("decode ...")
    dec = bench_decode(v2, args, stream.handle)
    log(f"decode {dec['ms']:.3f} ms, err {dec['max_abs_err']:.2e}")
    aux = {}
    if not args.skip_aux:
        log("write ...")
        aux["write"] = bench_write(v2, args, stream.handle)
        log(f"write {aux['write']}")
        for name in ("BFloat16", "Float16"):
            log(f"gather {name} ...")
            aux[f"gather_{name}"] = bench_gather(v2, args, stream.handle, name)
            log(f"gather {aux[f'gather_{name}']}")
        log("prefill ...")
        aux["prefill"] = bench_prefill(v2, args, stream.handle)
        log(f"prefill {aux['prefill']}")
        log("copy-on-write ...")
        aux["cow"] = bench_cow(v2, args, stream.handle)
        log(f"cow {aux['cow']}")
        aux["decode_step"] = dec["decode_step"]
        aux["offload"] = dec["offload"]
        for key in ("write", "gather_BFloat16", "gather_Float16", "cow"):
            aux[key]["pct_of_peak"] = round(100 * aux[key]["GBps"] / PEAK_HBM_GBPS, 2)

    s = dec["ms"] * 1e-3
    achieved = dec["unique_bytes"] / s / 1e9
    line = {
        "metric": METRIC,
        "value": round(dec["unique_bytes"] / s / 1e12, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 KV, fp32 math",
        "data": "synthetic (counter-based N(0,1) generator, seeded)",
        "config": {
            "workload": "batch GQA decode PagedAttention: B=128, seq_len U[1024,32768], 32 q / 8 kv heads, "
                        "head_size 128, block_size 16, BF16 KV, FP32 Q/O, 2048-token shared prefix, "
                        "2^18-page pool",
            "seed": args.seed,
            "sum_seq_len": dec["sum_len"],
        },
        "pct_of_peak": round(100 * achieved / PEAK_HBM_GBPS, 2),
        "logical_TBps": round(dec["logical_bytes"] / s / 1e12, 4),
        "tokens_per_s": round(128 / s, 1),
        "decode_max_abs_err_vs_oracle": dec["max_abs_err"],
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4),
            "traffic": read_traffic(),
            "kernel": "paged_decode_bs16_kernel<Bf16,128,4> (+ paged_attention_combine_kernel, "
                      "both inside the timed kvflux_paged_attention call)",
            "bytes_per_launch": dec["unique_bytes"],
        },
        "cpu_baseline": dec["cpu"],
        "decode_read_ceiling": {
            "ms": round(dec["read_ceiling"]["ms"], 4),
            "TBps": round(dec["read_ceiling"]["TBps"], 4),
            "bytes": dec["read_ceiling"]["bytes"],
            "kernel": dec["read_ceiling"]["kernel"],
            "what": "every unique page of the batch (K and V) read once, in the order the rows meet them",
            "decode_frac_of_ceiling": round(dec["unique_bytes"] / (dec["ms"] * 1e-3) / 1e12
                                            / dec["read_ceiling"]["TBps"], 4),
        },
        "decode_contiguous": {
            "ms": round(dec["ms_contiguous"], 4),
            "TBps": round(dec["unique_bytes"] / (dec["ms_contiguous"] * 1e-3) / 1e12, 4),
            "frag_over_contig": round(dec["ms_contiguous"] / dec["ms"], 4),
            "layout": "same lengths and shared prefix; each row's own pages consecutive",
        },
    }
    for k, v in aux.items():
        line[k] = v
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
