#pragma once
// GPU <-> CPU chunk migration (KV offload / onload). Same public surface and
// directory protocol as the reference's include/kvflux/v3/gpu_cpu_transfer.h:13-57
// (src/v3/gpu_cpu_transfer.cpp:32-136): while a transfer is in flight both
// replicas are non-READY and the chunk is pinned, so the directory refuses to
// drop either; finish_* waits for the transfer, marks the destination READY
// and optionally releases the source. Transfers run on this object's own
// non-blocking stream, so they overlap compute on other streams.
//
// Addition (no counterpart in the reference): the batch forms move every
// chunk of a batch in one kernel launch (kvflux_copy_chunks), reading and
// writing the pinned host slots directly, instead of one DMA copy per chunk.

#include "kvflux/v3/cache_directory.h"
#include "kvflux/v3/gpu_chunk_store.h"
#include "kvflux/v3/host_buffers.h"

#include <cstddef>
#include <memory>
#include <unordered_map>
#include <vector>

namespace kvflux::v3 {

class PinnedChunkPool;

class GpuCpuTransfer {
public:
    // The directory's GPU and CPU tiers must match the two stores' slot
    // layouts; all referenced objects must outlive this one.
    // std::invalid_argument when the chunk sizes differ.
    GpuCpuTransfer(CacheDirectory& directory, GpuChunkStore& gpu_store,
                   HostChunkBuffers& cpu_buffers, int device = 0);
    ~GpuCpuTransfer() noexcept;
    GpuCpuTransfer(const GpuCpuTransfer&) = delete;
    GpuCpuTransfer& operator=(const GpuCpuTransfer&) = delete;

    // GPU -> CPU. Requires a READY GPU replica and no CPU replica
    // (std::logic_error otherwise). Both replicas become COPYING and the
    // chunk is pinned; the GPU bytes must not change until finish.
    void begin_offload(const CacheKey& key);
    // Waits; the CPU replica becomes READY; release_gpu drops the GPU replica,
    // otherwise it returns to READY.
    void finish_offload(const CacheKey& key, bool release_gpu);

    // CPU -> GPU. Requires a READY CPU replica and no GPU replica.
    void begin_onload(const CacheKey& key);
    void finish_onload(const CacheKey& key, bool release_cpu);

    bool has_pending(const CacheKey& key) const;

    // Batch forms: every key is checked as by the single-key call before any
    // state changes; then all chunks move in one launch when the host buffers
    // are a PinnedChunkPool (one DMA copy per chunk otherwise). Keys are
    // finished one by one with finish_offload / finish_onload.
    void begin_offload(const std::vector<CacheKey>& keys);
    void begin_onload(const std::vector<CacheKey>& keys);

    // The transfer stream (a hipStream_t), for ordering other work after it.
    void* stream() const noexcept { return stream_; }

private:
    struct Batch;  // completion event (+ the batch's address pairs)
    // One chunk in flight: the tier its copy lands in (CPU for an offload,
    // GPU for an onload), the two replica slots begin() set up, and the
    // batch whose completion event covers the copy.
    struct Ticket {
        StorageTier lands_in;
        TierLocation read_from;
        TierLocation written_to;
        std::shared_ptr<Batch> batch;
    };

    void begin(const std::vector<CacheKey>& keys, bool offload);
    // Takes the chunk's ticket once its copy has completed; std::logic_error
    // when no copy of the chunk is in flight or it lands in the other tier.
    Ticket redeem(const CacheKey& key, StorageTier lands_in);
    // Moves the replicas out of their in-flight states (after checking they
    // are still the ones the ticket names) and drops the source on request.
    void settle(const CacheKey& key, const Ticket& ticket, bool drop_source);
    std::shared_ptr<Batch> acquire_batch(std::size_t pairs);

    CacheDirectory& directory_;
    GpuChunkStore& gpu_store_;
    HostChunkBuffers& cpu_buffers_;
    PinnedChunkPool* mapped_host_;  // cpu_buffers_ when it is mapped pinned memory, else null
    int device_;
    void* stream_ = nullptr;
    // Keyed by the chunk's directory record, whose address is stable while
    // the chunk is pinned (the directory refuses to destroy a pinned chunk).
    std::unordered_map<const ChunkRecord*, Ticket> tickets_;
    std::vector<std::shared_ptr<Batch>> idle_;  // finished batches, reused
};

} // namespace kvflux::v3
