#pragma once
// Device memory of the GPU tier's chunks: one allocation of
// total_slots * chunk_bytes, slot = PhysicalBlockID of the GpuTier's pool.
// Same public surface as the reference's include/kvflux/v3/gpu_chunk_store.h:11-26.
// Address arithmetic only; slot lifetimes belong to the tier and directory.

#include "kvflux/v3/tier.h"

#include <cstddef>

namespace kvflux::v3 {

class GpuChunkStore {
public:
    GpuChunkStore(std::size_t total_slots, std::size_t chunk_bytes, int device = 0);
    ~GpuChunkStore();
    GpuChunkStore(const GpuChunkStore&) = delete;
    GpuChunkStore& operator=(const GpuChunkStore&) = delete;

    // Device addresses (not dereferenceable on the host). std::out_of_range
    // for a slot past the store; generations are not checked here.
    void* device_ptr(const TierLocation& location) const;
    void* device_ptr(std::size_t slot) const;
    std::size_t chunk_bytes() const noexcept { return chunk_bytes_; }
    std::size_t slots() const noexcept { return slots_; }
    int device() const noexcept { return device_; }

private:
    std::size_t slots_;
    std::size_t chunk_bytes_;
    int device_;
    void* base_ = nullptr;
};

} // namespace kvflux::v3
