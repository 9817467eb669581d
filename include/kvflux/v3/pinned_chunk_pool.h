#pragma once
// Page-locked host memory for the CPU tier, allocated once (never on the
// transfer path). Same public surface as the reference's
// include/kvflux/v3/pinned_chunk_pool.h:12-26. Here all slots share one
// pinned allocation (slot i at i * chunk_bytes), which is also mapped into
// the GPU's address space, so a batch of chunks can be moved by one kernel.

#include "kvflux/v3/host_buffers.h"

#include <cstddef>

namespace kvflux::v3 {

class PinnedChunkPool : public HostChunkBuffers {
public:
    PinnedChunkPool(std::size_t slots, std::size_t chunk_bytes);
    ~PinnedChunkPool() override;
    PinnedChunkPool(const PinnedChunkPool&) = delete;
    PinnedChunkPool& operator=(const PinnedChunkPool&) = delete;

    std::size_t chunk_bytes() const noexcept override { return chunk_bytes_; }
    std::size_t slots() const noexcept override { return slots_; }
    void* data(std::size_t slot) override;
    const void* data(std::size_t slot) const override;
    // The device-side address of slot `slot` (for kernels; no counterpart in
    // the reference).
    void* device_data(std::size_t slot) const;

private:
    std::size_t slots_;
    std::size_t chunk_bytes_;
    unsigned char* base_ = nullptr;
    unsigned char* device_base_ = nullptr;
};

} // namespace kvflux::v3
