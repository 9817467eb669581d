#pragma once
// Host bytes of CPU-tier chunks. The tier holds slot metadata; these classes
// hold the memory. Same public surface as the reference's
// include/kvflux/v3/host_buffers.h:9-37.

#include "kvflux/v3/tier.h"

#include <cstddef>
#include <memory>
#include <vector>

namespace kvflux::v3 {

class HostChunkBuffers {
public:
    virtual ~HostChunkBuffers() = default;

    virtual std::size_t chunk_bytes() const noexcept = 0;
    virtual std::size_t slots() const noexcept = 0;
    // std::invalid_argument for a slot out of range (generations belong to
    // the tier).
    virtual void* data(std::size_t slot) = 0;
    virtual const void* data(std::size_t slot) const = 0;
};

// Pageable heap memory (CPU-only paths and tests).
class HeapChunkPool : public HostChunkBuffers {
public:
    HeapChunkPool(std::size_t slots, std::size_t chunk_bytes);

    std::size_t chunk_bytes() const noexcept override { return chunk_bytes_; }
    std::size_t slots() const noexcept override { return slots_; }
    void* data(std::size_t slot) override;
    const void* data(std::size_t slot) const override;

private:
    std::size_t slots_;
    std::size_t chunk_bytes_;
    std::unique_ptr<unsigned char[]> bytes_;  // slots * chunk_bytes, zero-filled
};

} // namespace kvflux::v3
