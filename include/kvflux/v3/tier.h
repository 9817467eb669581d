#pragma once
// Slot metadata of the three storage tiers of the tiered KV cache: GPU pages,
// pinned host chunks and NVMe file blocks. Same public surface as the
// reference's include/kvflux/v3/tier.h:9-117. Metadata only: no bytes move
// here. Single-threaded, like the v2 control plane.

#include "kvflux/physical_block_pool.h"

#include <cstddef>
#include <cstdint>
#include <vector>

namespace kvflux::v3 {

enum class StorageTier { GPU, CPU, NVME };

// A slot of one tier plus the generation of its current allocation; a
// location kept past its release no longer matches and is rejected.
struct TierLocation {
    std::size_t slot;
    std::uint64_t generation;
    bool operator==(const TierLocation& other) const noexcept {
        return slot == other.slot && generation == other.generation;
    }
};

class Tier {
public:
    virtual ~Tier() = default;

    virtual StorageTier kind() const noexcept = 0;
    virtual std::size_t chunk_bytes() const noexcept = 0;
    virtual std::size_t capacity() const noexcept = 0;
    virtual std::size_t allocated_chunks() const noexcept = 0;
    virtual std::size_t available() const noexcept = 0;
    virtual std::size_t used_bytes() const noexcept = 0;
    virtual std::size_t available_bytes() const noexcept = 0;

    // A live location; CapacityError when the tier is full.
    virtual TierLocation allocate() = 0;
    // std::invalid_argument for a stale, released or out-of-range location.
    virtual void release(const TierLocation& location) = 0;
};

// Fixed-size slots with a LIFO free list (the most recently released slot is
// handed out first) and per-slot generations.
class SlotTier : public Tier {
public:
    SlotTier(StorageTier kind, std::size_t chunk_slots, std::size_t chunk_bytes);

    StorageTier kind() const noexcept override { return kind_; }
    std::size_t chunk_bytes() const noexcept override { return chunk_bytes_; }
    std::size_t capacity() const noexcept override { return generation_.size(); }
    std::size_t allocated_chunks() const noexcept override { return capacity() - free_.size(); }
    std::size_t available() const noexcept override { return free_.size(); }
    std::size_t used_bytes() const noexcept override { return allocated_chunks() * chunk_bytes_; }
    std::size_t available_bytes() const noexcept override { return available() * chunk_bytes_; }

    TierLocation allocate() override;
    void release(const TierLocation& location) override;

private:
    StorageTier kind_;
    std::size_t chunk_bytes_;
    std::vector<std::uint64_t> generation_;  // current generation of each slot
    std::vector<unsigned char> live_;        // 1 while allocated
    std::vector<std::size_t> free_;          // free slots, next allocation at the back
};

class CpuTier : public SlotTier {
public:
    CpuTier(std::size_t chunk_slots, std::size_t chunk_bytes)
        : SlotTier(StorageTier::CPU, chunk_slots, chunk_bytes) {}
};

class NvmeTier : public SlotTier {
public:
    NvmeTier(std::size_t chunk_slots, std::size_t chunk_bytes)
        : SlotTier(StorageTier::NVME, chunk_slots, chunk_bytes) {}
};

// GPU slots are pages of a v2 PhysicalBlockPool: slot = PhysicalBlockID, and
// the pool's handle generation is the location's generation.
class GpuTier : public Tier {
public:
    GpuTier(PhysicalBlockPool& pool, std::size_t chunk_bytes);

    StorageTier kind() const noexcept override { return StorageTier::GPU; }
    std::size_t chunk_bytes() const noexcept override { return chunk_bytes_; }
    std::size_t capacity() const noexcept override;
    std::size_t allocated_chunks() const noexcept override { return allocated_; }
    std::size_t available() const noexcept override;
    std::size_t used_bytes() const noexcept override { return allocated_ * chunk_bytes_; }
    std::size_t available_bytes() const noexcept override { return available() * chunk_bytes_; }

    TierLocation allocate() override;
    void release(const TierLocation& location) override;

private:
    PhysicalBlockPool& pool_;  // outlives the tier
    std::size_t chunk_bytes_;
    std::size_t allocated_ = 0;
};

} // namespace kvflux::v3
