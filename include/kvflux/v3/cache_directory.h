#pragma once
// Directory of the tiered KV cache: the logical identity of every chunk, its
// replica on each tier with that replica's state, reference and pin counts
// and last access. Same public surface as the reference's
// include/kvflux/v3/cache_directory.h:14-125. Replica slots are allocated
// and returned only through the directory. Metadata only; single-threaded.

#include "kvflux/block_manager.h"  // Tokens, BlockManager::prefix_hash
#include "kvflux/kv_layout.h"      // DType
#include "kvflux/v3/tier.h"

#include <chrono>
#include <cstddef>
#include <cstdint>
#include <deque>
#include <optional>
#include <string>
#include <unordered_map>
#include <vector>

namespace kvflux::v3 {

enum class ChunkState { READY, COPYING, LOADING, EVICTING, ERROR };

// Identity of a KV chunk, independent of where it is stored: model, layout
// version, dtype, layer range [first_layer, last_layer) and the token prefix
// (kept verbatim, so equal hashes never alias different prefixes).
struct CacheKey {
    std::string model_id;
    std::uint32_t layout_version = 0;
    DType dtype = DType::Float16;
    std::uint32_t first_layer = 0;
    std::uint32_t last_layer = 0;
    std::uint64_t prefix_hash = 0;
    Tokens prefix;

    bool operator==(const CacheKey& other) const noexcept {
        return model_id == other.model_id && layout_version == other.layout_version &&
               dtype == other.dtype && first_layer == other.first_layer &&
               last_layer == other.last_layer && prefix_hash == other.prefix_hash &&
               prefix == other.prefix;
    }
};

struct CacheKeyHash {
    std::size_t operator()(const CacheKey& key) const noexcept;
};

// Builds a key with prefix_hash computed from `prefix`; std::invalid_argument
// for an empty layer range.
CacheKey make_cache_key(std::string model_id, std::uint32_t layout_version, DType dtype,
                        std::uint32_t first_layer, std::uint32_t last_layer, Tokens prefix);

struct Replica {
    TierLocation location;
    ChunkState state = ChunkState::READY;
};

struct ChunkRecord {
    CacheKey key;
    std::uint64_t version = 1;
    std::size_t ref_count = 0;
    std::size_t pin_count = 0;
    std::chrono::steady_clock::time_point last_access;
    std::optional<Replica> gpu;
    std::optional<Replica> cpu;
    std::optional<Replica> nvme;
};

class CacheDirectory {
public:
    // The tiers must be of kind GPU, CPU and NVME, and outlive the directory.
    CacheDirectory(Tier& gpu, Tier& cpu, Tier& nvme);

    // std::invalid_argument when the key is already registered.
    void create(const CacheKey& key);
    bool contains(const CacheKey& key) const;
    // std::out_of_range for an unknown key (every call below too).
    const ChunkRecord& at(const CacheKey& key) const;
    std::size_t size() const noexcept { return index_.size(); }

    // Allocates a slot on `tier` and records a replica there.
    // std::logic_error if the tier already holds one; CapacityError if full.
    TierLocation place(const CacheKey& key, StorageTier tier, ChunkState state = ChunkState::READY);
    // Returns the replica's slot to its tier. std::logic_error when there is
    // no replica or it is in transfer (only READY or ERROR replicas go).
    void remove(const CacheKey& key, StorageTier tier);
    // std::logic_error when the tier holds no replica.
    void set_state(const CacheKey& key, StorageTier tier, ChunkState state);

    void add_ref(const CacheKey& key);
    void release_ref(const CacheKey& key);
    void pin(const CacheKey& key);
    void unpin(const CacheKey& key);
    void touch(const CacheKey& key);
    // The content changed (moves between tiers keep the version).
    void bump_version(const CacheKey& key);

    std::size_t replica_count(const CacheKey& key) const;

    struct TierStats {
        std::size_t capacity;
        std::size_t available;
        std::size_t allocated_chunks;
        std::size_t used_bytes;
        std::size_t available_bytes;
        std::size_t replicas;  // chunks with a replica on the tier
    };
    TierStats stats(StorageTier tier) const;

    // std::logic_error while replicas, references or pins remain.
    void destroy(const CacheKey& key);

private:
    // Records live in a slab whose addresses never move (at() hands out
    // references); destroyed records leave a vacant entry for the next
    // create(). The index maps a key to its slab entry.
    ChunkRecord& record(const CacheKey& key);
    // Position of `tier` in tiers_ / replicas_ (std::invalid_argument for a
    // value outside the enum).
    static std::size_t tier_index(StorageTier tier);

    Tier* tiers_[3];                 // indexed by StorageTier
    std::size_t replicas_[3] = {};   // records holding a replica on each tier
    std::deque<ChunkRecord> slab_;
    std::vector<std::size_t> vacant_;
    std::unordered_map<CacheKey, std::size_t, CacheKeyHash> index_;
};

} // namespace kvflux::v3
