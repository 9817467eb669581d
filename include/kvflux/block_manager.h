#pragma once
// Page-id allocator underneath PhysicalBlockPool.
// Same public surface as the reference's include/kvflux/block_manager.h:14-78:
// LIFO reuse of freed ids (ids are handed out 0,1,2,... on a fresh manager and
// the most recently freed id comes back first), per-id reference counts,
// generation-checked handles, and publish/lookup of full-block token prefixes
// with a zero-reference LRU that allocate() evicts from when no id is free.
// Single-threaded: callers serialise access.

#include "kvflux/detail/index_lru.h"

#include <cstddef>
#include <cstdint>
#include <functional>
#include <stdexcept>
#include <unordered_map>
#include <vector>

namespace kvflux {

using Token = std::int32_t;
using Tokens = std::vector<Token>;

// `id` names a page; `generation` distinguishes successive lifetimes of that
// page so a handle kept past its last release is rejected.
struct BlockHandle {
    std::size_t id;
    std::uint64_t generation;
    bool operator==(const BlockHandle& other) const noexcept {
        return id == other.id && generation == other.generation;
    }
    bool operator!=(const BlockHandle& other) const noexcept { return !(*this == other); }
};

// v0 per-sequence table used by BlockManager::acquire/share/release.
// Copying the struct does not take references.
struct BlockTable {
    std::vector<BlockHandle> blocks;
    std::size_t token_count = 0;
};

// Thrown when every page is referenced and none can be evicted.
class CapacityError : public std::runtime_error {
public:
    CapacityError() : std::runtime_error("no reclaimable KV block") {}
};

class BlockManager {
public:
    using Hasher = std::function<std::uint64_t(const Tokens&)>;
    struct Stats {
        std::size_t capacity, free, active, cached_idle;
    };

    explicit BlockManager(std::size_t capacity, std::size_t block_size,
                          Hasher hasher = prefix_hash);
    BlockManager(const BlockManager&) = delete;
    BlockManager& operator=(const BlockManager&) = delete;
    BlockManager(BlockManager&&) = delete;
    BlockManager& operator=(BlockManager&&) = delete;

    // One reference per allocate/retain; release each exactly once.
    BlockHandle allocate();
    void retain(BlockHandle handle);
    void release(BlockHandle handle);
    std::size_t ref_count(BlockHandle handle) const;
    bool is_published(BlockHandle handle) const;
    // Page ids of n handles that each hold a reference, checked as
    // ref_count does (std::invalid_argument for a stale handle, or one with no
    // reference); out[i] = handles[i].id. One pass, for building tables.
    // No counterpart in the reference.
    void referenced_ids(const BlockHandle* handles, std::size_t n, std::size_t* out) const;

    // Index a privately held full block under the tokens from the start of
    // the sequence to the end of that block.
    void publish(BlockHandle handle, const Tokens& prefix);
    // On a hit, takes one reference and writes the handle to `out`.
    bool lookup(const Tokens& prefix, BlockHandle& out);

    // Whole-sequence helpers of the v0 API: full blocks are looked up or
    // published automatically, a partial tail block stays private.
    BlockTable acquire(const Tokens& tokens);
    BlockTable share(const BlockTable& table);
    void release(BlockTable& table);
    BlockHandle block_at(const BlockTable& table, std::size_t token_index) const;

    Stats stats() const noexcept;
    std::size_t capacity() const noexcept { return pages_.size(); }
    std::size_t block_size() const noexcept { return block_size_; }
    // 64-bit FNV-1a over each token's four little-endian bytes.
    static std::uint64_t prefix_hash(const Tokens& prefix) noexcept;

private:
    struct Page {
        std::uint64_t generation = 0;
        std::size_t refs = 0;
        bool in_use = false;   // false: sitting in the free stack
        bool published = false;
        std::uint64_t hash = 0;
        Tokens prefix;
    };
    const Page& live(BlockHandle handle) const;
    Page& live(BlockHandle handle);
    void unpublish(std::size_t id);
    void check_table(const BlockTable& table) const;

    std::vector<Page> pages_;
    std::vector<std::size_t> free_stack_;  // top = back(); next id to hand out
    std::size_t block_size_;
    Hasher hasher_;
    detail::IndexLru idle_;                // published pages with refs == 0
    std::size_t idle_count_ = 0;
    std::unordered_map<std::uint64_t, std::vector<std::size_t>> by_hash_;
};

} // namespace kvflux
