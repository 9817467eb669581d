#pragma once
// v0 page-id allocator. Same public surface as the reference's
// include/kvflux/block_manager.h:14-78: LIFO reuse of freed ids (ids are
// handed out 0, 1, 2, ... on a fresh manager and the most recently freed id
// comes back first), per-id reference counts, generation-checked handles,
// and publish/lookup of full-block token prefixes with eviction of the least
// recently idled published page when no id is free. Page state lives in a
// detail::PageLedger (include/kvflux/detail/page_ledger.h); this class adds
// the v0 whole-sequence table helpers. Single-threaded: callers serialise
// access.

#include "kvflux/detail/page_ledger.h"

#include <cstddef>
#include <cstdint>
#include <functional>
#include <vector>

namespace kvflux {

// v0 per-sequence table used by BlockManager::acquire/share/release.
// Copying the struct does not take references.
struct BlockTable {
    std::vector<BlockHandle> blocks;
    std::size_t token_count = 0;
};

class BlockManager {
public:
    using Hasher = detail::PageLedger::Hasher;
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
    BlockHandle allocate() { return ledger_.take(); }
    void retain(BlockHandle handle) { ledger_.hold(handle); }
    void release(BlockHandle handle) { ledger_.drop(handle); }
    std::size_t ref_count(BlockHandle handle) const { return ledger_.holders(handle); }
    bool is_published(BlockHandle handle) const { return ledger_.published(handle); }

    // Index a privately held full block under the tokens from the start of
    // the sequence to the end of that block.
    void publish(BlockHandle handle, const Tokens& prefix) { ledger_.publish(handle, prefix); }
    // On a hit, takes one reference and writes the handle to `out`.
    bool lookup(const Tokens& prefix, BlockHandle& out) { return ledger_.find(prefix, out); }

    // Whole-sequence helpers of the v0 API: full blocks are looked up or
    // published automatically, a partial tail block stays private.
    BlockTable acquire(const Tokens& tokens);
    BlockTable share(const BlockTable& table);
    void release(BlockTable& table);
    BlockHandle block_at(const BlockTable& table, std::size_t token_index) const;

    Stats stats() const noexcept;
    std::size_t capacity() const noexcept { return ledger_.capacity(); }
    std::size_t block_size() const noexcept { return ledger_.block_size(); }
    // 64-bit FNV-1a over each token's four little-endian bytes.
    static std::uint64_t prefix_hash(const Tokens& prefix) noexcept;

private:
    void check_table(const BlockTable& table) const;

    detail::PageLedger ledger_;
};

} // namespace kvflux
