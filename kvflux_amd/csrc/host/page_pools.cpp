// The two page pools over detail::PageLedger:
//   BlockManager      v0 API; its whole-sequence table helpers (acquire,
//                     share, release, block_at) keep the reference's results
//                     and rollback order, src/block_manager.cpp:136-202;
//   PhysicalBlockPool v2 API, include/kvflux/physical_block_pool.h:22-58.
#include "kvflux/block_manager.h"
#include "kvflux/physical_block_pool.h"

#include "pending_refs.h"

#include <algorithm>
#include <stdexcept>

namespace kvflux {

using host::ceil_div;
using host::pending_refs;
using host::Undo;

// ---------------------------------------------------------------- v0 manager
BlockManager::BlockManager(std::size_t capacity, std::size_t block_size, Hasher hasher)
    : ledger_(capacity, block_size, std::move(hasher)) {}

BlockTable BlockManager::acquire(const Tokens& tokens) {
    const std::size_t bs = ledger_.block_size();
    const std::size_t blocks = ceil_div(tokens.size(), bs);
    // On failure every reference taken so far is returned, first one first.
    auto taken = pending_refs([this](BlockHandle h) { ledger_.drop(h); }, blocks, Undo::InTakeOrder);
    Tokens prefix;
    prefix.reserve(tokens.size());
    for (std::size_t b = 0; b < blocks; ++b) {
        const std::size_t end = std::min(tokens.size(), (b + 1) * bs);
        prefix.insert(prefix.end(), tokens.begin() + static_cast<std::ptrdiff_t>(b * bs),
                      tokens.begin() + static_cast<std::ptrdiff_t>(end));
        // A full block is shared when its whole prefix is published, and
        // published when it is not; a partial tail block stays private.
        const bool full = end - b * bs == bs;
        BlockHandle cached{};
        if (full && ledger_.find(prefix, cached)) {
            taken.add(cached);
            continue;
        }
        taken.add(ledger_.take());
        if (full) ledger_.publish(taken.back(), prefix);
    }
    BlockTable table;
    table.token_count = tokens.size();
    table.blocks = taken.commit();
    return table;
}

void BlockManager::check_table(const BlockTable& table) const {
    if (table.blocks.size() != ceil_div(table.token_count, ledger_.block_size())) {
        throw std::invalid_argument("block table size does not match its token count");
    }
    std::vector<std::size_t> ids;
    ids.reserve(table.blocks.size());
    for (const BlockHandle h : table.blocks) {
        if (ledger_.holders(h) == 0) throw std::invalid_argument("block table entry holds no reference");
        ids.push_back(h.id);
    }
    std::sort(ids.begin(), ids.end());
    if (std::adjacent_find(ids.begin(), ids.end()) != ids.end()) {
        throw std::invalid_argument("block table names a page twice");
    }
}

BlockTable BlockManager::share(const BlockTable& table) {
    check_table(table);
    auto extra = pending_refs([this](BlockHandle h) { ledger_.drop(h); }, table.blocks.size(),
                              Undo::InTakeOrder);
    for (const BlockHandle h : table.blocks) {
        ledger_.hold(h);
        extra.add(h);
    }
    BlockTable copy;
    copy.token_count = table.token_count;
    copy.blocks = extra.commit();
    return copy;
}

void BlockManager::release(BlockTable& table) {
    check_table(table);  // the whole table is valid before anything is released
    for (const BlockHandle h : table.blocks) ledger_.drop(h);
    table.blocks.clear();
    table.token_count = 0;
}

BlockHandle BlockManager::block_at(const BlockTable& table, std::size_t token_index) const {
    if (token_index >= table.token_count) throw std::out_of_range("token index past the table's tokens");
    const std::size_t block = token_index / ledger_.block_size();
    if (block >= table.blocks.size()) throw std::out_of_range("block table shorter than its token count");
    const BlockHandle h = table.blocks[block];
    if (ledger_.holders(h) == 0) throw std::invalid_argument("block table entry holds no reference");
    return h;
}

BlockManager::Stats BlockManager::stats() const noexcept {
    return Stats{ledger_.capacity(), ledger_.free_pages(), ledger_.held_pages(), ledger_.idle_pages()};
}

std::uint64_t BlockManager::prefix_hash(const Tokens& prefix) noexcept {
    // 64-bit FNV-1a; each token contributes its 32-bit two's-complement
    // value least significant byte first, independent of host endianness.
    std::uint64_t h = 0xcbf29ce484222325ULL;
    for (const Token token : prefix) {
        std::uint32_t bits = static_cast<std::uint32_t>(token);
        for (int byte = 0; byte < 4; ++byte, bits >>= 8) h = (h ^ (bits & 0xffu)) * 0x100000001b3ULL;
    }
    return h;
}

// ---------------------------------------------------------------- v2 pool
PhysicalBlockPool::PhysicalBlockPool(std::size_t capacity, std::size_t block_size,
                                     BlockManager::Hasher hasher)
    : ledger_(capacity, block_size, std::move(hasher)) {}

PhysicalBlockHandle PhysicalBlockPool::allocate() { return ledger_.take(); }
void PhysicalBlockPool::retain(PhysicalBlockHandle handle) { ledger_.hold(handle); }
void PhysicalBlockPool::free(PhysicalBlockHandle handle) { ledger_.drop(handle); }
void PhysicalBlockPool::publish(PhysicalBlockHandle handle, const Tokens& prefix) {
    ledger_.publish(handle, prefix);
}
bool PhysicalBlockPool::lookup(const Tokens& prefix, PhysicalBlockHandle& out) {
    return ledger_.find(prefix, out);
}
bool PhysicalBlockPool::is_published(PhysicalBlockHandle handle) const { return ledger_.published(handle); }
std::size_t PhysicalBlockPool::ref_count(PhysicalBlockHandle handle) const { return ledger_.holders(handle); }
std::size_t PhysicalBlockPool::capacity() const noexcept { return ledger_.capacity(); }
std::size_t PhysicalBlockPool::block_size() const noexcept { return ledger_.block_size(); }
std::size_t PhysicalBlockPool::available() const noexcept {
    return ledger_.free_pages() + ledger_.idle_pages();
}

PhysicalBlockID PhysicalBlockPool::id(PhysicalBlockHandle handle) const {
    // An idle published page (no reference) is not addressable: only a page
    // someone holds may be read or written.
    if (ledger_.holders(handle) == 0) {
        throw std::invalid_argument("page is not held by anyone; its id may be reused");
    }
    return handle.id;
}

void PhysicalBlockPool::ids(const PhysicalBlockHandle* handles, std::size_t n, PhysicalBlockID* out) const {
    for (std::size_t i = 0; i < n; ++i) out[i] = id(handles[i]);
}

} // namespace kvflux
