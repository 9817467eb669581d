// Page-id allocator: observable behaviour follows the reference's
// src/block_manager.cpp (allocation order :8-18 and :45-64, reference
// counting :66-86, publish/lookup :91-134, v0 table helpers :136-202,
// FNV-1a prefix hash :214-226). Free ids live on an explicit LIFO stack
// instead of an intrusive list; the resulting id order is the same.
#include "kvflux/block_manager.h"

#include <algorithm>
#include <limits>
#include <unordered_set>
#include <utility>

namespace kvflux {

BlockManager::BlockManager(std::size_t capacity, std::size_t block_size, Hasher hasher)
    : pages_(capacity), block_size_(block_size), hasher_(std::move(hasher)), idle_(capacity) {
    if (capacity == 0 || block_size == 0 || !hasher_) {
        throw std::invalid_argument("capacity, block size and hasher must be valid");
    }
    // Top of the stack is the back: push ids in descending order so a fresh
    // manager hands out 0, 1, 2, ...
    free_stack_.reserve(capacity);
    for (std::size_t i = capacity; i-- > 0;) free_stack_.push_back(i);
}

const BlockManager::Page& BlockManager::live(BlockHandle handle) const {
    if (handle.id >= pages_.size() || !pages_[handle.id].in_use ||
        pages_[handle.id].generation != handle.generation) {
        throw std::invalid_argument("invalid or stale block handle");
    }
    return pages_[handle.id];
}

BlockManager::Page& BlockManager::live(BlockHandle handle) {
    return const_cast<Page&>(static_cast<const BlockManager&>(*this).live(handle));
}

void BlockManager::unpublish(std::size_t id) {
    auto& page = pages_[id];
    auto bucket = by_hash_.find(page.hash);
    auto& ids = bucket->second;
    ids.erase(std::find(ids.begin(), ids.end(), id));
    if (ids.empty()) by_hash_.erase(bucket);
    page.published = false;
    page.prefix.clear();
}

BlockHandle BlockManager::allocate() {
    const bool from_free = !free_stack_.empty();
    const std::size_t id = from_free ? free_stack_.back() : idle_.oldest();
    if (id == detail::IndexLru::none) throw CapacityError();
    auto& page = pages_[id];
    if (page.generation == std::numeric_limits<std::uint64_t>::max()) {
        throw std::overflow_error("block generation exhausted");
    }
    if (from_free) {
        free_stack_.pop_back();
    } else {
        // Evict the least recently idled published page (refs == 0).
        idle_.erase(id);
        --idle_count_;
        unpublish(id);
    }
    page.in_use = true;
    page.refs = 1;
    ++page.generation;
    return {id, page.generation};
}

void BlockManager::retain(BlockHandle handle) {
    auto& page = live(handle);
    if (page.refs == std::numeric_limits<std::size_t>::max()) {
        throw std::overflow_error("reference count exhausted");
    }
    if (page.refs == 0) {
        idle_.erase(handle.id);
        --idle_count_;
    }
    ++page.refs;
}

void BlockManager::release(BlockHandle handle) {
    auto& page = live(handle);
    if (page.refs == 0) throw std::invalid_argument("block already released");
    if (--page.refs != 0) return;
    if (page.published) {
        idle_.touch(handle.id);
        ++idle_count_;
    } else {
        page.in_use = false;
        free_stack_.push_back(handle.id);
    }
}

std::size_t BlockManager::ref_count(BlockHandle handle) const { return live(handle).refs; }

void BlockManager::referenced_ids(const BlockHandle* handles, std::size_t n, std::size_t* out) const {
    for (std::size_t i = 0; i < n; ++i) {
        if (live(handles[i]).refs == 0) throw std::invalid_argument("physical block has no active reference");
        out[i] = handles[i].id;
    }
}

bool BlockManager::is_published(BlockHandle handle) const { return live(handle).published; }

void BlockManager::publish(BlockHandle handle, const Tokens& prefix) {
    auto& page = live(handle);
    if (page.refs != 1 || page.published || prefix.empty() || prefix.size() % block_size_ != 0) {
        throw std::invalid_argument("publish requires a private block and a full prefix");
    }
    const auto hash = hasher_(prefix);
    if (const auto it = by_hash_.find(hash); it != by_hash_.end()) {
        for (const auto id : it->second) {
            if (pages_[id].prefix == prefix) {
                throw std::invalid_argument("prefix already published; use lookup");
            }
        }
    }
    // Do every allocation before touching the page so a failure leaves no
    // half-published state behind.
    Tokens copy = prefix;
    auto [bucket, created] = by_hash_.try_emplace(hash);
    try {
        bucket->second.push_back(handle.id);
    } catch (...) {
        if (created) by_hash_.erase(bucket);
        throw;
    }
    page.prefix = std::move(copy);
    page.hash = hash;
    page.published = true;
}

bool BlockManager::lookup(const Tokens& prefix, BlockHandle& out) {
    if (prefix.empty() || prefix.size() % block_size_ != 0) return false;
    const auto it = by_hash_.find(hasher_(prefix));
    if (it == by_hash_.end()) return false;
    for (const auto id : it->second) {
        // Equal hashes are not equal prefixes: compare the tokens.
        if (pages_[id].prefix == prefix) {
            const BlockHandle hit{id, pages_[id].generation};
            retain(hit);
            out = hit;
            return true;
        }
    }
    return false;
}

BlockTable BlockManager::acquire(const Tokens& tokens) {
    BlockTable table;
    table.token_count = tokens.size();
    table.blocks.reserve((tokens.size() + block_size_ - 1) / block_size_);
    Tokens prefix;
    prefix.reserve(tokens.size());
    try {
        for (std::size_t begin = 0; begin < tokens.size();) {
            const std::size_t n = std::min(block_size_, tokens.size() - begin);
            prefix.insert(prefix.end(), tokens.begin() + begin, tokens.begin() + begin + n);
            const bool full = n == block_size_;
            BlockHandle handle{};
            if (full && lookup(prefix, handle)) {
                table.blocks.push_back(handle);
            } else {
                handle = allocate();
                table.blocks.push_back(handle);  // capacity reserved above
                if (full) publish(handle, prefix);
            }
            begin += n;
        }
    } catch (...) {
        for (const auto handle : table.blocks) release(handle);
        throw;
    }
    return table;
}

void BlockManager::check_table(const BlockTable& table) const {
    const auto expected = (table.token_count + block_size_ - 1) / block_size_;
    if (expected != table.blocks.size()) throw std::invalid_argument("invalid block table size");
    std::unordered_set<std::size_t> seen;
    for (const auto handle : table.blocks) {
        if (live(handle).refs == 0) throw std::invalid_argument("unowned block");
        // A live handle is fully identified by its id.
        if (!seen.insert(handle.id).second) throw std::invalid_argument("duplicate block");
    }
}

BlockTable BlockManager::share(const BlockTable& table) {
    check_table(table);
    BlockTable copy = table;
    std::size_t retained = 0;
    try {
        for (const auto handle : copy.blocks) {
            retain(handle);
            ++retained;
        }
    } catch (...) {
        for (std::size_t i = 0; i < retained; ++i) release(copy.blocks[i]);
        throw;
    }
    return copy;
}

void BlockManager::release(BlockTable& table) {
    check_table(table);  // validate everything before releasing anything
    for (const auto handle : table.blocks) release(handle);
    table.blocks.clear();
    table.token_count = 0;
}

BlockHandle BlockManager::block_at(const BlockTable& table, std::size_t token_index) const {
    if (token_index >= table.token_count) throw std::out_of_range("token index out of range");
    const auto handle = table.blocks.at(token_index / block_size_);
    if (live(handle).refs == 0) throw std::invalid_argument("unowned block");
    return handle;
}

BlockManager::Stats BlockManager::stats() const noexcept {
    const std::size_t free = free_stack_.size();
    return Stats{pages_.size(), free, pages_.size() - free - idle_count_, idle_count_};
}

std::uint64_t BlockManager::prefix_hash(const Tokens& prefix) noexcept {
    // 64-bit FNV-1a; each token contributes its 32-bit two's-complement
    // value least significant byte first, independent of host endianness.
    constexpr std::uint64_t offset_basis = 0xcbf29ce484222325ULL;
    constexpr std::uint64_t prime = 0x100000001b3ULL;
    std::uint64_t h = offset_basis;
    for (const Token token : prefix) {
        const auto bits = static_cast<std::uint32_t>(token);
        for (int shift = 0; shift < 32; shift += 8) {
            h = (h ^ ((bits >> shift) & 0xffu)) * prime;
        }
    }
    return h;
}

} // namespace kvflux
