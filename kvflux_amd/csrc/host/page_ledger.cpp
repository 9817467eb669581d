// Page ownership ledger (include/kvflux/detail/page_ledger.h). Observable
// behaviour (the order page ids are handed out, eviction order of idle
// published pages, reference counts, generations, exception types) is the
// reference's v0 allocator's, src/block_manager.cpp:8-134; the data
// structures are this file's own (free stack, stamped idle ring, multimap
// prefix index).
#include "kvflux/detail/page_ledger.h"

#include <algorithm>
#include <limits>

namespace kvflux::detail {

PageLedger::PageLedger(std::size_t capacity, std::size_t block_size, Hasher hasher)
    : block_size_(block_size), hasher_(std::move(hasher)) {
    if (capacity == 0) throw std::invalid_argument("page ledger: capacity must be positive");
    if (block_size == 0) throw std::invalid_argument("page ledger: block size must be positive");
    if (!hasher_) throw std::invalid_argument("page ledger: a prefix hasher is required");
    pages_.resize(capacity);
    prefixes_.resize(capacity);
    free_.resize(capacity);
    // The stack's top is its back: ids in descending order hand out 0 first.
    for (std::size_t i = 0; i < capacity; ++i) free_[i] = capacity - 1 - i;
    ring_.resize(2 * capacity + 2);
}

std::size_t PageLedger::live_id(BlockHandle handle) const {
    if (handle.id < pages_.size()) {
        const Page& page = pages_[handle.id];
        if (page.state != State::Free && page.generation == handle.generation) return handle.id;
    }
    throw std::invalid_argument("page handle is unknown, released or from an earlier allocation");
}

bool PageLedger::current(const IdleRecord& record) const noexcept {
    const Page& page = pages_[record.id];
    return page.state == State::Idle && page.idle_stamp == record.stamp;
}

std::size_t PageLedger::oldest_idle() noexcept {
    while (ring_count_ > 0) {
        const IdleRecord& front = ring_[ring_head_];
        if (current(front)) return front.id;
        ring_head_ = (ring_head_ + 1) % ring_.size();
        --ring_count_;
    }
    return npos;
}

void PageLedger::squeeze_idle() noexcept {
    // Keep the current records, in order, packed from the head.
    std::size_t kept = 0;
    for (std::size_t i = 0; i < ring_count_; ++i) {
        const IdleRecord record = ring_[(ring_head_ + i) % ring_.size()];
        if (current(record)) ring_[(ring_head_ + kept++) % ring_.size()] = record;
    }
    ring_count_ = kept;
}

void PageLedger::push_idle(std::size_t id) noexcept {
    // At most `capacity` records are current, so after a squeeze a ring of
    // 2 * capacity + 2 always has room.
    if (ring_count_ == ring_.size()) squeeze_idle();
    Page& page = pages_[id];
    page.idle_stamp = ++clock_;
    ring_[(ring_head_ + ring_count_) % ring_.size()] = IdleRecord{page.idle_stamp, id};
    ++ring_count_;
}

void PageLedger::unpublish(std::size_t id) noexcept {
    Page& page = pages_[id];
    auto [first, last] = by_key_.equal_range(page.key);
    for (auto it = first; it != last; ++it) {
        if (it->second == id) {
            by_key_.erase(it);
            break;
        }
    }
    prefixes_[id].clear();
    page.published = false;
}

BlockHandle PageLedger::take() {
    const bool fresh = !free_.empty();
    const std::size_t id = fresh ? free_.back() : oldest_idle();
    if (id == npos) throw CapacityError();
    Page& page = pages_[id];
    if (page.generation == std::numeric_limits<std::uint64_t>::max()) {
        throw std::overflow_error("page generation counter exhausted");
    }
    if (fresh) {
        free_.pop_back();
    } else {
        // The record at the ring's front is this page's (oldest_idle).
        ring_head_ = (ring_head_ + 1) % ring_.size();
        --ring_count_;
        --idle_count_;
        unpublish(id);
    }
    page.state = State::Held;
    page.refs = 1;
    ++page.generation;
    return BlockHandle{id, page.generation};
}

void PageLedger::hold(BlockHandle handle) {
    Page& page = pages_[live_id(handle)];
    if (page.refs == std::numeric_limits<std::size_t>::max()) {
        throw std::overflow_error("page reference count exhausted");
    }
    if (page.state == State::Idle) {  // its ring record turns stale by state
        page.state = State::Held;
        --idle_count_;
    }
    ++page.refs;
}

void PageLedger::drop(BlockHandle handle) {
    const std::size_t id = live_id(handle);
    Page& page = pages_[id];
    if (page.refs == 0) throw std::invalid_argument("page has no reference left to release");
    if (--page.refs > 0) return;
    if (page.published) {
        page.state = State::Idle;
        ++idle_count_;
        push_idle(id);
    } else {
        page.state = State::Free;
        free_.push_back(id);  // capacity reserved: never reallocates
    }
}

std::size_t PageLedger::holders(BlockHandle handle) const { return pages_[live_id(handle)].refs; }

bool PageLedger::published(BlockHandle handle) const { return pages_[live_id(handle)].published; }

void PageLedger::publish(BlockHandle handle, const Tokens& prefix) {
    const std::size_t id = live_id(handle);
    Page& page = pages_[id];
    const bool whole_blocks = !prefix.empty() && prefix.size() % block_size_ == 0;
    if (page.refs != 1 || page.published || !whole_blocks) {
        throw std::invalid_argument(
            "publish needs a page held by exactly one owner and a prefix of whole blocks");
    }
    const std::uint64_t key = hasher_(prefix);
    auto [first, last] = by_key_.equal_range(key);
    if (std::any_of(first, last, [&](const auto& entry) { return prefixes_[entry.second] == prefix; })) {
        throw std::invalid_argument("this token prefix is already published");
    }
    // Everything that can throw happens before the page changes.
    Tokens stored(prefix);
    by_key_.emplace(key, id);
    prefixes_[id] = std::move(stored);
    page.key = key;
    page.published = true;
}

bool PageLedger::find(const Tokens& prefix, BlockHandle& out) {
    if (prefix.empty() || prefix.size() % block_size_ != 0) return false;
    auto [first, last] = by_key_.equal_range(hasher_(prefix));
    for (auto it = first; it != last; ++it) {
        if (prefixes_[it->second] != prefix) continue;  // same hash, other tokens
        const BlockHandle hit{it->second, pages_[it->second].generation};
        hold(hit);
        out = hit;
        return true;
    }
    return false;
}

} // namespace kvflux::detail
