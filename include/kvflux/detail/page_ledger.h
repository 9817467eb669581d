#pragma once
// Ownership ledger of a fixed set of page ids: the one implementation of page
// state that both the v0 BlockManager and the v2 PhysicalBlockPool sit on.
//
// A page is in one of three states:
//   free  - on the free stack; the next allocation takes the id pushed last,
//           and a fresh ledger hands ids out as 0, 1, 2, ...
//   held  - at least one reference;
//   idle  - published (indexed under its token prefix) with no reference:
//           still findable by prefix, and evicted (least recently idled
//           first) when an allocation finds the free stack empty.
// Handles carry the page's generation, bumped at every allocation, so a
// handle kept past the end of its allocation is rejected.
//
// Data structures (no allocation on any release path, so releases can run
// from destructors):
//   * free ids:  a stack reserved to the capacity up front;
//   * idle order: a ring of (stamp, id) records, reserved to twice the
//     capacity. Releasing a published page to zero references appends
//     (++clock, id) and stores the stamp on the page; a record is current
//     only while the page is still idle with that same stamp, so retaining
//     an idle page needs no unlinking. Stale records are skipped at the front
//     and squeezed out in place when the ring fills up;
//   * prefix index: hash -> page multimap plus the page's stored tokens;
//     a hit needs equal tokens, not only an equal hash.
// Single-threaded: callers serialise access.

#include <cstddef>
#include <cstdint>
#include <functional>
#include <stdexcept>
#include <unordered_map>
#include <utility>
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

// Thrown when every page is referenced and none can be evicted.
class CapacityError : public std::runtime_error {
public:
    CapacityError() : std::runtime_error("no reclaimable KV block") {}
};

namespace detail {

class PageLedger {
public:
    using Hasher = std::function<std::uint64_t(const Tokens&)>;
    static constexpr std::size_t npos = ~std::size_t{0};

    // std::invalid_argument for a zero capacity or block size or an empty hasher.
    PageLedger(std::size_t capacity, std::size_t block_size, Hasher hasher);

    // A new reference to the page on top of the free stack, else to the
    // least recently idled page (which loses its prefix). CapacityError when
    // neither exists; std::overflow_error when that page's generation is
    // exhausted (nothing changes then).
    BlockHandle take();
    // One more reference (an idle page becomes held again).
    void hold(BlockHandle handle);
    // One reference less; at zero the page goes idle if published, free if not.
    void drop(BlockHandle handle);

    // References of a live (held or idle) handle; std::invalid_argument for
    // an unknown or stale one (all handle-taking calls check the same way).
    std::size_t holders(BlockHandle handle) const;
    bool published(BlockHandle handle) const;
    // Indexes a privately held page (exactly one reference, not yet
    // published) under `prefix`, a non-empty whole number of blocks not
    // already published. std::invalid_argument otherwise.
    void publish(BlockHandle handle, const Tokens& prefix);
    // On a hit, takes a reference and stores the handle in `out`.
    bool find(const Tokens& prefix, BlockHandle& out);

    std::size_t capacity() const noexcept { return pages_.size(); }
    std::size_t block_size() const noexcept { return block_size_; }
    std::size_t free_pages() const noexcept { return free_.size(); }
    std::size_t idle_pages() const noexcept { return idle_count_; }
    std::size_t held_pages() const noexcept { return pages_.size() - free_.size() - idle_count_; }

private:
    enum class State : std::uint8_t { Free, Held, Idle };
    struct Page {
        std::uint64_t generation = 0;
        std::size_t refs = 0;
        std::uint64_t idle_stamp = 0;  // stamp of its current idle-ring record
        std::uint64_t key = 0;         // prefix hash while published
        State state = State::Free;
        bool published = false;
    };
    struct IdleRecord {
        std::uint64_t stamp;
        std::size_t id;
    };

    std::size_t live_id(BlockHandle handle) const;
    bool current(const IdleRecord& record) const noexcept;
    std::size_t oldest_idle() noexcept;  // drops stale records at the front
    void push_idle(std::size_t id) noexcept;
    void squeeze_idle() noexcept;
    void unpublish(std::size_t id) noexcept;

    std::vector<Page> pages_;
    std::vector<Tokens> prefixes_;    // tokens of published pages, empty otherwise
    std::vector<std::size_t> free_;   // top = back()
    std::vector<IdleRecord> ring_;    // idle order, oldest at ring_head_
    std::size_t ring_head_ = 0, ring_count_ = 0;
    std::uint64_t clock_ = 0;
    std::size_t idle_count_ = 0;
    std::unordered_multimap<std::uint64_t, std::size_t> by_key_;
    std::size_t block_size_;
    Hasher hasher_;
};

} // namespace detail
} // namespace kvflux
