#pragma once
// Recency list over dense integer ids [0, capacity): O(1) touch/erase/oldest.
// Used by BlockManager to remember published pages whose reference count
// dropped to zero, so allocate() can evict the least recently idled one
// (same role as include/kvflux/detail/index_lru.h in the reference).

#include <cstddef>
#include <cstdint>
#include <limits>
#include <vector>

namespace kvflux::detail {

class IndexLru {
public:
    static constexpr std::size_t none = std::numeric_limits<std::size_t>::max();

    explicit IndexLru(std::size_t capacity) : prev_(capacity, none), next_(capacity, none),
                                              linked_(capacity, 0) {}

    // Least recently touched id still in the list, or `none`.
    std::size_t oldest() const noexcept { return head_; }
    std::size_t next(std::size_t id) const noexcept { return next_[id]; }
    bool contains(std::size_t id) const noexcept { return linked_[id] != 0; }

    // Removes `id` if present; a no-op otherwise.
    void erase(std::size_t id) noexcept {
        if (!linked_[id]) return;
        const std::size_t p = prev_[id], n = next_[id];
        (p == none ? head_ : next_[p]) = n;
        (n == none ? tail_ : prev_[n]) = p;
        prev_[id] = next_[id] = none;
        linked_[id] = 0;
    }

    // Moves (or inserts) `id` to the most-recent end.
    void touch(std::size_t id) noexcept {
        erase(id);
        prev_[id] = tail_;
        next_[id] = none;
        (tail_ == none ? head_ : next_[tail_]) = id;
        tail_ = id;
        linked_[id] = 1;
    }

private:
    std::vector<std::size_t> prev_, next_;
    std::vector<std::uint8_t> linked_;
    std::size_t head_ = none, tail_ = none;
};

} // namespace kvflux::detail
