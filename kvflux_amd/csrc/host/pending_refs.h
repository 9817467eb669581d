// References taken during one control-plane operation, kept aside until the
// operation succeeds and handed back if it does not. The order of the
// hand-back is part of the contract: pages released to the free stack come
// back LIFO, and published pages re-enter the idle order in release order,
// so each caller names the order its reference semantics require.
#pragma once

#include "kvflux/detail/page_ledger.h"

#include <cstddef>
#include <utility>
#include <vector>

namespace kvflux::host {

enum class Undo {
    InTakeOrder,       // the first reference taken is returned first
    InReverseOrder,    // the last reference taken is returned first
};

template <typename Release>
class PendingRefs {
public:
    // Room for `expected` references is reserved here, so add() never throws.
    PendingRefs(Release release, std::size_t expected, Undo undo)
        : release_(std::move(release)), undo_(undo) {
        handles_.reserve(expected);
    }
    PendingRefs(const PendingRefs&) = delete;
    PendingRefs& operator=(const PendingRefs&) = delete;

    ~PendingRefs() {
        if (committed_) return;
        if (undo_ == Undo::InTakeOrder) {
            for (const BlockHandle h : handles_) release_(h);
        } else {
            for (auto it = handles_.rbegin(); it != handles_.rend(); ++it) release_(*it);
        }
    }

    // `handle` carries one reference this object now owns.
    void add(BlockHandle handle) noexcept { handles_.push_back(handle); }
    BlockHandle back() const noexcept { return handles_.back(); }
    std::size_t size() const noexcept { return handles_.size(); }
    const std::vector<BlockHandle>& handles() const noexcept { return handles_; }

    // The operation succeeded: the references belong to the caller now.
    std::vector<BlockHandle> commit() noexcept {
        committed_ = true;
        return std::move(handles_);
    }

private:
    Release release_;
    Undo undo_;
    std::vector<BlockHandle> handles_;
    bool committed_ = false;
};

template <typename Release>
PendingRefs<Release> pending_refs(Release release, std::size_t expected, Undo undo) {
    return PendingRefs<Release>(std::move(release), expected, undo);
}

inline std::size_t ceil_div(std::size_t n, std::size_t d) { return n / d + (n % d != 0); }

} // namespace kvflux::host
