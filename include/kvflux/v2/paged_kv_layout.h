#pragma once
// Byte layout of the single-layer paged KV arena:
//   K[num_blocks][num_kv_heads][block_size][head_size], then V of the same
//   shape; innermost dimension contiguous, no padding.
// Same surface as the reference's include/kvflux/v2/paged_kv_layout.h:12-40.

#include "kvflux/kv_layout.h"

#include <cstddef>
#include <cstdint>

namespace kvflux::v2 {

class PagedKVLayout {
public:
    PagedKVLayout(std::size_t num_blocks, std::size_t num_kv_heads,
                  std::size_t block_size, std::size_t head_size, DType dtype);

    std::size_t num_blocks() const noexcept { return blocks_; }
    std::size_t num_kv_heads() const noexcept { return heads_; }
    std::size_t block_size() const noexcept { return block_size_; }
    std::size_t head_size() const noexcept { return head_size_; }
    DType dtype() const noexcept { return dtype_; }
    std::size_t element_bytes() const noexcept { return element_bytes_; }
    std::size_t page_bytes() const noexcept { return page_bytes_; }
    std::size_t cache_bytes() const noexcept { return cache_bytes_; }
    std::size_t total_bytes() const noexcept { return 2 * cache_bytes_; }
    std::size_t slot_count() const noexcept { return slot_count_; }

    // Offsets from the start of the K+V allocation; every coordinate is
    // bounds-checked (std::out_of_range, std::invalid_argument for a bad kind).
    std::size_t page_byte_offset(KVKind kind, std::size_t block) const;
    std::size_t byte_offset(KVKind kind, std::size_t block, std::size_t head,
                            std::size_t token, std::size_t dimension) const;
    std::size_t slot_byte_offset(KVKind kind, std::uint64_t slot,
                                 std::size_t head, std::size_t dimension) const;

private:
    std::size_t blocks_, heads_, block_size_, head_size_;
    DType dtype_;
    std::size_t element_bytes_, page_bytes_, cache_bytes_, slot_count_;
};

} // namespace kvflux::v2
