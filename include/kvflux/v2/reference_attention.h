#pragma once
// CPU correctness reference of causal (suffix-aligned) attention
// (reference include/kvflux/v2/reference_attention.h:10-27).

#include <cstddef>
#include <vector>

namespace kvflux::v2 {

// Contiguous single-request shapes: Q and O are [query_tokens][query_heads][head_size],
// K and V are [kv_tokens][kv_heads][head_size], innermost dimension contiguous.
struct AttentionShape {
    std::size_t query_tokens;
    std::size_t kv_tokens;
    std::size_t query_heads;
    std::size_t kv_heads;
    std::size_t head_size;
};

// softmax(Q K^T / sqrt(head_size) + causal mask) V on the host, accumulated in
// double. The queries are the LAST query_tokens positions of the KV sequence:
// query i sits at kv_tokens - query_tokens + i and sees tokens up to it.
// query_heads must be a multiple of kv_heads; query head q reads kv head
// q / (query_heads / kv_heads). All inputs must be finite.
// Throws std::invalid_argument (shape, sizes, non-finite input) and
// std::overflow_error (tensor size overflow).
std::vector<float> reference_attention(const std::vector<float>& query,
                                       const std::vector<float>& key,
                                       const std::vector<float>& value,
                                       const AttentionShape& shape);

} // namespace kvflux::v2
