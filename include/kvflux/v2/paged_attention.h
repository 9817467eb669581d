#pragma once
// Causal GQA attention straight from the paged cache.
// Same signatures and contracts as the reference's
// include/kvflux/v2/paged_attention.h:20-33 (src/v2/paged_attention.cu:193-313).

#include "kvflux/v2/paged_kv_storage.h"

#include <cstddef>
#include <vector>

namespace kvflux::v2 {

// Arithmetic contract of an attention call.
//   Exact: FP32 Q and FP32 accumulation of every product; matches the
//          double-precision CPU reference to ~1e-6 for any KV dtype (the
//          reference's 1e-5 contract). The reference's own signature below
//          uses it. Calls of 16 or more query tokens at head_size 64 or 128
//          (block_size a power of two up to 256) run on the MFMA prefill:
//          on a 16-bit cache with Q and the weights split into three 16-bit
//          parts (exact products), on an FP32 cache with FP32 MFMAs; others
//          on the split-K kernel.
//   Auto:  Exact, except that calls of query_tokens >= 16 on a 16-bit cache
//          at the shapes the MFMA prefill takes (head_size 64, 128 or 256,
//          block_size a power of two up to 256) run there with Q and the
//          softmax weights rounded to the cache dtype (2e-2 contract). FP32
//          caches keep the Exact routing.
//   Fast:  the MFMA prefill whenever the shape allows it (any query_tokens;
//          rounded on 16-bit caches, FP32 MFMAs on FP32 caches), otherwise
//          Exact.
enum class AttentionPrecision { Exact, Auto, Fast };

// Single request: Q/O are device FP32 [query_tokens][query_heads][head_size];
// query i sees cache positions <= num_tokens - query_tokens + i.
// Uses AttentionPrecision::Exact, the reference's contract; pass Auto or Fast
// to the overload below for the MFMA prefill.
void paged_attention(const PagedKVStorage& storage, const SequenceState& sequence,
                     const float* query_device, float* output_device,
                     std::size_t query_tokens, std::size_t query_heads);

void paged_attention(const PagedKVStorage& storage, const SequenceState& sequence,
                     const float* query_device, float* output_device,
                     std::size_t query_tokens, std::size_t query_heads,
                     AttentionPrecision precision);

// Batch decode: one trailing query per request, Q/O device FP32
// [num_sequences][query_heads][head_size]. Always Exact.
void paged_attention_batch(const PagedKVStorage& storage,
                           const std::vector<const SequenceState*>& sequences,
                           const float* query_device, float* output_device,
                           std::size_t query_heads);

} // namespace kvflux::v2
