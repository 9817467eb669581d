#pragma once
// Synchronous single-request prefill/decode driver over the paged data path.
// Same surface as the reference's include/kvflux/v2/sequence_lifecycle.h:12-47.

#include "kvflux/v2/paged_attention.h"
#include "kvflux/v2/paged_kv_storage.h"

#include <cstddef>
#include <optional>

namespace kvflux::v2 {

class SequenceLifecycle {
public:
    // `precision` (an addition to the reference's constructor) selects the
    // attention contract of prefill and decode; Exact is the reference's.
    SequenceLifecycle(RequestID request_id, PhysicalBlockPool& pool, PagedKVStorage& storage,
                      std::size_t query_heads, AttentionPrecision precision = AttentionPrecision::Exact);
    ~SequenceLifecycle() noexcept { finish(); }
    SequenceLifecycle(const SequenceLifecycle&) = delete;
    SequenceLifecycle& operator=(const SequenceLifecycle&) = delete;
    SequenceLifecycle(SequenceLifecycle&&) = delete;
    SequenceLifecycle& operator=(SequenceLifecycle&&) = delete;

    // Once per request. K/V: device [token_count][kv_heads][head_size];
    // Q/O: device FP32 [token_count][query_heads][head_size].
    void prefill(std::size_t token_count, const void* key_device, const void* value_device,
                 const float* query_device, float* output_device);

    // One token: copy-on-write of a shared tail if needed, write its K/V,
    // attention of its query over the whole sequence.
    TokenLocation decode(const void* key_device, const void* value_device,
                         const float* query_device, float* output_device);

    void finish() noexcept;
    bool finished() const noexcept { return !sequence_.has_value(); }
    const SequenceState& sequence() const;

private:
    // Runs one step; on any exception waits for the device, finishes the
    // request (its pages go back) and rethrows.
    template <typename Step>
    auto guarded(Step&& step) -> decltype(step());
    void abort_after_failure() noexcept;

    PagedKVStorage& storage_;
    std::optional<SequenceState> sequence_;
    std::size_t query_heads_;
    AttentionPrecision precision_;
    bool prefilled_ = false;
};

} // namespace kvflux::v2
