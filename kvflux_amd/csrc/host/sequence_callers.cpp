// Callers of the data path: prefix sharing, copy-on-write decode append and
// the single-request lifecycle. Behaviour follows the reference:
//   PrefixCache        src/v2/prefix_cache.cpp:7-57
//   append_token_cow   src/v2/copy_on_write.cpp:7-16
//   SequenceLifecycle  src/v2/sequence_lifecycle.cpp:13-86
#include "kvflux/v2/copy_on_write.h"
#include "kvflux/v2/paged_attention.h"
#include "kvflux/v2/paged_kv_write.h"
#include "kvflux/v2/prefix_cache.h"
#include "kvflux/v2/sequence_lifecycle.h"

#include "device_runtime.h"

#include <stdexcept>
#include <vector>

namespace kvflux::v2 {

std::size_t PrefixCache::attach_cached_prefix(SequenceState& sequence, const Tokens& tokens) {
    if (!sequence.block_table().uses_pool(pool_)) {
        throw std::invalid_argument("sequence and prefix cache must use one physical pool");
    }
    if (sequence.num_tokens() != 0) {
        throw std::invalid_argument("cached prefix requires an empty sequence");
    }
    const std::size_t bs = pool_.block_size();
    Tokens prefix;
    prefix.reserve(tokens.size());
    try {
        for (std::size_t begin = 0; tokens.size() - begin >= bs; begin += bs) {
            prefix.insert(prefix.end(), tokens.begin() + begin, tokens.begin() + begin + bs);
            PhysicalBlockHandle hit{};
            if (!pool_.lookup(prefix, hit)) break;
            // lookup's reference is temporary; the table takes its own.
            try {
                sequence.append_cached_full_block(hit);
            } catch (...) {
                pool_.free(hit);
                throw;
            }
            pool_.free(hit);
        }
    } catch (...) {
        while (sequence.tokens_ != 0) {
            sequence.table_.pop_back();
            sequence.tokens_ -= bs;
        }
        throw;
    }
    return sequence.num_tokens();
}

void PrefixCache::publish_computed_block(const SequenceState& sequence, std::size_t logical_block,
                                         const Tokens& prefix) {
    if (!sequence.block_table().uses_pool(pool_)) {
        throw std::invalid_argument("sequence and prefix cache must use one physical pool");
    }
    const std::size_t bs = pool_.block_size();
    if (logical_block >= sequence.num_allocated_blocks() || prefix.size() % bs != 0 ||
        prefix.size() / bs != logical_block + 1 || prefix.size() > sequence.num_tokens()) {
        throw std::invalid_argument("publish requires the exact complete token prefix");
    }
    pool_.publish(sequence.block_handle(logical_block), prefix);
}

TokenLocation append_token_cow(const PagedKVStorage& storage, SequenceState& sequence) {
    if (!storage.uses_pool(sequence.block_table()) ||
        storage.layout().block_size() != sequence.block_size()) {
        throw std::invalid_argument("sequence and KV storage must use one physical pool");
    }
    return sequence.append_token_with_copy(
        [&](PhysicalBlockHandle source, PhysicalBlockHandle destination) {
            storage.copy_block(source, destination);
        });
}

SequenceLifecycle::SequenceLifecycle(RequestID request_id, PhysicalBlockPool& pool,
                                     PagedKVStorage& storage, std::size_t query_heads)
    : storage_(storage), sequence_(std::in_place, request_id, pool), query_heads_(query_heads) {
    if (!storage_.uses_pool(sequence_->block_table()) || query_heads_ == 0 ||
        query_heads_ % storage_.layout().num_kv_heads() != 0) {
        throw std::invalid_argument("invalid sequence lifecycle pool or query head count");
    }
}

const SequenceState& SequenceLifecycle::sequence() const {
    if (finished()) throw std::logic_error("request has finished");
    return *sequence_;
}

void SequenceLifecycle::prefill(std::size_t token_count, const void* key_device,
                                const void* value_device, const float* query_device,
                                float* output_device) {
    if (finished() || prefilled_) throw std::logic_error("request cannot prefill again");
    if (token_count == 0 || !key_device || !value_device || !query_device || !output_device) {
        throw std::invalid_argument("prefill requires tokens and device buffers");
    }
    try {
        sequence_->append_tokens(token_count);
        std::vector<TokenWrite> writes;
        writes.reserve(token_count);
        for (std::size_t t = 0; t < token_count; ++t) writes.push_back({&*sequence_, t});
        write_paged_kv(storage_, key_device, value_device, build_slot_mapping(writes));
        paged_attention(storage_, *sequence_, query_device, output_device, token_count,
                        query_heads_);
        prefilled_ = true;
    } catch (...) {
        abort_after_failure();
        throw;
    }
}

TokenLocation SequenceLifecycle::decode(const void* key_device, const void* value_device,
                                        const float* query_device, float* output_device) {
    if (finished() || !prefilled_) throw std::logic_error("request must prefill before decode");
    if (!key_device || !value_device || !query_device || !output_device) {
        throw std::invalid_argument("decode requires device buffers");
    }
    try {
        const std::size_t position = sequence_->num_tokens();
        const auto location = append_token_cow(storage_, *sequence_);
        write_paged_kv(storage_, key_device, value_device,
                       build_slot_mapping({{&*sequence_, position}}));
        paged_attention(storage_, *sequence_, query_device, output_device, 1, query_heads_);
        return location;
    } catch (...) {
        abort_after_failure();
        throw;
    }
}

void SequenceLifecycle::finish() noexcept {
    sequence_.reset();  // the BlockTable returns every page reference
    prefilled_ = false;
}

void SequenceLifecycle::abort_after_failure() noexcept {
    // A failed call may have left work queued on the pages about to be freed.
    int previous = 0;
    if (kvflux_get_device(&previous) == KVFLUX_OK &&
        kvflux_set_device(storage_.device()) == KVFLUX_OK) {
        (void)kvflux_device_synchronize();
        (void)kvflux_set_device(previous);
    }
    finish();
}

} // namespace kvflux::v2
