// Callers of the data path, with the reference's contracts:
//   PrefixCache        include/kvflux/v2/prefix_cache.h:9-27
//   append_token_cow   include/kvflux/v2/copy_on_write.h:7-10
//   SequenceLifecycle  include/kvflux/v2/sequence_lifecycle.h:12-47
// Prefix attachment keeps each lookup's reference as the sequence's own
// (no retain/release pair per block), the single-request copy-on-write
// append is the one-request case of the batched append (one copy launch),
// and the lifecycle writes a prompt's slots straight from its page list.
#include "kvflux/v2/copy_on_write.h"
#include "kvflux/v2/device_batch_table.h"
#include "kvflux/v2/paged_attention.h"
#include "kvflux/v2/paged_kv_read.h"
#include "kvflux/v2/paged_kv_write.h"
#include "kvflux/v2/prefix_cache.h"
#include "kvflux/v2/sequence_lifecycle.h"

#include "device_runtime.h"
#include "pending_refs.h"

#include <limits>
#include <stdexcept>
#include <vector>

namespace kvflux::v2 {

// ---------------------------------------------------------------- prefix cache
std::size_t PrefixCache::attach_cached_prefix(SequenceState& sequence, const Tokens& tokens) {
    if (!sequence.block_table().uses_pool(pool_)) {
        throw std::invalid_argument("prefix cache and sequence use different physical pools");
    }
    if (sequence.num_tokens() != 0) throw std::invalid_argument("a cached prefix attaches to an empty sequence only");
    const std::size_t bs = pool_.block_size();
    const std::size_t whole_blocks = tokens.size() / bs;
    // Hits in order until the first miss. Each lookup's reference becomes the
    // sequence's; on failure they go back last hit first.
    auto hits = host::pending_refs([this](PhysicalBlockHandle h) { pool_.free(h); }, whole_blocks,
                                   host::Undo::InReverseOrder);
    Tokens prefix;
    prefix.reserve(whole_blocks * bs);
    for (std::size_t b = 0; b < whole_blocks; ++b) {
        prefix.insert(prefix.end(), tokens.begin() + static_cast<std::ptrdiff_t>(b * bs),
                      tokens.begin() + static_cast<std::ptrdiff_t>((b + 1) * bs));
        PhysicalBlockHandle hit{};
        if (!pool_.lookup(prefix, hit)) break;
        hits.add(hit);
    }
    sequence.reserve_blocks(hits.size());
    sequence.adopt_cached_blocks(hits.commit());
    return sequence.num_tokens();
}

void PrefixCache::publish_computed_block(const SequenceState& sequence, std::size_t logical_block,
                                         const Tokens& prefix) {
    if (!sequence.block_table().uses_pool(pool_)) {
        throw std::invalid_argument("prefix cache and sequence use different physical pools");
    }
    const std::size_t bs = pool_.block_size();
    // `prefix` must be exactly the tokens from the sequence start through the
    // end of `logical_block`, all of them already in the sequence.
    const bool exact = logical_block < sequence.num_allocated_blocks() && prefix.size() % bs == 0 &&
                       prefix.size() / bs == logical_block + 1 && prefix.size() <= sequence.num_tokens();
    if (!exact) throw std::invalid_argument("publish needs the complete token prefix of that block");
    pool_.publish(sequence.block_handle(logical_block), prefix);
}

// ---------------------------------------------------------------- copy-on-write append
TokenLocation append_token_cow(const PagedKVStorage& storage, SequenceState& sequence) {
    // The batch of one makes the decision append_token_with_copy makes
    // (copy a shared partial tail, else append in place) and copies with the
    // same kernel a decode batch uses; it returns after the copy has landed.
    return append_tokens_cow(storage, {&sequence}).front();
}

// ---------------------------------------------------------------- lifecycle
namespace {

// Slots of tokens [0, n) of `sequence`, in order (the prompt's write).
SlotMapping prompt_slots(const SequenceState& sequence, std::size_t n) {
    const ReadBlockTable pages = build_read_block_table(sequence);
    const auto bs = static_cast<PhysicalSlot>(sequence.block_size());
    SlotMapping slots(n);
    for (std::size_t t = 0; t < n; ++t) {
        const auto page = static_cast<PhysicalSlot>(pages[t / sequence.block_size()]);
        const auto offset = static_cast<PhysicalSlot>(t % sequence.block_size());
        if (page > (std::numeric_limits<PhysicalSlot>::max() - offset) / bs) {
            throw std::overflow_error("slot number does not fit in 64 bits");
        }
        slots[t] = page * bs + offset;
    }
    return slots;
}

} // namespace

SequenceLifecycle::SequenceLifecycle(RequestID request_id, PhysicalBlockPool& pool, PagedKVStorage& storage,
                                     std::size_t query_heads, AttentionPrecision precision)
    : storage_(storage), sequence_(std::in_place, request_id, pool), query_heads_(query_heads),
      precision_(precision) {
    const std::size_t kv_heads = storage_.layout().num_kv_heads();
    const bool shape_ok = query_heads_ != 0 && query_heads_ % kv_heads == 0;
    if (!storage_.uses_pool(sequence_->block_table()) || !shape_ok) {
        throw std::invalid_argument("lifecycle needs the storage's pool and a multiple of its kv heads");
    }
}

const SequenceState& SequenceLifecycle::sequence() const {
    if (finished()) throw std::logic_error("the request has finished");
    return *sequence_;
}

template <typename Step>
auto SequenceLifecycle::guarded(Step&& step) -> decltype(step()) {
    try {
        return step();
    } catch (...) {
        abort_after_failure();
        throw;
    }
}

void SequenceLifecycle::prefill(std::size_t token_count, const void* key_device, const void* value_device,
                                const float* query_device, float* output_device) {
    if (finished() || prefilled_) throw std::logic_error("prefill runs once, before any decode");
    if (token_count == 0 || !key_device || !value_device || !query_device || !output_device) {
        throw std::invalid_argument("prefill needs tokens and four device buffers");
    }
    guarded([&] {
        SequenceState& s = *sequence_;
        s.append_tokens(token_count);
        write_paged_kv(storage_, key_device, value_device, prompt_slots(s, token_count));
        paged_attention(storage_, s, query_device, output_device, token_count, query_heads_, precision_);
    });
    prefilled_ = true;
}

TokenLocation SequenceLifecycle::decode(const void* key_device, const void* value_device,
                                        const float* query_device, float* output_device) {
    if (finished() || !prefilled_) throw std::logic_error("decode follows a prefill of a live request");
    if (!key_device || !value_device || !query_device || !output_device) {
        throw std::invalid_argument("decode needs four device buffers");
    }
    return guarded([&] {
        SequenceState& s = *sequence_;
        const TokenLocation at = append_token_cow(storage_, s);
        const auto bs = static_cast<PhysicalSlot>(s.block_size());
        write_paged_kv(storage_, key_device, value_device,
                       SlotMapping{static_cast<PhysicalSlot>(at.physical_block) * bs + at.offset_in_block});
        paged_attention(storage_, s, query_device, output_device, 1, query_heads_, precision_);
        return at;
    });
}

void SequenceLifecycle::finish() noexcept {
    sequence_.reset();  // the table returns every page reference
    prefilled_ = false;
}

void SequenceLifecycle::abort_after_failure() noexcept {
    // Work a failed call left queued may still touch the pages about to be
    // returned: wait for the storage's device first.
    int caller_device = 0;
    if (kvflux_get_device(&caller_device) == KVFLUX_OK) {
        if (kvflux_set_device(storage_.device()) == KVFLUX_OK) {
            (void)kvflux_device_synchronize();
            (void)kvflux_set_device(caller_device);
        }
    }
    finish();
}

} // namespace kvflux::v2
