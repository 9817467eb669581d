// Public data-path calls of the C++ layer. Validation order and exception
// types follow the reference; each call uploads its metadata once, launches
// the gfx950 kernel through the C ABI and waits for the default stream:
//   write_paged_kv         reference src/v2/paged_kv_write.cu:101-139
//   read_paged_kv          reference src/v2/paged_kv_read.cu:106-155
//   paged_attention        reference src/v2/paged_attention.cu:193-246
//   paged_attention_batch  reference src/v2/paged_attention.cu:248-313
#include "kvflux/v2/batch_block_table.h"
#include "kvflux/v2/paged_attention.h"
#include "kvflux/v2/paged_kv_read.h"
#include "kvflux/v2/paged_kv_write.h"

#include "device_runtime.h"

#include <algorithm>
#include <stdexcept>

namespace kvflux::v2 {
namespace {

using detail::abi_dtype;
using detail::attention_workspace;
using detail::prefill_workspace;
using detail::check;
using detail::mul_checked;
using detail::validate_q_o;

// Range and duplicate check in mapping order, so the first offending slot
// decides the exception exactly as the reference's in-order scan does.
void validate_slots(const PagedKVLayout& layout, const SlotMapping& slots,
                    std::vector<std::uint64_t>& seen) {
    const std::uint64_t count = layout.slot_count();
    if (seen.size() * 64 < count) seen.assign((count + 63) / 64, 0);
    std::size_t checked = 0;
    auto unmark = [&] {
        for (std::size_t i = 0; i < checked; ++i) seen[slots[i] >> 6] = 0;
    };
    for (; checked < slots.size(); ++checked) {
        const auto slot = slots[checked];
        if (slot >= count) {
            unmark();
            throw std::out_of_range("KV write slot out of range");
        }
        auto& word = seen[slot >> 6];
        const std::uint64_t bit = std::uint64_t{1} << (slot & 63);
        if (word & bit) {
            unmark();
            throw std::invalid_argument("duplicate KV write slot");
        }
        word |= bit;
    }
    unmark();
}

void finish(const char* operation) {
    check(kvflux_stream_synchronize(nullptr), operation);
}

} // namespace

void write_paged_kv(PagedKVStorage& storage, const void* key_new_device,
                    const void* value_new_device, const SlotMapping& slot_mapping) {
    if (slot_mapping.empty()) return;
    if (!key_new_device || !value_new_device) {
        throw std::invalid_argument("K_new and V_new device pointers are required");
    }
    const auto& layout = storage.layout();
    validate_slots(layout, slot_mapping, storage.scratch().seen_slots);
    const auto elements = mul_checked(mul_checked(slot_mapping.size(), layout.num_kv_heads(),
                                                  "paged KV write size overflow"),
                                      layout.head_size(), "paged KV write size overflow");
    (void)mul_checked(elements, layout.element_bytes(), "paged KV write size overflow");
    const auto slot_bytes = mul_checked(slot_mapping.size(), sizeof(PhysicalSlot),
                                        "paged KV write size overflow");

    detail::DeviceGuard guard(storage.device());
    detail::require_device_pointer(key_new_device, storage.device(), "K_new");
    detail::require_device_pointer(value_new_device, storage.device(), "V_new");
    const auto dev = storage.scratch().upload({{slot_mapping.data(), slot_bytes}});
    check(kvflux_write_paged_kv(storage.key_base(), storage.value_base(), layout.num_blocks(),
                                layout.num_kv_heads(), layout.block_size(), layout.head_size(),
                                abi_dtype(layout.dtype()), key_new_device, value_new_device,
                                dev[0], slot_mapping.size(), nullptr),
          "paged KV write kernel launch");
    finish("paged KV write synchronize");
}

namespace {

// Shared tail of read_paged_kv / read_paged_kv_batch once the packed token
// count and the flat table are known.
void launch_gather(const PagedKVStorage& storage, const std::vector<PhysicalBlockID>& table,
                   std::size_t width, const std::vector<std::uint64_t>& lengths,
                   const std::vector<std::uint64_t>& offsets, std::size_t total_tokens,
                   void* key_out, void* value_out) {
    const auto& layout = storage.layout();
    for (const auto block : table) {
        if (block != BatchBlockTable::invalid_block() && block >= layout.num_blocks()) {
            throw std::out_of_range("KV read block out of range");
        }
    }
    const auto elements = mul_checked(mul_checked(total_tokens, layout.num_kv_heads(),
                                                  "paged KV read size overflow"),
                                      layout.head_size(), "paged KV read size overflow");
    const auto out_bytes = mul_checked(elements, layout.element_bytes(),
                                       "paged KV read size overflow");
    const auto table_bytes = mul_checked(table.size(), sizeof(PhysicalBlockID),
                                         "paged KV read size overflow");

    detail::DeviceGuard guard(storage.device());
    detail::require_device_pointer(key_out, storage.device(), "K_out");
    detail::require_device_pointer(value_out, storage.device(), "V_out");
    if (detail::overlaps(key_out, out_bytes, value_out, out_bytes) ||
        detail::overlaps(key_out, out_bytes, storage.key_base(), layout.total_bytes()) ||
        detail::overlaps(value_out, out_bytes, storage.key_base(), layout.total_bytes())) {
        throw std::invalid_argument("KV read outputs must not overlap each other or the cache");
    }
    // Exclusive scan of the page counts: one workgroup per live page.
    std::vector<std::uint64_t> page_starts(lengths.size());
    std::uint64_t pages = 0;
    for (std::size_t i = 0; i < lengths.size(); ++i) {
        page_starts[i] = pages;
        pages += (lengths[i] + layout.block_size() - 1) / layout.block_size();
    }
    const auto dev = storage.scratch().upload({{table.data(), table_bytes},
                                               {lengths.data(), lengths.size() * 8},
                                               {offsets.data(), offsets.size() * 8},
                                               {page_starts.data(), page_starts.size() * 8}});
    check(kvflux_gather_paged_kv_live(storage.key_base(), storage.value_base(), layout.num_blocks(),
                                      layout.num_kv_heads(), layout.block_size(), layout.head_size(),
                                      abi_dtype(layout.dtype()), dev[0], width, dev[1], dev[2], dev[3],
                                      lengths.size(), pages, key_out, value_out, nullptr),
          "paged KV read kernel launch");
    finish("paged KV read synchronize");
}

} // namespace

void read_paged_kv(const PagedKVStorage& storage, const SequenceState& sequence,
                   void* key_out_device, void* value_out_device) {
    if (!storage.uses_pool(sequence.block_table())) {
        throw std::invalid_argument("sequence and KV storage must use one physical pool");
    }
    if (sequence.block_size() != storage.layout().block_size()) {
        throw std::invalid_argument("sequence and KV storage block sizes differ");
    }
    if (sequence.num_tokens() == 0) return;
    if (!key_out_device || !value_out_device) {
        throw std::invalid_argument("K and V output device pointers are required");
    }
    const auto table = build_read_block_table(sequence);
    launch_gather(storage, table, table.size(), {sequence.num_tokens()}, {0},
                  sequence.num_tokens(), key_out_device, value_out_device);
}

void read_paged_kv_batch(const PagedKVStorage& storage,
                         const std::vector<const SequenceState*>& sequences,
                         void* key_out_device, void* value_out_device) {
    const auto batch = build_batch_block_table(sequences);
    std::vector<std::uint64_t> lengths, offsets;
    std::size_t total = 0;
    for (std::size_t r = 0; r < sequences.size(); ++r) {
        if (!storage.uses_pool(sequences[r]->block_table())) {
            throw std::invalid_argument("sequence and KV storage must use one physical pool");
        }
        if (sequences[r]->block_size() != storage.layout().block_size()) {
            throw std::invalid_argument("sequence and KV storage block sizes differ");
        }
        lengths.push_back(batch.sequence_lengths()[r]);
        offsets.push_back(total);
        if (batch.sequence_lengths()[r] > std::numeric_limits<std::size_t>::max() - total) {
            throw std::overflow_error("paged KV read size overflow");
        }
        total += batch.sequence_lengths()[r];
    }
    if (total == 0) return;
    if (!key_out_device || !value_out_device) {
        throw std::invalid_argument("K and V output device pointers are required");
    }
    launch_gather(storage, batch.block_table(), batch.max_blocks_per_sequence(), lengths,
                  offsets, total, key_out_device, value_out_device);
}

namespace {

// Whether a call's shape is inside the MFMA prefill's limits (the same limits
// kvflux_paged_prefill checks), so its workspace is reserved only for calls
// that will use it.
bool prefill_shape_ok(const PagedKVLayout& layout, std::size_t query_tokens, std::size_t kv_len) {
    if (query_tokens == 0) return false;
    if (layout.head_size() != 64 && layout.head_size() != 128 && layout.head_size() != 256) return false;
    if (layout.dtype() == DType::Float32 && layout.head_size() == 256) return false;
    const std::size_t bs = layout.block_size();
    if (bs > 256 || (bs & (bs - 1)) != 0) return false;  // a power of two up to 256
    return layout.num_blocks() <= 0x7fffffffULL && layout.num_kv_heads() <= 65535 && kv_len <= 0x7fffffffULL &&
           layout.page_bytes() <= 0xffffffffULL;
}

// The rounded (2e-2) MFMA prefill: Fast, or Auto from 16 query tokens on.
// FP32 caches take FP32 MFMAs there, whose products are exact.
bool prefill_eligible(const PagedKVLayout& layout, std::size_t query_tokens, std::size_t kv_len,
                      AttentionPrecision precision) {
    if (precision == AttentionPrecision::Exact) return false;
    if (precision == AttentionPrecision::Auto && query_tokens < 16) return false;
    return prefill_shape_ok(layout, query_tokens, kv_len);
}

// The exact (1e-5) MFMA prefill: Exact calls of 16 or more query tokens at
// head_size 64 or 128, any cache dtype (fewer tokens run faster on the
// split-K kernel).
bool exact_prefill_eligible(const PagedKVLayout& layout, std::size_t query_tokens, std::size_t kv_len,
                            AttentionPrecision precision) {
    if (precision != AttentionPrecision::Exact || query_tokens < 16) return false;
    if (layout.head_size() == 256) return false;
    return prefill_shape_ok(layout, query_tokens, kv_len);
}

} // namespace

void paged_attention(const PagedKVStorage& storage, const SequenceState& sequence,
                     const float* query_device, float* output_device,
                     std::size_t query_tokens, std::size_t query_heads) {
    paged_attention(storage, sequence, query_device, output_device, query_tokens, query_heads,
                    AttentionPrecision::Exact);
}

void paged_attention(const PagedKVStorage& storage, const SequenceState& sequence,
                     const float* query_device, float* output_device,
                     std::size_t query_tokens, std::size_t query_heads,
                     AttentionPrecision precision) {
    if (!storage.uses_pool(sequence.block_table())) {
        throw std::invalid_argument("sequence and KV storage must use one physical pool");
    }
    const auto& layout = storage.layout();
    if (sequence.block_size() != layout.block_size() || query_heads == 0 ||
        query_heads % layout.num_kv_heads() != 0 || query_tokens > sequence.num_tokens()) {
        throw std::invalid_argument("invalid paged attention shape");
    }
    const auto elements = mul_checked(mul_checked(query_tokens, query_heads,
                                                  "paged attention size overflow"),
                                      layout.head_size(), "paged attention size overflow");
    const auto tensor_bytes = mul_checked(elements, sizeof(float), "paged attention size overflow");
    if (query_tokens == 0) return;
    if (!query_device || !output_device) {
        throw std::invalid_argument("Q and attention output device pointers are required");
    }
    const auto table = build_read_block_table(sequence);
    for (const auto block : table) {
        if (block >= layout.num_blocks()) throw std::out_of_range("attention block out of range");
    }
    const auto table_bytes = mul_checked(table.size(), sizeof(PhysicalBlockID),
                                         "paged attention size overflow");
    detail::DeviceGuard guard(storage.device());
    validate_q_o(storage, query_device, output_device, tensor_bytes);
    const auto dev = storage.scratch().upload({{table.data(), table_bytes}});
    bool launched = false;
    const bool exact_mfma = exact_prefill_eligible(layout, query_tokens, sequence.num_tokens(), precision);
    if (exact_mfma || prefill_eligible(layout, query_tokens, sequence.num_tokens(), precision)) {
        std::size_t ws_bytes = 0;
        void* ws = prefill_workspace(storage, query_tokens, sequence.num_tokens(), query_heads, &ws_bytes);
        const auto launch = exact_mfma ? kvflux_paged_prefill_exact : kvflux_paged_prefill_split;
        const int status = launch(
            storage.key_base(), storage.value_base(), layout.num_blocks(), layout.num_kv_heads(),
            layout.block_size(), layout.head_size(), abi_dtype(layout.dtype()), dev[0],
            table.size(), sequence.num_tokens(), query_tokens, query_heads, query_device,
            output_device, ws, ws_bytes, nullptr);
        // A shape the MFMA kernel declines runs on the FP32 kernel instead.
        if (status != KVFLUX_ERR_UNSUPPORTED) check(status, "paged prefill kernel launch");
        launched = status == KVFLUX_OK;
    }
    if (!launched) {
        std::size_t ws_bytes = 0;
        void* ws = attention_workspace(storage, query_tokens, sequence.num_tokens(), query_heads,
                                       &ws_bytes);
        check(kvflux_paged_attention(storage.key_base(), storage.value_base(), layout.num_blocks(),
                                     layout.num_kv_heads(), layout.block_size(), layout.head_size(),
                                     abi_dtype(layout.dtype()), dev[0], table.size(), nullptr,
                                     sequence.num_tokens(), query_tokens, query_heads,
                                     query_device, output_device, ws, ws_bytes, nullptr),
              "paged attention kernel launch");
    }
    finish("paged attention synchronize");
}

void paged_attention_batch(const PagedKVStorage& storage,
                           const std::vector<const SequenceState*>& sequences,
                           const float* query_device, float* output_device,
                           std::size_t query_heads) {
    const auto& layout = storage.layout();
    if (query_heads == 0 || query_heads % layout.num_kv_heads() != 0) {
        throw std::invalid_argument("invalid batch attention head count");
    }
    const auto batch = build_batch_block_table(sequences);
    for (std::size_t r = 0; r < sequences.size(); ++r) {
        if (!storage.uses_pool(sequences[r]->block_table()) ||
            sequences[r]->block_size() != layout.block_size() ||
            batch.sequence_lengths()[r] == 0) {
            throw std::invalid_argument("invalid batch attention sequence");
        }
    }
    for (const auto block : batch.block_table()) {
        if (block != BatchBlockTable::invalid_block() && block >= layout.num_blocks()) {
            throw std::out_of_range("batch attention block out of range");
        }
    }
    const auto elements = mul_checked(mul_checked(sequences.size(), query_heads,
                                                  "paged attention size overflow"),
                                      layout.head_size(), "paged attention size overflow");
    const auto tensor_bytes = mul_checked(elements, sizeof(float), "paged attention size overflow");
    if (sequences.empty()) return;
    if (!query_device || !output_device) {
        throw std::invalid_argument("Q and attention output device pointers are required");
    }
    const auto table_bytes = mul_checked(batch.block_table().size(), sizeof(PhysicalBlockID),
                                         "paged attention size overflow");
    detail::DeviceGuard guard(storage.device());
    validate_q_o(storage, query_device, output_device, tensor_bytes);
    std::vector<std::uint64_t> lengths(batch.sequence_lengths().begin(),
                                       batch.sequence_lengths().end());
    const auto dev = storage.scratch().upload({{batch.block_table().data(), table_bytes},
                                               {lengths.data(), lengths.size() * 8}});
    const auto max_len = *std::max_element(lengths.begin(), lengths.end());
    std::size_t ws_bytes = 0;
    void* ws = attention_workspace(storage, sequences.size(), max_len, query_heads, &ws_bytes);
    check(kvflux_paged_attention(storage.key_base(), storage.value_base(), layout.num_blocks(),
                                 layout.num_kv_heads(), layout.block_size(), layout.head_size(),
                                 abi_dtype(layout.dtype()), dev[0],
                                 batch.max_blocks_per_sequence(), dev[1], max_len,
                                 sequences.size(), query_heads, query_device, output_device, ws,
                                 ws_bytes, nullptr),
          "paged attention batch kernel launch");
    finish("paged attention batch synchronize");
}

} // namespace kvflux::v2
