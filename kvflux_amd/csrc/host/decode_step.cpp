// Batched decode-step callers of the data path: batched copy-on-write append,
// the device-resident batch table and the decode step built on both.
// Per-sequence semantics follow the reference's append_token_cow
// (src/v2/copy_on_write.cpp:7-16, SequenceState::append_token_with_copy
// src/v2/sequence_state.cpp:60-90) and SequenceLifecycle::decode
// (src/v2/sequence_lifecycle.cpp:53-69), for a whole batch at once.
#include "kvflux/v2/copy_on_write.h"
#include "kvflux/v2/device_batch_table.h"

#include "device_runtime.h"

#include <algorithm>
#include <limits>
#include <stdexcept>
#include <unordered_map>
#include <unordered_set>

namespace kvflux::v2 {
namespace detail {

// Writes of the batched appends into SequenceState (a friend).
struct SequenceAccess {
    static BlockTable& table(SequenceState& s) noexcept { return s.table_; }
    static void add_token(SequenceState& s) noexcept { ++s.tokens_; }
};

}  // namespace detail

namespace {

using detail::check;

// One reserved append per sequence: the tail page stays (kind Same), a new
// page starts at a block boundary (Boundary), or a shared partial tail is
// replaced by a private copy (Copy). Pages are allocated up front so the
// commit cannot fail.
struct AppendPlan {
    enum Kind : unsigned char { Same, Boundary, Copy };
    PhysicalBlockPool* pool = nullptr;
    std::vector<Kind> kind;
    std::vector<PhysicalBlockHandle> fresh;   // Boundary / Copy pages (one reference each)
    std::vector<std::uint64_t> pairs;         // {source id, destination id} of the copies
    std::vector<TokenLocation> locations;
    bool committed = false;

    AppendPlan() = default;
    AppendPlan(const AppendPlan&) = delete;
    AppendPlan& operator=(const AppendPlan&) = delete;
    ~AppendPlan() {
        if (committed || !pool) return;
        for (std::size_t i = 0; i < fresh.size(); ++i) {
            if (kind[i] != Same) pool->free(fresh[i]);
        }
    }
};

void plan_appends(const PagedKVStorage& storage, const std::vector<SequenceState*>& sequences,
                  AppendPlan& plan) {
    const std::size_t bs = storage.layout().block_size();
    std::unordered_set<const SequenceState*> seen;
    for (const auto* s : sequences) {
        if (!s || !storage.uses_pool(s->block_table()) || s->block_size() != bs) {
            throw std::invalid_argument("sequence and KV storage must use one physical pool");
        }
        if (!seen.insert(s).second) throw std::invalid_argument("a sequence appears twice in the batch");
        if (s->num_tokens() == std::numeric_limits<std::size_t>::max()) {
            throw std::overflow_error("sequence token count overflow");
        }
    }
    if (sequences.empty()) return;
    plan.pool = &sequences.front()->block_table().pool();
    plan.kind.assign(sequences.size(), AppendPlan::Same);
    plan.fresh.resize(sequences.size());
    plan.locations.resize(sequences.size());
    // References each shared tail loses to the copies planned before it, so
    // that the decision for every request is the one append_token_cow makes
    // when the requests are appended one after another in input order (the
    // last holder of a shared tail appends in place).
    std::unordered_map<PhysicalBlockID, std::size_t> released;
    for (std::size_t i = 0; i < sequences.size(); ++i) {
        const SequenceState& s = *sequences[i];
        const std::size_t offset = s.num_tokens() % bs;
        const BlockTable& table = s.block_table();
        if (offset == 0) {
            plan.fresh[i] = plan.pool->allocate();  // CapacityError: the destructor frees the rest
            plan.kind[i] = AppendPlan::Boundary;
            plan.locations[i] = {plan.pool->id(plan.fresh[i]), 0};
            continue;
        }
        const PhysicalBlockID tail = table.physical_id(table.size() - 1);
        std::size_t& gone = released[tail];
        if (table.ref_count(table.size() - 1) - gone > 1) {
            ++gone;
            plan.fresh[i] = plan.pool->allocate();
            plan.kind[i] = AppendPlan::Copy;
            const auto destination = plan.pool->id(plan.fresh[i]);
            plan.pairs.push_back(tail);
            plan.pairs.push_back(destination);
            plan.locations[i] = {destination, offset};
        } else {
            plan.locations[i] = {tail, offset};
        }
    }
}

// Enqueues the copies of a plan (one launch). Sources are live pages of other
// sequences and destinations are fresh, so the batch never overlaps itself.
void enqueue_copies(const PagedKVStorage& storage, const AppendPlan& plan) {
    if (plan.pairs.empty()) return;
    const auto& layout = storage.layout();
    const auto dev = storage.scratch().upload({{plan.pairs.data(), plan.pairs.size() * 8}});
    check(kvflux_copy_pages(storage.key_base(), storage.value_base(), layout.num_blocks(),
                            layout.page_bytes(), dev[0], plan.pairs.size() / 2, nullptr),
          "copy-on-write page copy");
}

void commit(const std::vector<SequenceState*>& sequences, AppendPlan& plan) noexcept {
    for (std::size_t i = 0; i < sequences.size(); ++i) {
        SequenceState& s = *sequences[i];
        BlockTable& table = detail::SequenceAccess::table(s);
        switch (plan.kind[i]) {
        case AppendPlan::Boundary:
            table.append_existing(plan.fresh[i]);  // the table takes its own reference
            plan.pool->free(plan.fresh[i]);
            break;
        case AppendPlan::Copy:
            table.replace_last_owned(plan.fresh[i]);  // hands over the reference
            break;
        case AppendPlan::Same: break;
        }
        detail::SequenceAccess::add_token(s);
    }
    plan.committed = true;
}

}  // namespace

std::vector<TokenLocation> append_tokens_cow(const PagedKVStorage& storage,
                                             const std::vector<SequenceState*>& sequences) {
    AppendPlan plan;
    plan_appends(storage, sequences, plan);
    if (sequences.empty()) return {};
    if (!plan.pairs.empty()) {
        detail::DeviceGuard guard(storage.device());
        try {
            enqueue_copies(storage, plan);
            check(kvflux_stream_synchronize(nullptr), "synchronize copy-on-write");
        } catch (...) {
            (void)kvflux_stream_synchronize(nullptr);
            throw;  // the plan returns its pages; no sequence changed
        }
    }
    commit(sequences, plan);
    return plan.locations;
}

// ---------------------------------------------------------------- DeviceBatchTable

struct DeviceBatchTable::Device {
    detail::DeviceBuffer table, lengths, updates;
    detail::PinnedBuffer staging;
};

namespace {
constexpr std::uint64_t kNoPage = std::numeric_limits<std::uint64_t>::max();
}

DeviceBatchTable::DeviceBatchTable(const PagedKVStorage& storage,
                                   std::vector<SequenceState*> sequences,
                                   std::size_t capacity_blocks)
    : storage_(storage), sequences_(std::move(sequences)), capacity_(capacity_blocks),
      device_(std::make_unique<Device>()) {
    if (capacity_ == 0) throw std::invalid_argument("device batch table needs a row capacity");
    std::unordered_set<const SequenceState*> seen;
    for (const auto* s : sequences_) {
        if (!s || !storage_.uses_pool(s->block_table()) ||
            s->block_size() != storage_.layout().block_size()) {
            throw std::invalid_argument("sequence and KV storage must use one physical pool");
        }
        if (!seen.insert(s).second) throw std::invalid_argument("a sequence appears twice in the batch");
    }
    const auto cells = detail::mul_checked(sequences_.size(), capacity_, "batch table size overflow");
    (void)detail::mul_checked(cells, sizeof(std::uint64_t), "batch table size overflow");
    shadow_.assign(cells, kNoPage);
    lengths_.assign(sequences_.size(), 0);
    blocks_.assign(sequences_.size(), 0);
    refresh();
}

DeviceBatchTable::~DeviceBatchTable() {
    // The buffers belong to the storage's device; free them there.
    int previous = 0;
    const int device = storage_.device();
    const bool switched = kvflux_get_device(&previous) == KVFLUX_OK &&
                          (previous == device || kvflux_set_device(device) == KVFLUX_OK);
    device_.reset();
    if (switched && previous != device) (void)kvflux_set_device(previous);
}

const std::uint64_t* DeviceBatchTable::device_table() const noexcept {
    return static_cast<const std::uint64_t*>(device_->table.data());
}
const std::uint64_t* DeviceBatchTable::device_lengths() const noexcept {
    return static_cast<const std::uint64_t*>(device_->lengths.data());
}

void DeviceBatchTable::upload_all() {
    for (std::size_t r = 0; r < sequences_.size(); ++r) {
        const SequenceState& s = *sequences_[r];
        const std::size_t n = s.num_allocated_blocks();
        if (n > capacity_) throw std::length_error("sequence outgrew the device batch table row");
        std::uint64_t* row = shadow_.data() + r * capacity_;
        std::fill(row, row + capacity_, kNoPage);
        for (std::size_t b = 0; b < n; ++b) row[b] = s.physical_block_id(b);
        lengths_[r] = s.num_tokens();
        blocks_[r] = n;
    }
    const std::size_t table_bytes = shadow_.size() * sizeof(std::uint64_t);
    const std::size_t length_bytes = lengths_.size() * sizeof(std::uint64_t);
    if (sequences_.empty()) return;
    auto* host = static_cast<unsigned char*>(device_->staging.reserve(table_bytes + length_bytes));
    std::memcpy(host, shadow_.data(), table_bytes);
    std::memcpy(host + table_bytes, lengths_.data(), length_bytes);
    void* table = device_->table.reserve(table_bytes);
    void* lengths = device_->lengths.reserve(length_bytes);
    check(kvflux_memcpy_async(table, host, table_bytes, nullptr), "upload batch table");
    check(kvflux_memcpy_async(lengths, host + table_bytes, length_bytes, nullptr),
          "upload batch lengths");
}

void DeviceBatchTable::enqueue_refresh() {
    detail::DeviceGuard guard(storage_.device());
    if (stale_) {
        upload_all();
        stale_ = false;
        return;
    }
    // Records {row, length, block, page}: the entries from each row's former
    // last block on (copy-on-write may have replaced it), and the length.
    std::vector<std::uint64_t> records;
    std::vector<std::uint64_t> next_blocks(sequences_.size());
    for (std::size_t r = 0; r < sequences_.size(); ++r) {
        const SequenceState& s = *sequences_[r];
        const std::size_t n = s.num_allocated_blocks();
        if (n > capacity_) throw std::length_error("sequence outgrew the device batch table row");
        if (n < blocks_[r]) throw std::logic_error("a batch table row lost pages");
        next_blocks[r] = n;
    }
    for (std::size_t r = 0; r < sequences_.size(); ++r) {
        const SequenceState& s = *sequences_[r];
        const std::uint64_t len = s.num_tokens();
        bool wrote = false;
        for (std::size_t b = blocks_[r] ? blocks_[r] - 1 : 0; b < next_blocks[r]; ++b) {
            const std::uint64_t id = s.physical_block_id(b);
            if (shadow_[r * capacity_ + b] == id) continue;
            records.insert(records.end(), {r, len, b, id});
            wrote = true;
        }
        if (!wrote && len != lengths_[r]) records.insert(records.end(), {r, len, kNoPage, 0});
    }
    if (!records.empty()) {
        const std::size_t bytes = records.size() * sizeof(std::uint64_t);
        auto* host = device_->staging.reserve(bytes);
        std::memcpy(host, records.data(), bytes);
        void* dev = device_->updates.reserve(bytes);
        try {
            check(kvflux_memcpy_async(dev, host, bytes, nullptr), "upload batch table updates");
            check(kvflux_table_apply(static_cast<std::uint64_t*>(device_->table.data()), capacity_,
                                     static_cast<std::uint64_t*>(device_->lengths.data()),
                                     sequences_.size(), static_cast<const std::uint64_t*>(dev),
                                     records.size() / 4, nullptr),
                  "apply batch table updates");
        } catch (...) {
            stale_ = true;  // the device copy may be half updated
            throw;
        }
    }
    for (std::size_t i = 0; i < records.size(); i += 4) {
        if (records[i + 2] != kNoPage) shadow_[records[i] * capacity_ + records[i + 2]] = records[i + 3];
    }
    for (std::size_t r = 0; r < sequences_.size(); ++r) {
        lengths_[r] = sequences_[r]->num_tokens();
        blocks_[r] = next_blocks[r];
    }
}

void DeviceBatchTable::refresh() {
    detail::DeviceGuard guard(storage_.device());
    try {
        enqueue_refresh();
        check(kvflux_stream_synchronize(nullptr), "synchronize batch table refresh");
    } catch (...) {
        (void)kvflux_stream_synchronize(nullptr);
        stale_ = true;
        throw;
    }
}

// ---------------------------------------------------------------- attention and decode step

namespace {

std::size_t validate_batch_attention(const PagedKVStorage& storage, const DeviceBatchTable& batch,
                                     const float* query, float* output, std::size_t query_heads) {
    const auto& layout = storage.layout();
    if (query_heads == 0 || query_heads % layout.num_kv_heads() != 0) {
        throw std::invalid_argument("invalid batch attention head count");
    }
    const auto elements = detail::mul_checked(
        detail::mul_checked(batch.rows(), query_heads, "paged attention size overflow"),
        layout.head_size(), "paged attention size overflow");
    const auto bytes = detail::mul_checked(elements, sizeof(float), "paged attention size overflow");
    if (batch.rows() == 0) return bytes;
    if (!query || !output) {
        throw std::invalid_argument("Q and attention output device pointers are required");
    }
    detail::validate_q_o(storage, query, output, bytes);
    return bytes;
}

void enqueue_batch_attention(const PagedKVStorage& storage, const DeviceBatchTable& batch,
                             const float* query, float* output, std::size_t query_heads) {
    const auto& layout = storage.layout();
    const auto& lengths = batch.lengths();
    if (std::find(lengths.begin(), lengths.end(), 0) != lengths.end()) {
        throw std::invalid_argument("invalid batch attention sequence");
    }
    const std::size_t max_len = *std::max_element(lengths.begin(), lengths.end());
    std::size_t ws_bytes = 0;
    void* ws = detail::attention_workspace(storage, batch.rows(), max_len, query_heads, &ws_bytes);
    check(kvflux_paged_attention(storage.key_base(), storage.value_base(), layout.num_blocks(),
                                 layout.num_kv_heads(), layout.block_size(), layout.head_size(),
                                 detail::abi_dtype(layout.dtype()), batch.device_table(),
                                 batch.capacity_blocks(), batch.device_lengths(), max_len,
                                 batch.rows(), query_heads, query, output, ws, ws_bytes, nullptr),
          "paged attention batch kernel launch");
}

}  // namespace

void paged_attention_batch(const PagedKVStorage& storage, const DeviceBatchTable& batch,
                           const float* query_device, float* output_device,
                           std::size_t query_heads) {
    detail::DeviceGuard guard(storage.device());
    validate_batch_attention(storage, batch, query_device, output_device, query_heads);
    if (batch.rows() == 0) return;
    enqueue_batch_attention(storage, batch, query_device, output_device, query_heads);
    check(kvflux_stream_synchronize(nullptr), "paged attention batch synchronize");
}

std::vector<TokenLocation> decode_step(PagedKVStorage& storage, DeviceBatchTable& batch,
                                       const void* key_new_device, const void* value_new_device,
                                       const float* query_device, float* output_device,
                                       std::size_t query_heads) {
    const auto& layout = storage.layout();
    const auto& sequences = batch.sequences();
    detail::DeviceGuard guard(storage.device());
    validate_batch_attention(storage, batch, query_device, output_device, query_heads);
    if (sequences.empty()) return {};
    if (!key_new_device || !value_new_device) {
        throw std::invalid_argument("K_new and V_new device pointers are required");
    }
    detail::require_device_pointer(key_new_device, storage.device(), "K_new");
    detail::require_device_pointer(value_new_device, storage.device(), "V_new");
    for (const auto* s : sequences) {
        if (s->num_tokens() % layout.block_size() == 0 &&
            s->num_allocated_blocks() + 1 > batch.capacity_blocks()) {
            throw std::length_error("sequence outgrew the device batch table row");
        }
    }
    AppendPlan plan;
    plan_appends(storage, sequences, plan);
    try {
        enqueue_copies(storage, plan);
    } catch (...) {
        (void)kvflux_stream_synchronize(nullptr);
        throw;  // nothing changed; the plan returns its pages
    }
    commit(sequences, plan);
    try {
        batch.enqueue_refresh();
        check(kvflux_write_paged_kv_tail(storage.key_base(), storage.value_base(), layout.num_blocks(),
                                         layout.num_kv_heads(), layout.block_size(),
                                         layout.head_size(), detail::abi_dtype(layout.dtype()),
                                         key_new_device, value_new_device, batch.device_table(),
                                         batch.capacity_blocks(), batch.device_lengths(),
                                         batch.rows(), nullptr),
              "decode step KV write");
        enqueue_batch_attention(storage, batch, query_device, output_device, query_heads);
        check(kvflux_stream_synchronize(nullptr), "decode step synchronize");
    } catch (...) {
        (void)kvflux_stream_synchronize(nullptr);
        throw;
    }
    return plan.locations;
}

} // namespace kvflux::v2
