// v2 control plane: page pool, per-sequence tables and the integer metadata
// the device kernels consume. Observable behaviour (page ids, reference
// counts, exception types, rollback) follows the reference:
//   PhysicalBlockPool   src/physical_block_pool.cpp:8-50
//   BlockTable          src/v2/block_table.cpp:8-101
//   SequenceState       src/v2/sequence_state.cpp:9-113
//   build_slot_mapping  src/v2/slot_mapping.cpp:8-31
//   BatchBlockTable     src/v2/batch_block_table.cpp:8-48
//   build_read_block_table src/v2/paged_kv_read_table.cpp:5-12
//   PagedKVLayout       src/v2/paged_kv_layout.cpp:27-68
#include "kvflux/physical_block_pool.h"
#include "kvflux/v2/batch_block_table.h"
#include "kvflux/v2/block_table.h"
#include "kvflux/v2/paged_kv_layout.h"
#include "kvflux/v2/paged_kv_read.h"
#include "kvflux/v2/sequence_state.h"
#include "kvflux/v2/slot_mapping.h"

#include <limits>
#include <stdexcept>
#include <utility>

namespace kvflux {

// ---------------------------------------------------------------- pool
PhysicalBlockPool::PhysicalBlockPool(std::size_t capacity, std::size_t block_size,
                                     BlockManager::Hasher hasher)
    : manager_(capacity, block_size, std::move(hasher)) {}

PhysicalBlockHandle PhysicalBlockPool::allocate() { return manager_.allocate(); }
void PhysicalBlockPool::retain(PhysicalBlockHandle handle) { manager_.retain(handle); }
void PhysicalBlockPool::free(PhysicalBlockHandle handle) { manager_.release(handle); }
void PhysicalBlockPool::publish(PhysicalBlockHandle handle, const Tokens& prefix) {
    manager_.publish(handle, prefix);
}
bool PhysicalBlockPool::lookup(const Tokens& prefix, PhysicalBlockHandle& out) {
    return manager_.lookup(prefix, out);
}
bool PhysicalBlockPool::is_published(PhysicalBlockHandle handle) const {
    return manager_.is_published(handle);
}

void PhysicalBlockPool::ids(const PhysicalBlockHandle* handles, std::size_t n, PhysicalBlockID* out) const {
    manager_.referenced_ids(handles, n, out);
}

PhysicalBlockID PhysicalBlockPool::id(PhysicalBlockHandle handle) const {
    // ref_count validates range, liveness and generation; an idle published
    // page (zero references) is not addressable either.
    if (manager_.ref_count(handle) == 0) {
        throw std::invalid_argument("physical block has no active reference");
    }
    return handle.id;
}

std::size_t PhysicalBlockPool::ref_count(PhysicalBlockHandle handle) const {
    return manager_.ref_count(handle);
}
std::size_t PhysicalBlockPool::capacity() const noexcept { return manager_.capacity(); }
std::size_t PhysicalBlockPool::block_size() const noexcept { return manager_.block_size(); }
std::size_t PhysicalBlockPool::available() const noexcept {
    const auto s = manager_.stats();
    return s.free + s.cached_idle;
}

} // namespace kvflux

namespace kvflux::v2 {

// ---------------------------------------------------------------- BlockTable
BlockTable::BlockTable(PhysicalBlockPool& pool) noexcept : pool_(&pool) {}

BlockTable::~BlockTable() noexcept { clear(); }

BlockTable::BlockTable(BlockTable&& other) noexcept
    : pool_(std::exchange(other.pool_, nullptr)), entries_(std::move(other.entries_)) {
    other.entries_.clear();
}

BlockTable& BlockTable::operator=(BlockTable&& other) noexcept {
    if (this == &other) return *this;
    clear();  // return our references before adopting the other table's
    pool_ = std::exchange(other.pool_, nullptr);
    entries_ = std::move(other.entries_);
    other.entries_.clear();
    return *this;
}

PhysicalBlockID BlockTable::append_new() {
    if (!pool_) throw std::logic_error("cannot append to a moved-from block table");
    const auto handle = pool_->allocate();
    try {
        entries_.push_back(handle);
    } catch (...) {
        pool_->free(handle);
        throw;
    }
    return handle.id;
}

void BlockTable::append_existing(PhysicalBlockHandle handle) {
    if (!pool_) throw std::logic_error("cannot append to a moved-from block table");
    pool_->retain(handle);
    try {
        entries_.push_back(handle);
    } catch (...) {
        pool_->free(handle);
        throw;
    }
}

void BlockTable::append_shared(const BlockTable& source, std::size_t logical_block) {
    if (!pool_ || pool_ != source.pool_) {
        throw std::invalid_argument("block tables must use the same physical pool");
    }
    // Copy the handle first: `source` may be *this and push_back may reallocate.
    const PhysicalBlockHandle handle = source.entries_.at(logical_block);
    append_existing(handle);
}

PhysicalBlockID BlockTable::physical_id(std::size_t logical_block) const {
    return pool_->id(entries_.at(logical_block));
}

void BlockTable::physical_ids(PhysicalBlockID* out) const {
    if (!entries_.empty()) pool_->ids(entries_.data(), entries_.size(), out);
}

PhysicalBlockHandle BlockTable::handle(std::size_t logical_block) const {
    const auto h = entries_.at(logical_block);
    (void)pool_->id(h);
    return h;
}

std::size_t BlockTable::ref_count(std::size_t logical_block) const {
    return pool_->ref_count(entries_.at(logical_block));
}

PhysicalBlockPool& BlockTable::pool() const {
    if (!pool_) throw std::logic_error("moved-from block table has no pool");
    return *pool_;
}

void BlockTable::pop_back() {
    if (entries_.empty()) throw std::out_of_range("block table is empty");
    pool_->free(entries_.back());
    entries_.pop_back();
}

void BlockTable::replace_last_owned(PhysicalBlockHandle new_handle) {
    if (entries_.empty()) throw std::out_of_range("block table is empty");
    (void)pool_->id(new_handle);
    if (new_handle == entries_.back() || pool_->ref_count(new_handle) != 1 ||
        pool_->is_published(new_handle)) {
        throw std::invalid_argument("replacement block must be private and unpublished");
    }
    // Release first (it validates the old handle); the assignment cannot
    // throw, so on failure the caller still owns new_handle.
    pool_->free(entries_.back());
    entries_.back() = new_handle;
}

void BlockTable::clear() noexcept {
    for (const auto handle : entries_) pool_->free(handle);
    entries_.clear();
}

// ---------------------------------------------------------------- SequenceState
SequenceState::SequenceState(RequestID request_id, PhysicalBlockPool& pool) noexcept
    : id_(request_id), block_size_(pool.block_size()), table_(pool) {}

SequenceState::SequenceState(SequenceState&& other) noexcept
    : id_(other.id_), tokens_(std::exchange(other.tokens_, 0)),
      block_size_(other.block_size_), table_(std::move(other.table_)) {}

SequenceState& SequenceState::operator=(SequenceState&& other) noexcept {
    if (this == &other) return *this;
    table_ = std::move(other.table_);
    id_ = other.id_;
    tokens_ = std::exchange(other.tokens_, 0);
    block_size_ = other.block_size_;
    return *this;
}

std::size_t SequenceState::last_block_num_tokens() const noexcept {
    return tokens_ == 0 ? 0 : (tokens_ - 1) % block_size_ + 1;
}

void SequenceState::append_tokens(std::size_t count) {
    if (count == 0) return;
    if (count > std::numeric_limits<std::size_t>::max() - tokens_) {
        throw std::overflow_error("sequence token count overflow");
    }
    if (tokens_ % block_size_ != 0 && table_.ref_count(table_.size() - 1) > 1) {
        throw std::logic_error("shared partial block requires copy-on-write");
    }
    const std::size_t total = tokens_ + count;
    const std::size_t needed = total / block_size_ + (total % block_size_ != 0);
    const std::size_t before = table_.size();
    try {
        while (table_.size() < needed) table_.append_new();
    } catch (...) {
        while (table_.size() > before) table_.pop_back();
        throw;
    }
    tokens_ = total;
}

TokenLocation SequenceState::append_token() {
    const std::size_t position = tokens_;
    append_tokens(1);
    return token_location(position);
}

SequenceState SequenceState::fork_shared(RequestID new_request_id) const {
    SequenceState fork(new_request_id, table_.pool());
    // On failure `fork` is destroyed and returns what it already retained.
    for (std::size_t i = 0; i < table_.size(); ++i) fork.table_.append_shared(table_, i);
    fork.tokens_ = tokens_;
    return fork;
}

TokenLocation SequenceState::append_token_with_copy(const BlockCopier& copy) {
    if (tokens_ == std::numeric_limits<std::size_t>::max()) {
        throw std::overflow_error("sequence token count overflow");
    }
    const std::size_t offset = tokens_ % block_size_;
    if (offset == 0 || table_.ref_count(table_.size() - 1) == 1) return append_token();
    if (!copy) throw std::invalid_argument("copy callback is required for shared partial block");

    const auto shared_tail = table_.handle(table_.size() - 1);
    auto& pool = table_.pool();
    const auto fresh = pool.allocate();
    try {
        copy(shared_tail, fresh);  // the mapping changes only after the copy
        table_.replace_last_owned(fresh);
    } catch (...) {
        pool.free(fresh);
        throw;
    }
    ++tokens_;
    return {fresh.id, offset};
}

void SequenceState::append_cached_full_block(PhysicalBlockHandle handle) {
    if (tokens_ % block_size_ != 0 ||
        block_size_ > std::numeric_limits<std::size_t>::max() - tokens_) {
        throw std::invalid_argument("cached block requires a complete preceding prefix");
    }
    table_.append_existing(handle);
    tokens_ += block_size_;
}

PhysicalBlockID SequenceState::physical_block_id(std::size_t logical_block) const {
    return table_.physical_id(logical_block);
}

void SequenceState::physical_block_ids(PhysicalBlockID* out) const { table_.physical_ids(out); }

PhysicalBlockHandle SequenceState::block_handle(std::size_t logical_block) const {
    return table_.handle(logical_block);
}

TokenLocation SequenceState::token_location(std::size_t token_index) const {
    if (token_index >= tokens_) throw std::out_of_range("token index is outside sequence");
    return {physical_block_id(token_index / block_size_), token_index % block_size_};
}

// ---------------------------------------------------------------- slot mapping
SlotMapping build_slot_mapping(const std::vector<TokenWrite>& batch) {
    static_assert(sizeof(std::size_t) <= sizeof(PhysicalSlot), "size_t must fit in a slot");
    SlotMapping slots;
    slots.reserve(batch.size());
    if (batch.empty()) return slots;
    if (!batch.front().sequence) throw std::invalid_argument("null sequence in slot mapping");
    const auto& first = batch.front().sequence->block_table();
    for (const auto& write : batch) {
        if (!write.sequence) throw std::invalid_argument("null sequence in slot mapping");
        if (!first.shares_pool_with(write.sequence->block_table())) {
            throw std::invalid_argument("slot mapping batch must use one physical pool");
        }
        const auto where = write.sequence->token_location(write.token_position);
        const auto bs = static_cast<PhysicalSlot>(write.sequence->block_size());
        const auto page = static_cast<PhysicalSlot>(where.physical_block);
        const auto offset = static_cast<PhysicalSlot>(where.offset_in_block);
        if (page > (std::numeric_limits<PhysicalSlot>::max() - offset) / bs) {
            throw std::overflow_error("physical slot overflow");
        }
        slots.push_back(page * bs + offset);
    }
    return slots;
}

// ---------------------------------------------------------------- batch table
PhysicalBlockID BatchBlockTable::physical_id(std::size_t request, std::size_t logical_block) const {
    if (request >= num_sequences() || logical_block >= width_) {
        throw std::out_of_range("batch block table index out of range");
    }
    const auto id = table_[request * width_ + logical_block];
    if (id == invalid_block()) throw std::out_of_range("batch block table padding");
    return id;
}

BatchBlockTable build_batch_block_table(const std::vector<const SequenceState*>& sequences) {
    BatchBlockTable out;
    if (sequences.empty()) return out;
    if (!sequences.front()) throw std::invalid_argument("null batch sequence");
    out.lengths_.reserve(sequences.size());
    for (const auto* s : sequences) {
        if (!s) throw std::invalid_argument("null batch sequence");
        if (!s->block_table().shares_pool_with(sequences.front()->block_table())) {
            throw std::invalid_argument("batch sequences must use one physical pool");
        }
        out.lengths_.push_back(s->num_tokens());
        if (s->num_allocated_blocks() > out.width_) out.width_ = s->num_allocated_blocks();
    }
    if (out.width_ > std::numeric_limits<std::size_t>::max() / sequences.size()) {
        throw std::overflow_error("batch block table size overflow");
    }
    out.table_.assign(sequences.size() * out.width_, BatchBlockTable::invalid_block());
    for (std::size_t r = 0; r < sequences.size(); ++r) {
        sequences[r]->physical_block_ids(out.table_.data() + r * out.width_);
    }
    return out;
}

ReadBlockTable build_read_block_table(const SequenceState& sequence) {
    ReadBlockTable ids;
    ids.resize(sequence.num_allocated_blocks());
    sequence.physical_block_ids(ids.data());
    return ids;
}

// ---------------------------------------------------------------- layout
namespace {

std::size_t mul_checked(std::size_t a, std::size_t b) {
    if (b != 0 && a > std::numeric_limits<std::size_t>::max() / b) {
        throw std::overflow_error("paged KV layout size overflow");
    }
    return a * b;
}

std::size_t element_size(DType dtype) {
    switch (dtype) {
    case DType::Float16:
    case DType::BFloat16: return 2;
    case DType::Float32: return 4;
    }
    throw std::invalid_argument("unsupported paged KV dtype");
}

} // namespace

PagedKVLayout::PagedKVLayout(std::size_t num_blocks, std::size_t num_kv_heads,
                             std::size_t block_size, std::size_t head_size, DType dtype)
    : blocks_(num_blocks), heads_(num_kv_heads), block_size_(block_size),
      head_size_(head_size), dtype_(dtype), element_bytes_(element_size(dtype)),
      page_bytes_(0), cache_bytes_(0), slot_count_(0) {
    if (num_blocks == 0 || num_kv_heads == 0 || block_size == 0 || head_size == 0) {
        throw std::invalid_argument("paged KV dimensions must be positive");
    }
    page_bytes_ = mul_checked(mul_checked(mul_checked(heads_, block_size_), head_size_),
                              element_bytes_);
    cache_bytes_ = mul_checked(blocks_, page_bytes_);
    (void)mul_checked(2, cache_bytes_);  // total_bytes() must be representable
    slot_count_ = mul_checked(blocks_, block_size_);
}

std::size_t PagedKVLayout::page_byte_offset(KVKind kind, std::size_t block) const {
    if (kind != KVKind::Key && kind != KVKind::Value) {
        throw std::invalid_argument("invalid KV kind");
    }
    if (block >= blocks_) throw std::out_of_range("physical block out of range");
    return (kind == KVKind::Value ? cache_bytes_ : 0) + block * page_bytes_;
}

std::size_t PagedKVLayout::byte_offset(KVKind kind, std::size_t block, std::size_t head,
                                       std::size_t token, std::size_t dimension) const {
    const auto page = page_byte_offset(kind, block);
    if (head >= heads_ || token >= block_size_ || dimension >= head_size_) {
        throw std::out_of_range("paged KV coordinate out of range");
    }
    return page + ((head * block_size_ + token) * head_size_ + dimension) * element_bytes_;
}

std::size_t PagedKVLayout::slot_byte_offset(KVKind kind, std::uint64_t slot,
                                            std::size_t head, std::size_t dimension) const {
    if (slot >= slot_count_) throw std::out_of_range("physical slot out of range");
    return byte_offset(kind, static_cast<std::size_t>(slot / block_size_), head,
                       static_cast<std::size_t>(slot % block_size_), dimension);
}

} // namespace kvflux::v2
