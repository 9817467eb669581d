// v2 control plane: per-sequence page tables and the integer metadata the
// kernels consume. The observable contract (page ids and the order they are
// taken and returned, reference counts, exception types, all-or-nothing
// failures) is the reference's:
//   BlockTable             include/kvflux/v2/block_table.h:14-61
//   SequenceState          include/kvflux/v2/sequence_state.h:14-71
//   build_slot_mapping     src/v2/slot_mapping.cpp:8-31 (slot = page * bs + offset)
//   BatchBlockTable        include/kvflux/v2/batch_block_table.h:12-36
//   build_read_block_table include/kvflux/v2/paged_kv_read.h:10-11
//   PagedKVLayout          src/v2/paged_kv_layout.cpp:42-68 (byte offsets)
// Multi-page operations stage the references they take (pending_refs.h) and
// touch the table only once nothing more can fail.
#include "kvflux/physical_block_pool.h"
#include "kvflux/v2/batch_block_table.h"
#include "kvflux/v2/block_table.h"
#include "kvflux/v2/paged_kv_layout.h"
#include "kvflux/v2/paged_kv_read.h"
#include "kvflux/v2/sequence_state.h"
#include "kvflux/v2/slot_mapping.h"

#include "pending_refs.h"

#include <algorithm>
#include <initializer_list>
#include <limits>
#include <stdexcept>
#include <utility>

namespace kvflux::v2 {

using host::ceil_div;
using host::pending_refs;
using host::Undo;

namespace {

constexpr std::size_t kMaxSize = std::numeric_limits<std::size_t>::max();

auto releaser(PhysicalBlockPool& pool) {
    return [&pool](PhysicalBlockHandle h) { pool.free(h); };
}

} // namespace

// ---------------------------------------------------------------- BlockTable
BlockTable::BlockTable(PhysicalBlockPool& pool) noexcept : pool_(&pool) {}

BlockTable::~BlockTable() noexcept { clear(); }

BlockTable::BlockTable(BlockTable&& other) noexcept
    : pool_(std::exchange(other.pool_, nullptr)), entries_(std::exchange(other.entries_, {})) {}

BlockTable& BlockTable::operator=(BlockTable&& other) noexcept {
    if (this != &other) {
        clear();  // our references go back before we take over the other's
        pool_ = std::exchange(other.pool_, nullptr);
        entries_ = std::exchange(other.entries_, {});
    }
    return *this;
}

PhysicalBlockPool& BlockTable::pool() const {
    if (pool_ == nullptr) throw std::logic_error("this block table was moved from and has no pool");
    return *pool_;
}

void BlockTable::make_room(std::size_t n) {
    if (entries_.capacity() - entries_.size() >= n) return;
    entries_.reserve(std::max(entries_.size() + n, 2 * entries_.capacity()));
}

void BlockTable::adopt(const std::vector<PhysicalBlockHandle>& handles) noexcept {
    entries_.insert(entries_.end(), handles.begin(), handles.end());  // room was made
}

PhysicalBlockID BlockTable::append_new() {
    PhysicalBlockPool& owner = pool();
    make_room(1);  // before the page is taken: nothing to give back if this fails
    const PhysicalBlockHandle fresh = owner.allocate();
    entries_.push_back(fresh);
    return fresh.id;
}

void BlockTable::append_existing(PhysicalBlockHandle handle) {
    PhysicalBlockPool& owner = pool();
    make_room(1);
    owner.retain(handle);  // validates the handle; the table's own reference
    entries_.push_back(handle);
}

void BlockTable::append_shared(const BlockTable& source, std::size_t logical_block) {
    if (pool_ == nullptr || source.pool_ != pool_) {
        throw std::invalid_argument("shared block tables must use one physical pool");
    }
    // A copy, not a reference: `source` may be this table.
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
    const PhysicalBlockHandle h = entries_.at(logical_block);
    pool_->id(h);  // checks the generation and that the page is held
    return h;
}

std::size_t BlockTable::ref_count(std::size_t logical_block) const {
    return pool_->ref_count(entries_.at(logical_block));
}

void BlockTable::pop_back() {
    if (entries_.empty()) throw std::out_of_range("pop_back on an empty block table");
    pool_->free(entries_.back());
    entries_.pop_back();
}

void BlockTable::replace_last_owned(PhysicalBlockHandle new_handle) {
    if (entries_.empty()) throw std::out_of_range("replace_last_owned on an empty block table");
    pool_->id(new_handle);
    const bool private_page = new_handle != entries_.back() && pool_->ref_count(new_handle) == 1 &&
                              !pool_->is_published(new_handle);
    if (!private_page) {
        throw std::invalid_argument("a replacement tail must be a private, unpublished page");
    }
    // free() checks the old handle; the assignment after it cannot fail, so
    // on any failure the caller still owns new_handle.
    pool_->free(entries_.back());
    entries_.back() = new_handle;
}

void BlockTable::clear() noexcept {
    for (const PhysicalBlockHandle h : entries_) pool_->free(h);
    entries_.clear();
}

// ---------------------------------------------------------------- SequenceState
SequenceState::SequenceState(RequestID request_id, PhysicalBlockPool& pool) noexcept
    : id_(request_id), block_size_(pool.block_size()), table_(pool) {}

SequenceState::SequenceState(SequenceState&& other) noexcept
    : id_(other.id_), tokens_(std::exchange(other.tokens_, 0)), block_size_(other.block_size_),
      table_(std::move(other.table_)) {}

SequenceState& SequenceState::operator=(SequenceState&& other) noexcept {
    if (this != &other) {
        table_ = std::move(other.table_);
        id_ = other.id_;
        tokens_ = std::exchange(other.tokens_, 0);
        block_size_ = other.block_size_;
    }
    return *this;
}

std::size_t SequenceState::last_block_num_tokens() const noexcept {
    if (tokens_ == 0) return 0;
    const std::size_t rest = tokens_ % block_size_;
    return rest == 0 ? block_size_ : rest;
}

bool SequenceState::tail_shared_and_partial() const {
    return tokens_ % block_size_ != 0 && table_.ref_count(table_.size() - 1) > 1;
}

void SequenceState::reserve_blocks(std::size_t n) { table_.make_room(n); }

void SequenceState::adopt_cached_blocks(const std::vector<PhysicalBlockHandle>& handles) noexcept {
    table_.adopt(handles);
    tokens_ += handles.size() * block_size_;
}

void SequenceState::append_tokens(std::size_t count) {
    if (count == 0) return;
    if (count > kMaxSize - tokens_) throw std::overflow_error("sequence token count would overflow");
    if (tail_shared_and_partial()) {
        throw std::logic_error("the partial tail page is shared: append through copy-on-write");
    }
    const std::size_t total = tokens_ + count;
    const std::size_t missing = ceil_div(total, block_size_) - table_.size();
    PhysicalBlockPool& pool = table_.pool();
    table_.make_room(missing);
    // On failure the new pages go back newest first.
    auto fresh = pending_refs(releaser(pool), missing, Undo::InReverseOrder);
    for (std::size_t i = 0; i < missing; ++i) fresh.add(pool.allocate());
    table_.adopt(fresh.commit());
    tokens_ = total;
}

TokenLocation SequenceState::append_token() {
    const std::size_t position = tokens_;
    append_tokens(1);
    return token_location(position);
}

SequenceState SequenceState::fork_shared(RequestID new_request_id) const {
    PhysicalBlockPool& pool = table_.pool();
    SequenceState fork(new_request_id, pool);
    fork.table_.make_room(table_.size());
    auto shared = pending_refs(releaser(pool), table_.size(), Undo::InTakeOrder);
    for (const PhysicalBlockHandle h : table_.entries_) {
        pool.retain(h);
        shared.add(h);
    }
    fork.table_.adopt(shared.commit());
    fork.tokens_ = tokens_;
    return fork;
}

TokenLocation SequenceState::append_token_with_copy(const BlockCopier& copy) {
    if (tokens_ == kMaxSize) throw std::overflow_error("sequence token count would overflow");
    if (!tail_shared_and_partial()) return append_token();
    if (!copy) throw std::invalid_argument("a shared partial tail page needs a copy callback");
    const std::size_t offset = tokens_ % block_size_;
    const PhysicalBlockHandle shared_tail = table_.handle(table_.size() - 1);
    PhysicalBlockPool& pool = table_.pool();
    auto fresh = pending_refs(releaser(pool), 1, Undo::InTakeOrder);
    fresh.add(pool.allocate());
    copy(shared_tail, fresh.back());        // the mapping changes only after a good copy
    table_.replace_last_owned(fresh.back());
    const PhysicalBlockHandle tail = fresh.commit().front();
    ++tokens_;
    return {tail.id, offset};
}

PhysicalBlockID SequenceState::physical_block_id(std::size_t logical_block) const {
    return table_.physical_id(logical_block);
}

void SequenceState::physical_block_ids(PhysicalBlockID* out) const { table_.physical_ids(out); }

PhysicalBlockHandle SequenceState::block_handle(std::size_t logical_block) const {
    return table_.handle(logical_block);
}

TokenLocation SequenceState::token_location(std::size_t token_index) const {
    if (token_index >= tokens_) throw std::out_of_range("token position past the end of the sequence");
    return {physical_block_id(token_index / block_size_), token_index % block_size_};
}

// ---------------------------------------------------------------- slot mapping
SlotMapping build_slot_mapping(const std::vector<TokenWrite>& batch) {
    static_assert(sizeof(std::size_t) <= sizeof(PhysicalSlot), "a page id must fit in a slot number");
    SlotMapping slots(batch.size());
    const BlockTable* reference_table = nullptr;
    for (std::size_t i = 0; i < batch.size(); ++i) {
        const SequenceState* sequence = batch[i].sequence;
        if (sequence == nullptr) throw std::invalid_argument("slot mapping entry without a sequence");
        if (reference_table == nullptr) reference_table = &sequence->block_table();
        if (!reference_table->shares_pool_with(sequence->block_table())) {
            throw std::invalid_argument("every entry of a slot mapping must use one physical pool");
        }
        const TokenLocation at = sequence->token_location(batch[i].token_position);
        const auto bs = static_cast<PhysicalSlot>(sequence->block_size());
        const auto page = static_cast<PhysicalSlot>(at.physical_block);
        const auto offset = static_cast<PhysicalSlot>(at.offset_in_block);
        if (page > (std::numeric_limits<PhysicalSlot>::max() - offset) / bs) {
            throw std::overflow_error("slot number does not fit in 64 bits");
        }
        slots[i] = page * bs + offset;
    }
    return slots;
}

// ---------------------------------------------------------------- batch and read tables
PhysicalBlockID BatchBlockTable::physical_id(std::size_t request, std::size_t logical_block) const {
    if (request >= num_sequences() || logical_block >= width_) {
        throw std::out_of_range("batch block table coordinate outside the table");
    }
    const PhysicalBlockID id = table_[request * width_ + logical_block];
    if (id == invalid_block()) throw std::out_of_range("batch block table entry is padding");
    return id;
}

BatchBlockTable build_batch_block_table(const std::vector<const SequenceState*>& sequences) {
    BatchBlockTable out;
    if (sequences.empty()) return out;
    const SequenceState* first = sequences.front();
    if (first == nullptr) throw std::invalid_argument("batch block table entry without a sequence");
    std::size_t width = 0;
    for (const SequenceState* s : sequences) {
        if (s == nullptr) throw std::invalid_argument("batch block table entry without a sequence");
        if (!s->block_table().shares_pool_with(first->block_table())) {
            throw std::invalid_argument("every row of a batch block table must use one physical pool");
        }
        width = std::max(width, s->num_allocated_blocks());
    }
    if (width > kMaxSize / sequences.size()) throw std::overflow_error("batch block table is too large");
    out.width_ = width;
    out.lengths_.resize(sequences.size());
    out.table_.assign(sequences.size() * width, BatchBlockTable::invalid_block());
    PhysicalBlockID* row = out.table_.data();
    for (std::size_t r = 0; r < sequences.size(); ++r, row += width) {
        out.lengths_[r] = sequences[r]->num_tokens();
        sequences[r]->physical_block_ids(row);  // ids only: the sequences keep the references
    }
    return out;
}

ReadBlockTable build_read_block_table(const SequenceState& sequence) {
    ReadBlockTable ids(sequence.num_allocated_blocks());
    sequence.physical_block_ids(ids.data());
    return ids;
}

// ---------------------------------------------------------------- layout
namespace {

// Product of `factors`, std::overflow_error if it does not fit in size_t.
std::size_t product(std::initializer_list<std::size_t> factors) {
    std::size_t p = 1;
    for (const std::size_t f : factors) {
        if (f != 0 && p > kMaxSize / f) throw std::overflow_error("paged KV arena size does not fit in size_t");
        p *= f;
    }
    return p;
}

std::size_t bytes_per_element(DType dtype) {
    if (dtype == DType::Float16 || dtype == DType::BFloat16) return 2;
    if (dtype == DType::Float32) return 4;
    throw std::invalid_argument("paged KV storage supports Float16, BFloat16 and Float32");
}

} // namespace

PagedKVLayout::PagedKVLayout(std::size_t num_blocks, std::size_t num_kv_heads,
                             std::size_t block_size, std::size_t head_size, DType dtype)
    : blocks_(num_blocks), heads_(num_kv_heads), block_size_(block_size), head_size_(head_size),
      dtype_(dtype), element_bytes_(bytes_per_element(dtype)), page_bytes_(0), cache_bytes_(0),
      slot_count_(0) {
    if (num_blocks == 0 || num_kv_heads == 0 || block_size == 0 || head_size == 0) {
        throw std::invalid_argument("paged KV dimensions must all be positive");
    }
    page_bytes_ = product({heads_, block_size_, head_size_, element_bytes_});
    cache_bytes_ = product({blocks_, page_bytes_});
    product({2, cache_bytes_});  // K and V together must be addressable too
    slot_count_ = product({blocks_, block_size_});
}

std::size_t PagedKVLayout::page_byte_offset(KVKind kind, std::size_t block) const {
    std::size_t base = 0;
    switch (kind) {
    case KVKind::Key: break;
    case KVKind::Value: base = cache_bytes_; break;
    default: throw std::invalid_argument("KV kind must be Key or Value");
    }
    if (block >= blocks_) throw std::out_of_range("physical block id outside the arena");
    return base + block * page_bytes_;
}

std::size_t PagedKVLayout::byte_offset(KVKind kind, std::size_t block, std::size_t head,
                                       std::size_t token, std::size_t dimension) const {
    const std::size_t page = page_byte_offset(kind, block);
    if (head >= heads_ || token >= block_size_ || dimension >= head_size_) {
        throw std::out_of_range("paged KV coordinate outside the page");
    }
    // Strides of the [head][token][dim] page, in elements.
    const std::size_t token_stride = head_size_, head_stride = block_size_ * head_size_;
    return page + (head * head_stride + token * token_stride + dimension) * element_bytes_;
}

std::size_t PagedKVLayout::slot_byte_offset(KVKind kind, std::uint64_t slot, std::size_t head,
                                            std::size_t dimension) const {
    if (slot >= slot_count_) throw std::out_of_range("physical slot outside the arena");
    const auto page = static_cast<std::size_t>(slot / block_size_);
    const auto token = static_cast<std::size_t>(slot % block_size_);
    return byte_offset(kind, page, head, token, dimension);
}

} // namespace kvflux::v2
