#pragma once
// Device-resident batch block table for a decode loop, and the decode step
// built on it. No counterpart in the reference, which rebuilds the row-major
// BatchBlockTable and the length array on the host and uploads both on every
// paged_attention_batch call (src/v2/batch_block_table.cpp:18-48,
// src/v2/paged_attention.cu:248-313), and builds and uploads a slot mapping
// for every write (src/v2/slot_mapping.cpp:8-31, src/v2/paged_kv_write.cu:101-139).
//
// Here the table lives on the device with a fixed row capacity and is kept
// current with O(changed entries) uploads: a sequence only ever appends
// pages, and copy-on-write only replaces its last page, so per refresh each
// row contributes its new length and the entries from its former last block
// on. The decode step's slots are then read from the device table by the
// write kernel.

#include "kvflux/v2/paged_kv_storage.h"
#include "kvflux/v2/sequence_state.h"

#include <cstddef>
#include <cstdint>
#include <memory>
#include <vector>

namespace kvflux::v2 {

class DeviceBatchTable {
public:
    // Row r is sequences[r] (distinct, using storage's pool, each with at
    // most capacity_blocks pages). The sequences must outlive the table and
    // stay at their addresses. Uploads the full table once and waits.
    DeviceBatchTable(const PagedKVStorage& storage, std::vector<SequenceState*> sequences,
                     std::size_t capacity_blocks);
    ~DeviceBatchTable();
    DeviceBatchTable(const DeviceBatchTable&) = delete;
    DeviceBatchTable& operator=(const DeviceBatchTable&) = delete;

    // Brings the device copy up to date with the sequences and waits.
    // std::length_error when a sequence has outgrown capacity_blocks.
    void refresh();

    std::size_t rows() const noexcept { return sequences_.size(); }
    std::size_t capacity_blocks() const noexcept { return capacity_; }
    const std::vector<SequenceState*>& sequences() const noexcept { return sequences_; }
    // Device arrays (not dereferenceable on the host): uint64 [rows][capacity]
    // page ids (~0 past a row's pages) and uint64 [rows] lengths.
    const std::uint64_t* device_table() const noexcept;
    const std::uint64_t* device_lengths() const noexcept;
    // Lengths as of the last refresh (host copy).
    const std::vector<std::uint64_t>& lengths() const noexcept { return lengths_; }

    // Library-internal: enqueues the refresh on the default stream without
    // waiting (the caller synchronises before the next refresh).
    void enqueue_refresh();

private:
    struct Device;
    void upload_all();

    const PagedKVStorage& storage_;
    std::vector<SequenceState*> sequences_;
    std::size_t capacity_;
    std::vector<std::uint64_t> shadow_;   // host copy of the device table
    std::vector<std::uint64_t> lengths_;  // host copy of the device lengths
    std::vector<std::uint64_t> blocks_;   // pages per row at the last refresh
    bool stale_ = true;                   // device copy must be uploaded whole
    std::unique_ptr<Device> device_;
};

// Batch decode attention over a refreshed device table: row r attends to
// tokens [0, length_r) of sequences()[r]. Same contract as
// paged_attention_batch (Q/O device FP32 [rows][query_heads][head_size],
// Exact arithmetic).
void paged_attention_batch(const PagedKVStorage& storage, const DeviceBatchTable& batch,
                           const float* query_device, float* output_device,
                           std::size_t query_heads);

// One decode step for every row of `batch`: appends one token to each
// sequence (shared partial tails copied in one launch, as append_tokens_cow),
// writes the new K/V rows (device [rows][num_kv_heads][head_size] in the
// cache dtype) at those positions with slots taken from the device table,
// and computes each row's attention (device FP32 [rows][query_heads][head_size]).
// One synchronisation, no host slot mapping or table rebuild. Returns the
// new tokens' locations. Validation failures change nothing; if a launch
// fails after the appends, the sequences keep their new (unwritten) token
// and the caller aborts those requests, as SequenceLifecycle::decode does.
std::vector<TokenLocation> decode_step(PagedKVStorage& storage, DeviceBatchTable& batch,
                                       const void* key_new_device, const void* value_new_device,
                                       const float* query_device, float* output_device,
                                       std::size_t query_heads);

} // namespace kvflux::v2
