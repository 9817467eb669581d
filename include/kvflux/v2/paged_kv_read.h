#pragma once
// Gather of a sequence's K/V from its pages into contiguous token order.
// Same surface as the reference's include/kvflux/v2/paged_kv_read.h:10-19.

#include "kvflux/v2/paged_kv_storage.h"

#include <vector>

namespace kvflux::v2 {

using ReadBlockTable = std::vector<PhysicalBlockID>;
ReadBlockTable build_read_block_table(const SequenceState& sequence);

// Outputs: device arrays [num_tokens][num_kv_heads][head_size] of the storage
// dtype. Empty sequence: no-op. Foreign pool / block-size mismatch, null,
// host or foreign-device outputs, outputs overlapping each other or the
// cache: std::invalid_argument. Returns after the copy completes.
void read_paged_kv(const PagedKVStorage& storage, const SequenceState& sequence,
                   void* key_out_device, void* value_out_device);

// Extension (no counterpart in the reference): one launch gathering every
// sequence, packed back to back in input order, i.e. sequence i starts at
// token sum(num_tokens of sequences before i). Empty sequences contribute
// nothing. Same validation as read_paged_kv, applied to the packed size.
void read_paged_kv_batch(const PagedKVStorage& storage,
                         const std::vector<const SequenceState*>& sequences,
                         void* key_out_device, void* value_out_device);

} // namespace kvflux::v2
