#pragma once
// Decode append with device copy-on-write of a shared partial tail page.
// Same surface as the reference's include/kvflux/v2/copy_on_write.h:10.

#include "kvflux/v2/paged_kv_storage.h"

#include <vector>

namespace kvflux::v2 {

// Reserves one token; a shared, partially filled tail page is first copied
// (K and V) to a private page with PagedKVStorage::copy_block. The returned
// position has not been written yet.
TokenLocation append_token_cow(const PagedKVStorage& storage, SequenceState& sequence);

// Batch form for a decode step over many requests (no counterpart in the
// reference): one token for each of `sequences` (distinct), locations in
// input order. Every shared partial tail page is copied in a single launch
// (PagedKVStorage::copy_blocks). All or nothing: the new pages are reserved
// and the copies done before any sequence changes.
std::vector<TokenLocation> append_tokens_cow(const PagedKVStorage& storage,
                                             const std::vector<SequenceState*>& sequences);

} // namespace kvflux::v2
