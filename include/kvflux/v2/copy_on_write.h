#pragma once
// Decode append with device copy-on-write of a shared partial tail page.
// Same surface as the reference's include/kvflux/v2/copy_on_write.h:10.

#include "kvflux/v2/paged_kv_storage.h"

namespace kvflux::v2 {

// Reserves one token; a shared, partially filled tail page is first copied
// (K and V) to a private page with PagedKVStorage::copy_block. The returned
// position has not been written yet.
TokenLocation append_token_cow(const PagedKVStorage& storage, SequenceState& sequence);

} // namespace kvflux::v2
