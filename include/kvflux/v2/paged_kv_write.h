#pragma once
// Scatter of new K/V rows into the paged cache by slot number.
// Same signature and contract as the reference's
// include/kvflux/v2/paged_kv_write.h:14-15 (src/v2/paged_kv_write.cu:101-139).

#include "kvflux/v2/paged_kv_storage.h"

namespace kvflux::v2 {

// K_new/V_new: device arrays [slot_mapping.size()][num_kv_heads][head_size]
// of the storage dtype, ready on the default stream. Raw bit copy.
// Empty mapping: no-op, pointers not touched. Null pointers, duplicate slots
// and non-device / foreign-device inputs: std::invalid_argument. Slot beyond
// slot_count(): std::out_of_range. Returns after the copy completes.
void write_paged_kv(PagedKVStorage& storage, const void* key_new_device,
                    const void* value_new_device, const SlotMapping& slot_mapping);

} // namespace kvflux::v2
