#pragma once
// Element-type and K/V tags shared by every paged-KV entry point.
// Mirrors include/kvflux/kv_layout.h:7-8 of the reference (same enumerators,
// same order, so the integer values match across the drop-in boundary).
// The reference's v1 capacity planner (KVBlockLayout, kv_layout.h:30-43) is
// not part of the paged-KV data path and is not provided here.

namespace kvflux {

// Float16 and BFloat16 are 2-byte elements, Float32 is 4 bytes.
enum class DType { Float16, BFloat16, Float32 };

// Selects the K arena or the V arena of a PagedKVStorage.
enum class KVKind { Key, Value };

} // namespace kvflux
