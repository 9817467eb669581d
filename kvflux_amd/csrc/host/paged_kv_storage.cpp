// PagedKVStorage: one device allocation per cache, K region then V region
// (reference src/v2/paged_kv_storage.cpp:12-17,38-68; copy_block :70-93).
#include "kvflux/v2/paged_kv_storage.h"

#include "device_runtime.h"

#include <limits>
#include <stdexcept>
#include <unordered_set>

namespace kvflux::v2 {

PagedKVStorage::PagedKVStorage(PhysicalBlockPool& pool, std::size_t num_kv_heads,
                               std::size_t head_size, DType dtype, int device)
    : pool_(pool),
      layout_(pool.capacity(), num_kv_heads, pool.block_size(), head_size, dtype),
      device_(device),
      scratch_(std::make_unique<detail::DeviceScratch>()) {
    int count = 0;
    detail::check(kvflux_device_count(&count), "count devices");
    if (device < 0 || device >= count) throw std::invalid_argument("invalid GPU device");
    detail::DeviceGuard guard(device_);
    detail::check(kvflux_device_malloc(&arena_, layout_.total_bytes()), "allocate paged KV arena");
}

PagedKVStorage::~PagedKVStorage() {
    // Scratch buffers and the arena belong to device_; free them there.
    int previous = 0;
    const bool switched = kvflux_get_device(&previous) == KVFLUX_OK &&
                          (previous == device_ || kvflux_set_device(device_) == KVFLUX_OK);
    scratch_.reset();
    if (arena_) (void)kvflux_device_free(arena_);
    if (switched && previous != device_) (void)kvflux_set_device(previous);
}

void* PagedKVStorage::key_base() const { return arena_; }

void* PagedKVStorage::value_base() const {
    return static_cast<unsigned char*>(arena_) + layout_.cache_bytes();
}

void* PagedKVStorage::page_address(KVKind kind, PhysicalBlockHandle handle) const {
    const auto offset = layout_.page_byte_offset(kind, pool_.id(handle));
    return static_cast<unsigned char*>(arena_) + offset;
}

void* PagedKVStorage::element_address(KVKind kind, PhysicalBlockHandle handle, std::size_t head,
                                      std::size_t token, std::size_t dimension) const {
    const auto offset = layout_.byte_offset(kind, pool_.id(handle), head, token, dimension);
    return static_cast<unsigned char*>(arena_) + offset;
}

void* PagedKVStorage::slot_address(KVKind kind, PhysicalSlot slot, std::size_t head,
                                   std::size_t dimension) const {
    const auto offset = layout_.slot_byte_offset(kind, slot, head, dimension);
    return static_cast<unsigned char*>(arena_) + offset;
}

void PagedKVStorage::copy_block(PhysicalBlockHandle source, PhysicalBlockHandle destination) const {
    const auto from = pool_.id(source);
    const auto to = pool_.id(destination);
    if (from == to || pool_.ref_count(destination) != 1 || pool_.is_published(destination)) {
        throw std::invalid_argument("copy destination must be a private, unpublished page");
    }
    detail::DeviceGuard guard(device_);
    try {
        // Both pages must land before the caller switches its table entry.
        detail::check(kvflux_memcpy_async(page_address(KVKind::Key, destination),
                                          page_address(KVKind::Key, source),
                                          layout_.page_bytes(), nullptr), "copy K page");
        detail::check(kvflux_memcpy_async(page_address(KVKind::Value, destination),
                                          page_address(KVKind::Value, source),
                                          layout_.page_bytes(), nullptr), "copy V page");
        detail::check(kvflux_stream_synchronize(nullptr), "synchronize KV page copy");
    } catch (...) {
        (void)kvflux_stream_synchronize(nullptr);
        throw;
    }
}

void PagedKVStorage::copy_blocks(
    const std::vector<std::pair<PhysicalBlockHandle, PhysicalBlockHandle>>& pairs) const {
    if (pairs.empty()) return;
    std::vector<std::uint64_t> ids;
    ids.reserve(2 * pairs.size());
    std::unordered_set<PhysicalBlockID> destinations;
    for (const auto& [source, destination] : pairs) {
        const auto from = pool_.id(source);
        const auto to = pool_.id(destination);
        if (from == to || pool_.ref_count(destination) != 1 || pool_.is_published(destination) ||
            !destinations.insert(to).second) {
            throw std::invalid_argument("copy destination must be a private, unpublished page");
        }
        ids.push_back(from);
        ids.push_back(to);
    }
    for (std::size_t i = 0; i < ids.size(); i += 2) {
        if (destinations.count(ids[i])) {
            throw std::invalid_argument("a copy source is also a destination of the batch");
        }
    }
    detail::DeviceGuard guard(device_);
    const auto dev = scratch_->upload({{ids.data(), ids.size() * sizeof(std::uint64_t)}});
    try {
        // All pages must land before the callers switch their table entries.
        detail::check(kvflux_copy_pages(key_base(), value_base(), layout_.num_blocks(),
                                        layout_.page_bytes(), dev[0], pairs.size(), nullptr),
                      "copy KV pages");
        detail::check(kvflux_stream_synchronize(nullptr), "synchronize KV page copy");
    } catch (...) {
        (void)kvflux_stream_synchronize(nullptr);
        throw;
    }
}

} // namespace kvflux::v2
