// Paged KV write: scatter of K_new/V_new rows into the cache by slot.
// Same result as the reference's paged_kv_write_kernel
// (src/v2/paged_kv_write.cu:62-83): for token n, head h, element d,
//   cache[((slot_n / bs * H + h) * bs + slot_n % bs) * D + d] = new[(n * H + h) * D + d]
// for K and V. The copy is a raw bit copy, so only the element width matters.
//
// gfx950 mapping: a (token, head) row of D*esize bytes is moved as
// `row_bytes / W` vectors of W bytes (W = 16 when the row and the four base
// pointers allow it, i.e. global_load/store_dwordx4). Consecutive lanes take
// consecutive vectors of the input, so a wavefront reads 1 KiB of contiguous
// input and writes whole rows (256 bytes for D=128 BF16) into their pages.
// A thread moves four vectors of K and four of V, 256 threads apart: all
// eight row loads and the four slot loads are issued before the first store,
// so a thread pays one memory round trip for 128 bytes.
//
// Measured on MI355X, 4096 tokens x 8 heads x 128 BF16 (33.6 MB moved) into
// random pages of a 4 GiB arena, with 16 rotated input/slot sets (537 MB, so
// no launch finds its inputs or pages in the 256 MB Infinity Cache); kernel
// durations from rocprofv3:
//   one vector per thread, 1024 threads, plain stores   9.7-10.1 us
//   the same with non-temporal stores                    8.4 us
//   four vectors per thread, 256 threads, nt stores      6.7-7.2 us
// Non-temporal stores matter most: the rows land in random pages, and letting
// them allocate in the caches only delays their write-back. Non-temporal
// input loads were 3-6% slower than plain ones here.
#include "common.h"

namespace kvflux_hip {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

// Slot of input row n: from a slot array (write_paged_kv), or the position
// just appended to sequence n, looked up in a device batch block table
// (decode append: slot = table[n][(len_n - 1) / bs] * bs + (len_n - 1) % bs).
// ~0 (never < slot_count) when the row has no valid slot.
struct SlotList {
    const std::uint64_t* slots;
    __device__ std::uint64_t operator()(std::uint64_t n) const { return slots[n]; }
};
struct SlotAtTail {
    const std::uint64_t* table;
    std::uint64_t width;
    const std::uint64_t* lens;
    std::uint64_t block_size, num_blocks;
    __device__ std::uint64_t operator()(std::uint64_t n) const {
        const std::uint64_t len = lens[n];
        if (len == 0) return ~0ULL;
        const std::uint64_t b = (len - 1) / block_size;
        if (b >= width) return ~0ULL;
        const std::uint64_t page = table[n * width + b];
        return page < num_blocks ? page * block_size + (len - 1) % block_size : ~0ULL;
    }
};

template <typename Vec, typename Slots>
__global__ __launch_bounds__(kThreads) void paged_kv_write_kernel(
    Vec* __restrict__ key_cache, Vec* __restrict__ value_cache, const Vec* __restrict__ key_new,
    const Vec* __restrict__ value_new, Slots slot_of,
    std::uint32_t total_vectors, FastDiv vectors_per_row, FastDiv heads, FastDiv block_size,
    std::uint32_t slot_count) {
    const std::uint32_t first = blockIdx.x * (kThreads * kUnroll) + threadIdx.x;
    Vec k[kUnroll], v[kUnroll];
    std::uint64_t dst[kUnroll];
    bool live[kUnroll];
    // The row loads do not depend on the slot: they are issued unconditionally
    // (a thread past the end rereads vector 0) together with the slot load,
    // so a thread waits for one memory round trip, not two (a load under the
    // slot test is issued only after the slot has arrived).
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const std::uint32_t i0 = first + u * kThreads;
        const bool in_range = i0 < total_vectors;
        const std::uint32_t i = in_range ? i0 : 0u;  // total_vectors >= 1
        k[u] = key_new[i];
        v[u] = value_new[i];
        const std::uint32_t row = vectors_per_row.div(i);
        const std::uint32_t col = i - row * vectors_per_row.divisor;
        const std::uint32_t token = heads.div(row);
        const std::uint32_t head = row - token * heads.divisor;
        const std::uint64_t slot = slot_of(token);
        live[u] = in_range && slot < slot_count;  // never write outside the arena
        const std::uint32_t s = static_cast<std::uint32_t>(slot);
        const std::uint32_t page = block_size.div(s);
        const std::uint32_t offset = s - page * block_size.divisor;
        dst[u] = ((static_cast<std::uint64_t>(page) * heads.divisor + head) *
                      block_size.divisor + offset) * vectors_per_row.divisor + col;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        keep_in_registers(k[u]);
        keep_in_registers(v[u]);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        if (live[u]) {
            stream_store(key_cache + dst[u], k[u]);
            stream_store(value_cache + dst[u], v[u]);
        }
    }
}

// Same mapping with 64-bit index arithmetic, for arenas or batches whose
// vector or slot counts do not fit in 32 bits.
template <typename Vec, typename Slots>
__global__ __launch_bounds__(kThreads) void paged_kv_write_kernel_wide(
    Vec* __restrict__ key_cache, Vec* __restrict__ value_cache, const Vec* __restrict__ key_new,
    const Vec* __restrict__ value_new, Slots slot_of,
    std::uint64_t total_vectors, std::uint64_t vectors_per_row, std::uint64_t heads,
    std::uint64_t block_size, std::uint64_t slot_count) {
    const std::uint64_t stride = static_cast<std::uint64_t>(gridDim.x) * blockDim.x;
    for (std::uint64_t i = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
         i < total_vectors; i += stride) {
        const Vec k = key_new[i];
        const Vec v = value_new[i];
        const std::uint64_t row = i / vectors_per_row, col = i % vectors_per_row;
        const std::uint64_t token = row / heads, head = row % heads;
        const std::uint64_t slot = slot_of(token);
        keep_in_registers(k);
        keep_in_registers(v);
        if (slot >= slot_count) continue;
        const std::uint64_t d =
            ((slot / block_size * heads + head) * block_size + slot % block_size) *
                vectors_per_row + col;
        stream_store(key_cache + d, k);
        stream_store(value_cache + d, v);
    }
}

template <typename Vec, typename Slots>
int launch(void* kc, void* vc, const void* kn, const void* vn, Slots slots,
           std::uint64_t tokens, std::uint64_t heads, std::uint64_t block_size,
           std::uint64_t row_bytes, std::uint64_t slot_count, hipStream_t stream) {
    const std::uint64_t vpr = row_bytes / sizeof(Vec);
    const std::uint64_t total = tokens * heads * vpr;
    // 32-bit path: the last thread index (grid * per_block) must not wrap.
    constexpr std::uint64_t limit = 0xffffffffULL - kThreads * kUnroll;
    if (total <= limit && slot_count <= limit && vpr <= limit && heads <= limit &&
        block_size <= limit) {
        const std::uint64_t per_block = kThreads * kUnroll;
        const auto grid = static_cast<unsigned>((total + per_block - 1) / per_block);
        hipLaunchKernelGGL((paged_kv_write_kernel<Vec, Slots>), dim3(grid), dim3(kThreads), 0, stream,
                           static_cast<Vec*>(kc), static_cast<Vec*>(vc),
                           static_cast<const Vec*>(kn), static_cast<const Vec*>(vn), slots,
                           static_cast<std::uint32_t>(total),
                           FastDiv(static_cast<std::uint32_t>(vpr)),
                           FastDiv(static_cast<std::uint32_t>(heads)),
                           FastDiv(static_cast<std::uint32_t>(block_size)),
                           static_cast<std::uint32_t>(slot_count));
    } else {
        const std::uint64_t blocks = (total + kThreads - 1) / kThreads;
        const auto grid = static_cast<unsigned>(blocks < 65536 ? blocks : 65536);
        hipLaunchKernelGGL((paged_kv_write_kernel_wide<Vec, Slots>), dim3(grid), dim3(kThreads), 0, stream,
                           static_cast<Vec*>(kc), static_cast<Vec*>(vc),
                           static_cast<const Vec*>(kn), static_cast<const Vec*>(vn), slots, total,
                           vpr, heads, block_size, slot_count);
    }
    return launch_status("paged_kv_write_kernel");
}

} // namespace
} // namespace kvflux_hip

using namespace kvflux_hip;

namespace {

// Validation and vector-width dispatch shared by both entry points.
template <typename Slots>
int write_rows(void* key_cache, void* value_cache, uint64_t num_blocks, uint64_t num_kv_heads,
               uint64_t block_size, uint64_t head_size, int dtype, const void* key_new,
               const void* value_new, Slots slots, uint64_t num_tokens, void* stream) {
    const std::size_t esize = dtype_bytes(dtype);
    if (esize == 0) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
    if (!key_cache || !value_cache || !key_new || !value_new) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged KV write: null pointer");
    }
    if (num_blocks == 0 || num_kv_heads == 0 || block_size == 0 || head_size == 0) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged KV write: zero dimension");
    }
    if (head_size > (~0ULL) / esize || num_blocks > (~0ULL) / block_size) {
        return fail(KVFLUX_ERR_OVERFLOW, "paged KV write: size overflow");
    }
    const std::uint64_t row_bytes = head_size * esize;
    const std::uint64_t slot_count = num_blocks * block_size;
    const void* ptrs[4] = {key_cache, value_cache, key_new, value_new};
    const unsigned width = copy_width(row_bytes, ptrs, 4);
    const hipStream_t s = as_stream(stream);
    switch (width) {
    case 16: return launch<V16>(key_cache, value_cache, key_new, value_new, slots, num_tokens,
                                num_kv_heads, block_size, row_bytes, slot_count, s);
    case 8: return launch<V8>(key_cache, value_cache, key_new, value_new, slots, num_tokens,
                              num_kv_heads, block_size, row_bytes, slot_count, s);
    case 4: return launch<std::uint32_t>(key_cache, value_cache, key_new, value_new, slots,
                                         num_tokens, num_kv_heads, block_size, row_bytes,
                                         slot_count, s);
    case 2: return launch<std::uint16_t>(key_cache, value_cache, key_new, value_new, slots,
                                         num_tokens, num_kv_heads, block_size, row_bytes,
                                         slot_count, s);
    default: return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged KV write: misaligned buffers");
    }
}

} // namespace

extern "C" int kvflux_write_paged_kv(void* key_cache, void* value_cache, uint64_t num_blocks,
                                     uint64_t num_kv_heads, uint64_t block_size,
                                     uint64_t head_size, int dtype, const void* key_new,
                                     const void* value_new, const uint64_t* slots,
                                     uint64_t num_tokens, void* stream) {
    if (num_tokens == 0) return KVFLUX_OK;
    if (!slots) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged KV write: null pointer");
    return write_rows(key_cache, value_cache, num_blocks, num_kv_heads, block_size, head_size, dtype,
                      key_new, value_new, SlotList{slots}, num_tokens, stream);
}

extern "C" int kvflux_write_paged_kv_tail(void* key_cache, void* value_cache, uint64_t num_blocks,
                                          uint64_t num_kv_heads, uint64_t block_size,
                                          uint64_t head_size, int dtype, const void* key_new,
                                          const void* value_new, const uint64_t* block_table,
                                          uint64_t table_width, const uint64_t* seq_lens,
                                          uint64_t num_rows, void* stream) {
    if (num_rows == 0) return KVFLUX_OK;
    if (!block_table || !seq_lens || table_width == 0) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged KV tail write: null table");
    }
    if (num_rows > (~0ULL) / table_width) return fail(KVFLUX_ERR_OVERFLOW, "paged KV tail write: size overflow");
    return write_rows(key_cache, value_cache, num_blocks, num_kv_heads, block_size, head_size, dtype,
                      key_new, value_new, SlotAtTail{block_table, table_width, seq_lens, block_size, num_blocks},
                      num_rows, stream);
}
