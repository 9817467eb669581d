// Device-side batch metadata: in-place updates of a device batch block table.
//
// The reference rebuilds the whole row-major batch table
// (size_t[B][max_blocks], SIZE_MAX padding) and the length array on the host
// and copies them to the device on every call
// (src/v2/batch_block_table.cpp:18-48, src/v2/paged_attention.cu:248-313).
// A decode step changes at most a few entries per sequence (its length, and
// the tail entry when a page is appended or copied on write), so a table kept
// on the device is brought up to date by scattering just those records:
//   update i = {row, new_length, block_index, page_id}
//   lengths[row] = new_length; table[row][block_index] = page_id
// (block_index >= width: length only). Records of one row carry the same
// length and distinct block indexes, so the scatter is order-free.
#include "common.h"

namespace kvflux_hip {
namespace {

constexpr int kApplyThreads = 256;

__global__ __launch_bounds__(kApplyThreads) void table_apply_kernel(std::uint64_t* __restrict__ table,
                                                                     std::uint64_t width,
                                                                     std::uint64_t* __restrict__ lengths,
                                                                     std::uint64_t rows,
                                                                     const std::uint64_t* __restrict__ updates,
                                                                     std::uint64_t count) {
    const std::uint64_t i = static_cast<std::uint64_t>(blockIdx.x) * kApplyThreads + threadIdx.x;
    if (i >= count) return;
    const std::uint64_t row = updates[4 * i], len = updates[4 * i + 1];
    const std::uint64_t index = updates[4 * i + 2], page = updates[4 * i + 3];
    if (row >= rows) return;
    lengths[row] = len;
    if (index < width) table[row * width + index] = page;
}

} // namespace
} // namespace kvflux_hip

using namespace kvflux_hip;

extern "C" int kvflux_table_apply(uint64_t* block_table, uint64_t table_width, uint64_t* seq_lens,
                                  uint64_t num_rows, const uint64_t* updates, uint64_t num_updates,
                                  void* stream) {
    if (num_updates == 0) return KVFLUX_OK;
    if (!block_table || !seq_lens || !updates || table_width == 0) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "table apply: null pointer");
    }
    if (num_rows > (~0ULL) / table_width) return fail(KVFLUX_ERR_OVERFLOW, "table apply: size overflow");
    const std::uint64_t blocks = (num_updates + kApplyThreads - 1) / kApplyThreads;
    if (blocks > 0x7fffffffULL) return fail(KVFLUX_ERR_UNSUPPORTED, "table apply: too many updates");
    hipLaunchKernelGGL(table_apply_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kApplyThreads), 0,
                       as_stream(stream), block_table, table_width, seq_lens, num_rows, updates, num_updates);
    return launch_status("table_apply_kernel");
}
