// C ABI: error reporting, device memory, pointer queries, streams, events,
// and the test/benchmark support kernels (counter-based fill, byte compare,
// byte fill).
#include "common.h"

#include <cstdarg>
#include <cstdio>
#include <cstring>

namespace kvflux_hip {
namespace {
thread_local char g_last_error[512] = "";
}

int fail(int status, const char* format, ...) {
    va_list args;
    va_start(args, format);
    std::vsnprintf(g_last_error, sizeof(g_last_error), format, args);
    va_end(args);
    return status;
}

int hip_status(hipError_t error, const char* operation) {
    if (error == hipSuccess) return KVFLUX_OK;
    return fail(KVFLUX_ERR_RUNTIME, "%s: %s", operation, hipGetErrorString(error));
}

int launch_status(const char* kernel) { return hip_status(hipGetLastError(), kernel); }

const char* last_error() { return g_last_error; }

namespace {

// i-th output of a splitmix64 generator seeded with `seed`.
__device__ inline std::uint64_t splitmix64_at(std::uint64_t seed, std::uint64_t i) {
    std::uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

__device__ inline float uniform_at(std::uint64_t seed, std::uint64_t i) {
    const auto k = static_cast<std::uint32_t>(splitmix64_at(seed, i) >> 40);  // 24 bits
    return static_cast<float>(k) * 0x1p-23f - 1.0f;                            // exact
}

__device__ inline float normal_at(std::uint64_t seed, std::uint64_t i) {
    std::int32_t sum = 0;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const std::uint64_t h = splitmix64_at(seed, 3 * i + j);
        sum += static_cast<std::int32_t>(h & 0xffff) + static_cast<std::int32_t>((h >> 16) & 0xffff) +
               static_cast<std::int32_t>((h >> 32) & 0xffff) + static_cast<std::int32_t>(h >> 48);
    }
    return static_cast<float>(sum - 393210) * 0x1p-16f;  // exact: |sum - mean| < 2^20
}

// Round-to-nearest-even FP32 -> BF16 on the bit pattern (finite inputs).
__device__ inline std::uint16_t to_bf16_bits(float x) {
    std::uint32_t u = __float_as_uint(x);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<std::uint16_t>(u >> 16);
}

// Round-to-nearest-even FP32 -> FP16 on the bit pattern, subnormals kept
// (finite inputs below the FP16 overflow threshold).
__device__ inline std::uint16_t to_f16_bits(float x) {
    const std::uint32_t u = __float_as_uint(x);
    const std::uint32_t sign = (u >> 16) & 0x8000u;
    const std::uint32_t mag = u & 0x7fffffffu;
    if (mag < 0x33000000u) return static_cast<std::uint16_t>(sign);  // < 2^-25: rounds to 0
    const int exp = static_cast<int>(mag >> 23) - 127;
    std::uint32_t mant = (mag & 0x7fffffu) | 0x800000u;  // 24-bit significand
    std::uint32_t shift;
    std::uint32_t base;
    if (exp < -14) {  // subnormal result: unit 2^-24
        shift = static_cast<std::uint32_t>(-exp - 14 + 13);
        base = 0;
    } else {
        shift = 13;
        base = static_cast<std::uint32_t>(exp + 15) << 10;
        mant &= 0x7fffffu;
    }
    const std::uint32_t half = 1u << (shift - 1);
    const std::uint32_t rem = mant & ((1u << shift) - 1);
    std::uint32_t q = mant >> shift;
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return static_cast<std::uint16_t>(sign | (base + q));  // carry into exponent is correct
}

__global__ void fill_random_kernel(void* dst, std::uint64_t count, int dtype, int distribution,
                                   std::uint64_t seed) {
    const std::uint64_t stride = static_cast<std::uint64_t>(gridDim.x) * blockDim.x;
    for (std::uint64_t i = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
         i < count; i += stride) {
        const float x = distribution == 0 ? uniform_at(seed, i) : normal_at(seed, i);
        if (dtype == KVFLUX_DTYPE_F32) {
            static_cast<float*>(dst)[i] = x;
        } else if (dtype == KVFLUX_DTYPE_BF16) {
            static_cast<std::uint16_t*>(dst)[i] = to_bf16_bits(x);
        } else {
            static_cast<std::uint16_t*>(dst)[i] = to_f16_bits(x);
        }
    }
}

// Streaming form of the two byte kernels (they double as the read-only and
// write-only bandwidth probes of the benchmark): 512-thread workgroups walk
// 32 KiB chunks, a thread's four 16-byte accesses per chunk (consecutive
// lanes on consecutive vectors) all issued before their results are used,
// with the non-temporal hint (each byte is touched once).
constexpr int kByteThreads = 512;
constexpr int kByteVectors = 4;  // 16-byte vectors per thread per chunk
constexpr std::uint64_t kChunkVectors = kByteThreads * kByteVectors;

__device__ inline unsigned long long differing_bytes(const V16& x, const V16& y) {
    unsigned long long n = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const std::uint32_t d = x.w[k] ^ y.w[k];
        n += ((d & 0xffu) != 0) + ((d & 0xff00u) != 0) + ((d & 0xff0000u) != 0) + ((d & 0xff000000u) != 0);
    }
    return n;
}

__global__ __launch_bounds__(kByteThreads) void compare_kernel(const unsigned char* a, const unsigned char* b,
                                                               std::uint64_t bytes, unsigned long long* mismatches) {
    unsigned long long local = 0;
    const std::uint64_t words = bytes / 16;
    const std::uint64_t chunks = words / kChunkVectors;
    const auto* a16 = reinterpret_cast<const V16*>(a);
    const auto* b16 = reinterpret_cast<const V16*>(b);
    for (std::uint64_t c = blockIdx.x; c < chunks; c += gridDim.x) {
        V16 x[kByteVectors], y[kByteVectors];
#pragma unroll
        for (int u = 0; u < kByteVectors; ++u) {
            const std::uint64_t i = c * kChunkVectors + threadIdx.x + u * kByteThreads;
            x[u] = stream_load(a16 + i);
            y[u] = stream_load(b16 + i);
        }
#pragma unroll
        for (int u = 0; u < kByteVectors; ++u) local += differing_bytes(x[u], y[u]);
    }
    // Vectors past the last whole chunk, then bytes past the last vector.
    const std::uint64_t stride = static_cast<std::uint64_t>(gridDim.x) * blockDim.x;
    const std::uint64_t self = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    for (std::uint64_t i = chunks * kChunkVectors + self; i < words; i += stride) local += differing_bytes(a16[i], b16[i]);
    for (std::uint64_t i = words * 16 + self; i < bytes; i += stride) local += a[i] != b[i];
    if (local) atomicAdd(mismatches, local);
}

__global__ __launch_bounds__(kByteThreads) void fill_bytes_kernel(unsigned char* dst, std::uint32_t word,
                                                                  std::uint64_t bytes) {
    const std::uint64_t words = bytes / 16;
    const std::uint64_t chunks = words / kChunkVectors;
    auto* d16 = reinterpret_cast<V16*>(dst);
    const V16 v{{word, word, word, word}};
    for (std::uint64_t c = blockIdx.x; c < chunks; c += gridDim.x) {
#pragma unroll
        for (int u = 0; u < kByteVectors; ++u) stream_store(d16 + c * kChunkVectors + threadIdx.x + u * kByteThreads, v);
    }
    const std::uint64_t stride = static_cast<std::uint64_t>(gridDim.x) * blockDim.x;
    const std::uint64_t self = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    for (std::uint64_t i = chunks * kChunkVectors + self; i < words; i += stride) d16[i] = v;
    for (std::uint64_t i = words * 16 + self; i < bytes; i += stride) dst[i] = static_cast<unsigned char>(word);
}

// Workgroups of the byte kernels: one per 32 KiB chunk, at most 4096 (a
// few resident per CU walk the rest).
unsigned byte_grid(std::uint64_t bytes) {
    const std::uint64_t chunks = bytes / (16 * kChunkVectors);
    return static_cast<unsigned>(chunks < 1 ? 1 : (chunks > 4096 ? 4096 : chunks));
}

unsigned grid_for(std::uint64_t work, unsigned block) {
    const std::uint64_t blocks = (work + block - 1) / block;
    return static_cast<unsigned>(blocks < 1 ? 1 : (blocks > 8192 ? 8192 : blocks));
}

} // namespace
} // namespace kvflux_hip

using namespace kvflux_hip;

extern "C" {

const char* kvflux_last_error(void) { return last_error(); }

int kvflux_abi_version(void) { return 1; }

int kvflux_device_count(int* count) {
    if (!count) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "count is null");
    *count = 0;
    const hipError_t e = hipGetDeviceCount(count);
    if (e == hipErrorNoDevice) {
        (void)hipGetLastError();
        *count = 0;
        return KVFLUX_OK;
    }
    return hip_status(e, "hipGetDeviceCount");
}

int kvflux_get_device(int* device) {
    if (!device) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "device is null");
    return hip_status(hipGetDevice(device), "hipGetDevice");
}

int kvflux_set_device(int device) { return hip_status(hipSetDevice(device), "hipSetDevice"); }

int kvflux_device_malloc(void** ptr, size_t bytes) {
    if (!ptr) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "ptr is null");
    *ptr = nullptr;
    if (bytes == 0) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "zero-byte device allocation");
    return hip_status(hipMalloc(ptr, bytes), "hipMalloc");
}

int kvflux_device_free(void* ptr) { return hip_status(hipFree(ptr), "hipFree"); }

int kvflux_host_malloc_pinned(void** ptr, size_t bytes) {
    if (!ptr) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "ptr is null");
    *ptr = nullptr;
    return hip_status(hipHostMalloc(ptr, bytes, hipHostMallocMapped), "hipHostMalloc");
}

int kvflux_host_free_pinned(void* ptr) { return hip_status(hipHostFree(ptr), "hipHostFree"); }

int kvflux_host_device_pointer(void* host_ptr, void** device_ptr) {
    if (!host_ptr || !device_ptr) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "pointer is null");
    *device_ptr = nullptr;
    return hip_status(hipHostGetDevicePointer(device_ptr, host_ptr, 0), "hipHostGetDevicePointer");
}

int kvflux_pointer_device(const void* ptr, int* device) {
    if (!device) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "device is null");
    *device = -1;
    if (!ptr) return KVFLUX_OK;
    hipPointerAttribute_t attributes{};
    const hipError_t e = hipPointerGetAttributes(&attributes, ptr);
    if (e != hipSuccess) {
        (void)hipGetLastError();  // host pointers may leave a sticky error
        return KVFLUX_OK;
    }
    if (attributes.type == hipMemoryTypeDevice) *device = attributes.device;
    return KVFLUX_OK;
}

int kvflux_memcpy_async(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return KVFLUX_OK;
    return hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, as_stream(stream)),
                      "hipMemcpyAsync");
}

int kvflux_memcpy(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return KVFLUX_OK;
    return hip_status(hipMemcpy(dst, src, bytes, hipMemcpyDefault), "hipMemcpy");
}

int kvflux_fill_bytes(void* dst, int value, size_t bytes, void* stream) {
    if (bytes == 0) return KVFLUX_OK;
    if (!dst) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "dst is null");
    if (reinterpret_cast<std::uintptr_t>(dst) % 16 != 0) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "fill destination must be 16-byte aligned");
    }
    const std::uint32_t b = static_cast<std::uint8_t>(value);
    const std::uint32_t word = b | (b << 8) | (b << 16) | (b << 24);
    hipLaunchKernelGGL(fill_bytes_kernel, dim3(byte_grid(bytes)), dim3(kByteThreads), 0,
                       as_stream(stream), static_cast<unsigned char*>(dst), word,
                       static_cast<std::uint64_t>(bytes));
    return launch_status("fill_bytes_kernel");
}

int kvflux_stream_create(void** stream) {
    if (!stream) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "stream is null");
    hipStream_t s = nullptr;
    const int status = hip_status(hipStreamCreateWithFlags(&s, hipStreamNonBlocking),
                                  "hipStreamCreate");
    *stream = s;
    return status;
}

int kvflux_stream_destroy(void* stream) {
    return hip_status(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy");
}

int kvflux_stream_synchronize(void* stream) {
    return hip_status(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
}

int kvflux_device_synchronize(void) {
    return hip_status(hipDeviceSynchronize(), "hipDeviceSynchronize");
}

int kvflux_event_create(void** event) {
    if (!event) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "event is null");
    hipEvent_t e = nullptr;
    const int status = hip_status(hipEventCreate(&e), "hipEventCreate");
    *event = e;
    return status;
}

int kvflux_event_destroy(void* event) {
    return hip_status(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy");
}

int kvflux_event_record(void* event, void* stream) {
    return hip_status(hipEventRecord(static_cast<hipEvent_t>(event), as_stream(stream)),
                      "hipEventRecord");
}

int kvflux_event_synchronize(void* event) {
    return hip_status(hipEventSynchronize(static_cast<hipEvent_t>(event)), "hipEventSynchronize");
}

int kvflux_event_query(void* event, int* complete) {
    if (!complete) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "complete is null");
    const hipError_t e = hipEventQuery(static_cast<hipEvent_t>(event));
    *complete = e == hipSuccess;
    return e == hipErrorNotReady ? KVFLUX_OK : hip_status(e, "hipEventQuery");
}

int kvflux_stream_wait_event(void* stream, void* event) {
    return hip_status(hipStreamWaitEvent(as_stream(stream), static_cast<hipEvent_t>(event), 0),
                      "hipStreamWaitEvent");
}

int kvflux_event_elapsed_ms(float* ms, void* start, void* stop) {
    if (!ms) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "ms is null");
    const int status = hip_status(hipEventSynchronize(static_cast<hipEvent_t>(stop)),
                                  "hipEventSynchronize");
    if (status != KVFLUX_OK) return status;
    return hip_status(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                          static_cast<hipEvent_t>(stop)),
                      "hipEventElapsedTime");
}

int kvflux_fill_random(void* dst, uint64_t count, int dtype, int distribution, uint64_t seed,
                       void* stream) {
    if (count == 0) return KVFLUX_OK;
    if (!dst) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "dst is null");
    if (dtype_bytes(dtype) == 0) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
    if (distribution != 0 && distribution != 1) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "unknown distribution %d", distribution);
    }
    if (reinterpret_cast<std::uintptr_t>(dst) % dtype_bytes(dtype) != 0) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "dst is not aligned to its dtype");
    }
    hipLaunchKernelGGL(fill_random_kernel, dim3(grid_for(count, 256)), dim3(256), 0,
                       as_stream(stream), dst, count, dtype, distribution, seed);
    return launch_status("fill_random_kernel");
}

int kvflux_compare_bytes(const void* a, const void* b, uint64_t bytes, uint64_t* mismatches) {
    if (!mismatches) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "mismatches is null");
    *mismatches = 0;
    if (bytes == 0) return KVFLUX_OK;
    if (!a || !b) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "null buffer");
    if (reinterpret_cast<std::uintptr_t>(a) % 16 || reinterpret_cast<std::uintptr_t>(b) % 16) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "compare buffers must be 16-byte aligned");
    }
    unsigned long long* counter = nullptr;
    int status = hip_status(hipMalloc(&counter, sizeof(*counter)), "hipMalloc compare counter");
    if (status != KVFLUX_OK) return status;
    unsigned long long zero = 0;
    status = hip_status(hipMemcpy(counter, &zero, sizeof(zero), hipMemcpyHostToDevice),
                        "reset compare counter");
    if (status == KVFLUX_OK) {
        hipLaunchKernelGGL(compare_kernel, dim3(byte_grid(bytes)), dim3(kByteThreads), 0,
                           nullptr, static_cast<const unsigned char*>(a),
                           static_cast<const unsigned char*>(b), bytes, counter);
        status = launch_status("compare_kernel");
    }
    unsigned long long result = 0;
    if (status == KVFLUX_OK) {
        status = hip_status(hipMemcpy(&result, counter, sizeof(result), hipMemcpyDeviceToHost),
                            "read compare counter");
    }
    (void)hipFree(counter);
    *mismatches = result;
    return status;
}

} // extern "C"
