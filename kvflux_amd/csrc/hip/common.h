// Shared helpers of the gfx950 kernels and the C ABI implementation.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "kvflux_hip.h"

namespace kvflux_hip {

// Records `message` as this thread's last error and returns `status`.
int fail(int status, const char* format, ...);
// KVFLUX_OK, or KVFLUX_ERR_RUNTIME carrying "<op>: <hip error string>".
int hip_status(hipError_t error, const char* operation);
// Checks the launch just enqueued (kernel configuration errors).
int launch_status(const char* kernel);

inline std::size_t dtype_bytes(int dtype) {
    switch (dtype) {
    case KVFLUX_DTYPE_F16:
    case KVFLUX_DTYPE_BF16: return 2;
    case KVFLUX_DTYPE_F32: return 4;
    default: return 0;
    }
}

inline hipStream_t as_stream(void* stream) { return static_cast<hipStream_t>(stream); }

inline bool is_pow2(std::uint64_t x) { return x != 0 && (x & (x - 1)) == 0; }

// Division of a 32-bit numerator by a runtime-invariant divisor with one
// multiply-high, an add and a shift (round-up magic number method,
// Granlund & Montgomery 1994): with l = ceil(log2 d) and
// m = floor(2^32 * (2^l - d) / d) + 1, n / d = (umulhi(n, m) + n) >> l for
// every n < 2^32 (the sum is formed in 64 bits).
struct FastDiv {
    std::uint32_t divisor = 1, magic = 1, shift = 0;

    FastDiv() = default;
    explicit FastDiv(std::uint32_t d) : divisor(d) {
        std::uint32_t l = 0;
        while ((std::uint64_t{1} << l) < d) ++l;
        shift = l;
        magic = static_cast<std::uint32_t>(
                    ((std::uint64_t{1} << 32) * ((std::uint64_t{1} << l) - d)) / d) + 1;
    }
    __host__ __device__ std::uint32_t div(std::uint32_t n) const {
        const std::uint64_t hi = (static_cast<std::uint64_t>(n) * magic) >> 32;
        return static_cast<std::uint32_t>((hi + n) >> shift);
    }
    __host__ __device__ std::uint32_t mod(std::uint32_t n) const { return n - div(n) * divisor; }
};

// 16-byte, 8-byte, 4-byte and 2-byte raw vectors for bit-exact copies.
struct alignas(16) V16 { std::uint32_t w[4]; };
struct alignas(8) V8 { std::uint32_t w[2]; };

// Non-temporal load / store of one raw vector (16, 8, 4 or 2 bytes): the
// `nt` form of global_load / global_store, for data touched once (streamed
// pages). Measured on MI355X, a read-only stream of random 32 KiB blocks
// gains 0.5-1.5% with the hint; a copy gains more (the batch gather: 448 ->
// 415 us with non-temporal loads and stores). Loads whose 128-byte
// lines are completed by other instructions of the same wave must not use
// it (the line may be gone before the second half is read).
template <typename Vec>
__device__ inline Vec stream_load(const Vec* p) {
    if constexpr (sizeof(Vec) == 16) {
        typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
        return __builtin_bit_cast(Vec, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p)));
    } else if constexpr (sizeof(Vec) == 8) {
        typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(Vec, __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p)));
    } else {
        return __builtin_nontemporal_load(p);
    }
}
template <typename Vec>
__device__ inline void stream_store(Vec* p, const Vec& v) {
    if constexpr (sizeof(Vec) == 16) {
        typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, v), reinterpret_cast<u32x4_t*>(p));
    } else if constexpr (sizeof(Vec) == 8) {
        typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
        __builtin_nontemporal_store(__builtin_bit_cast(u32x2_t, v), reinterpret_cast<u32x2_t*>(p));
    } else {
        __builtin_nontemporal_store(v, p);
    }
}

// An empty asm that reads v: the loads filling a thread's registers must all
// be complete here, and the compiler cannot sink a load into the branch that
// stores its value. Used between a thread's (unconditional) loads and its
// conditional stores: with loads inside the branches the compiler's wait
// counts turn conservative and every store waits for the previous store
// (vmcnt counts stores on gfx9), which serialises them.
template <typename Vec>
__device__ inline void keep_in_registers(const Vec& v) {
    if constexpr (sizeof(Vec) == 16) {
        typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
        asm volatile("" ::"v"(__builtin_bit_cast(u32x4_t, v)));
    } else if constexpr (sizeof(Vec) == 8) {
        typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
        asm volatile("" ::"v"(__builtin_bit_cast(u32x2_t, v)));
    } else if constexpr (sizeof(Vec) == 4) {
        asm volatile("" ::"v"(__builtin_bit_cast(std::uint32_t, v)));
    } else {
        static_assert(sizeof(Vec) < 4, "raw vectors of 1, 2, 4, 8 or 16 bytes");
        std::uint32_t w = 0;
        __builtin_memcpy(&w, &v, sizeof(Vec));
        asm volatile("" ::"v"(w));
    }
}

// hi + lo += b with the rounding error of the addition kept in lo (Knuth's
// TwoSum: s + e == hi + b exactly). Softmax row sums use it: a row whose
// maximum weight is 1 collects thousands of weights near 2^-25, each below
// half an ulp of the running sum, so a plain FP32 sum drops them all the
// same way. No contraction inside (an FMA would break the identity).
__device__ inline void two_sum_add(float& hi, float& lo, float b) {
#pragma clang fp contract(off)
    const float s = hi + b;
    const float bp = s - hi;
    const float e = (hi - (s - bp)) + (b - bp);
    hi = s;
    lo += e;
}

// Widest power-of-two byte width (<= 16) that divides `row_bytes` and every
// address in `ptrs`.
inline unsigned copy_width(std::uint64_t row_bytes, const void* const* ptrs, int n) {
    for (unsigned w = 16; w > 1; w >>= 1) {
        if (row_bytes % w) continue;
        bool ok = true;
        for (int i = 0; i < n; ++i) ok &= (reinterpret_cast<std::uintptr_t>(ptrs[i]) % w) == 0;
        if (ok) return w;
    }
    return 1;
}

} // namespace kvflux_hip
