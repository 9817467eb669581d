// Paged attention, FP32 arithmetic, split-K ("flash decoding") form.
//
// Semantics follow the reference's attention_element / batch kernel
// (src/v2/paged_attention.cu:73-153): for query row r and query head qh,
//   kv_head = qh / (Hq / H), visible tokens t < len_r,
//   s_t = (q . k_t) / sqrt(D),  o = sum_t softmax(s)_t v_t,
// with K/V read straight from the pages through the block table. The
// reference accumulates in double with one thread per output element; here
// every product and sum is FP32 (agreement with the double CPU reference is
// ~1e-6 for unit-scale data).
//
// gfx950 design (one workgroup = 4 wavefronts = one (row, kv_head, chunk)):
//  * the chunk is CHUNK consecutive tokens of the row; its page ids are
//    staged in LDS once;
//  * all G = Hq/H query heads of the kv head are processed together, so each
//    K and V element is read from HBM once per row (GQA-shared read);
//  * a token row of D elements is split over LPT lanes, DPL contiguous
//    elements (16 or 32 bytes) each, loaded with 128-bit loads; the QK dot
//    product is finished with DPP row operations (quad_perm, row_half_mirror,
//    row_ror) and ds_swizzle, no LDS round trip;
//  * phase A writes the chunk's scores (log2 domain) to LDS, phase B takes
//    the exact chunk max and exp-sum per head (no running rescale), phase C
//    streams V and accumulates p * v; token-lane partial sums are folded with
//    DPP / swizzle and across waves through LDS;
//  * rows longer than CHUNK write (acc, m, l) partials that a second kernel
//    combines in chunk order, so results are bit-reproducible.
#include "common.h"

#include <atomic>
#include <mutex>
#include <cmath>
#include <type_traits>

namespace kvflux_hip {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kChunk = 512;  // tokens per split
constexpr float kLog2e = 1.4426950408889634f;
constexpr std::uint64_t kNoPage = ~0ULL;

// ---------------------------------------------------------------- elements
struct Bf16 {
    using Storage = std::uint16_t;
    static constexpr int kBytes = 2;
};
struct F16 {
    using Storage = std::uint16_t;
    static constexpr int kBytes = 2;
};
struct F32 {
    using Storage = float;
    static constexpr int kBytes = 4;
};

// Widening of packed 32-bit words to floats (exact for every format).
template <typename E>
__device__ inline void widen(const std::uint32_t* w, float* out, int n);

template <>
__device__ inline void widen<Bf16>(const std::uint32_t* w, float* out, int n) {
    for (int i = 0; i < n / 2; ++i) {
        out[2 * i] = __uint_as_float(w[i] << 16);
        out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}

template <>
__device__ inline void widen<F16>(const std::uint32_t* w, float* out, int n) {
    for (int i = 0; i < n / 2; ++i) {
        const auto lo = static_cast<std::uint16_t>(w[i] & 0xffffu);
        const auto hi = static_cast<std::uint16_t>(w[i] >> 16);
        out[2 * i] = static_cast<float>(__builtin_bit_cast(_Float16, lo));
        out[2 * i + 1] = static_cast<float>(__builtin_bit_cast(_Float16, hi));
    }
}

template <>
__device__ inline void widen<F32>(const std::uint32_t* w, float* out, int n) {
    for (int i = 0; i < n; ++i) out[i] = __uint_as_float(w[i]);
}

template <typename E>
__device__ inline float to_float(typename E::Storage x);
template <>
__device__ inline float to_float<Bf16>(std::uint16_t x) {
    return __uint_as_float(static_cast<std::uint32_t>(x) << 16);
}
template <>
__device__ inline float to_float<F16>(std::uint16_t x) {
    return static_cast<float>(__builtin_bit_cast(_Float16, x));
}
template <>
__device__ inline float to_float<F32>(float x) {
    return x;
}

// ---------------------------------------------------------------- lane ops
template <int kCtrl>
__device__ inline float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xf, 0xf, true));
}
constexpr int kQuadXor1 = 0xb1;        // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4e;        // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;  // lane i <- 7-i within 8 lanes
constexpr int kRowRor8 = 0x128;        // lane i <- (i+8) mod 16 within a row
constexpr int kRowRor4 = 0x124;        // lane i <- (i+4) mod 16 within a row
constexpr int kRowRor2 = 0x122;        // lane i <- (i+2) mod 16 within a row

__device__ inline float swizzle_xor16(float x) {
    // ds_swizzle bit mode: and_mask 0x1f, or_mask 0, xor_mask 0x10.
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x401f));
}

// Sum over aligned groups of kWidth lanes (1..32); every lane of the group
// receives the total.
template <int kWidth>
__device__ inline float group_sum(float x) {
    if constexpr (kWidth >= 2) x += dpp<kQuadXor1>(x);
    if constexpr (kWidth >= 4) x += dpp<kQuadXor2>(x);
    if constexpr (kWidth >= 8) x += dpp<kRowHalfMirror>(x);
    if constexpr (kWidth >= 16) x += dpp<kRowRor8>(x);
    if constexpr (kWidth >= 32) x += swizzle_xor16(x);
    return x;
}

__device__ inline float wave_max(float x) {
    x = fmaxf(x, dpp<kQuadXor1>(x));
    x = fmaxf(x, dpp<kQuadXor2>(x));
    x = fmaxf(x, dpp<kRowHalfMirror>(x));
    x = fmaxf(x, dpp<kRowRor8>(x));
    x = fmaxf(x, swizzle_xor16(x));
    return fmaxf(x, __shfl_xor(x, 32));
}

__device__ inline float wave_sum(float x) {
    x = group_sum<32>(x);
    return x + __shfl_xor(x, 32);
}

// exp2(s - m) with the conventions the softmax needs: a masked score
// (-inf) gives 0, and s == m gives 1 even when both are +inf.
__device__ inline float exp2_shifted(float s, float m) {
    if (s == -INFINITY) return 0.0f;
    if (s == m) return 1.0f;
    return exp2f(s - m);
}

// ---------------------------------------------------------------- geometry
template <int kD, int kG>
struct Shape {
    // Elements per lane: 16 keeps Q and the accumulators at 2*G*16 VGPRs;
    // G = 8 uses 8 so the budget stays at 128.
    // Head sizes 96 and 80 (groups of at most 2 and 1 per launch): 24 and 40
    // elements per lane, whole 16-byte vectors of a row split over 4 and 2
    // lanes.
    static constexpr int kDpl = kD == 96 ? 24 : kD == 80 ? 40 : (kD == 64 || kG >= 8) ? 8 : 16;
    static constexpr int kLpt = kD / kDpl;  // lanes per token row
    static constexpr int kTpp = 64 / kLpt;  // tokens per wave pass
    static_assert(kLpt >= 2 && kLpt <= 32 && (kLpt & (kLpt - 1)) == 0, "lane split");
};

struct Params {
    const void* key_cache;
    const void* value_cache;
    std::uint64_t num_blocks;
    std::uint32_t heads;         // H
    FastDiv block_size;          // bs
    const std::uint64_t* table;  // [rows or 1][width]
    std::uint64_t width;
    const std::uint64_t* seq_lens;  // nullable
    std::uint64_t kv_len;
    std::uint32_t num_rows;
    std::uint32_t query_heads;  // Hq
    const float* query;
    float* output;
    float* partial_acc;  // [rows][Hq][max_chunks][D]
    float* partial_ml;   // [rows][Hq][max_chunks][2]
    std::uint32_t max_chunks;  // partial slots per (row, query head): ceil(kv_len / kChunk)
    std::uint32_t row_base;  // first row of this launch slice
    std::uint32_t slice_rows;  // block-size-16 kernel: rows of this launch (at most kPlanRows)
    float scale_log2;        // log2(e) / sqrt(D)
    std::uint32_t chunk_shift;  // block-size-16 kernel: log2(tokens per work item), 9..12
    // Block-size-16 kernel: query heads per kv head (the GQA group), the
    // first of them a launch serves (0), and the head sets of a group above 8
    // (group / sub-group, each a work item of its own; 1 otherwise).
    std::uint32_t q_group;
    std::uint32_t q_first;
    std::uint32_t q_sets;
    // Block-size-16 kernel: log2(block_size / 16) (pages of 16 to 256
    // tokens are cut into 16-token tiles).
    std::uint32_t page_tiles_shift;
    // Block-size-16 kernel on pages of 1 to 8 tokens: log2(16 / block_size)
    // (a 16-token tile gathers its rows from that many pages) and
    // log2(block_size); both 0 for pages of 16 tokens or more.
    std::uint32_t tile_pages_shift;
    std::uint32_t bs_shift;
};

__device__ inline std::uint64_t row_length(const Params& p, std::uint32_t row) {
    return p.seq_lens ? p.seq_lens[row] : p.kv_len - p.num_rows + row + 1;
}

// Loads kDpl elements of one token row (16 or 32 bytes per 16-bit element
// lane, 32 or 64 bytes for FP32) as 32-bit words.
template <typename E, int kDpl>
__device__ inline void load_slice(const typename E::Storage* base, std::uint32_t* w) {
    constexpr int kWords = kDpl * E::kBytes / 4;
    static_assert(kWords % 4 == 0, "slice must be whole 16-byte vectors");
    const auto* src = reinterpret_cast<const uint4*>(base);
#pragma unroll
    for (int v = 0; v < kWords / 4; ++v) {
        const uint4 x = src[v];
        w[4 * v] = x.x;
        w[4 * v + 1] = x.y;
        w[4 * v + 2] = x.z;
        w[4 * v + 3] = x.w;
    }
}

template <typename E, int kD, int kG>
__global__ __launch_bounds__(kThreads, 2) void paged_attention_split_kernel(Params p) {
    using S = Shape<kD, kG>;
    using T = typename E::Storage;
    constexpr int kDpl = S::kDpl, kLpt = S::kLpt, kTpp = S::kTpp;
    constexpr int kWords = kDpl * E::kBytes / 4;
    constexpr int kUnroll = 4;

    __shared__ float scores[kChunk * kG];
    __shared__ float reduce[kWaves * 2 * kG * kD];
    __shared__ std::uint64_t pages[kChunk + 1];
    __shared__ float stats[2 * kG];

    const std::uint32_t chunk = blockIdx.x;
    const std::uint32_t row = p.row_base + blockIdx.y / p.heads;
    const std::uint32_t kvh = blockIdx.y % p.heads;
    const std::uint64_t len = row_length(p, row);
    const std::uint64_t tok_begin = static_cast<std::uint64_t>(chunk) * kChunk;
    if (tok_begin >= len) return;
    const std::uint64_t tok_end = len - tok_begin > kChunk ? tok_begin + kChunk : len;
    const std::uint32_t ntok = static_cast<std::uint32_t>(tok_end - tok_begin);
    const std::uint32_t bs = p.block_size.divisor;

    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int tsub = lane / kLpt, slice = lane % kLpt;

    // Stage the chunk's page ids (invalid ids become kNoPage).
    const std::uint64_t first_page = tok_begin / bs;
    const std::uint32_t npages = static_cast<std::uint32_t>((tok_end - 1) / bs - first_page + 1);
    const std::uint64_t* table_row = p.table + (p.seq_lens ? row : 0) * p.width;
    for (std::uint32_t i = tid; i < npages; i += kThreads) {
        const std::uint64_t logical = first_page + i;
        std::uint64_t id = logical < p.width ? table_row[logical] : kNoPage;
        pages[i] = id < p.num_blocks ? id : kNoPage;
    }

    // Q slice of every head of the group, pre-scaled into the log2 domain.
    const std::uint32_t qh0 = kvh * p.q_group + p.q_first;  // the heads of this launch
    float q[kG][kDpl];
#pragma unroll
    for (int g = 0; g < kG; ++g) {
        const float* src = p.query + (static_cast<std::uint64_t>(row) * p.query_heads + qh0 + g) * kD +
                           slice * kDpl;
#pragma unroll
        for (int i = 0; i < kDpl; ++i) q[g][i] = src[i] * p.scale_log2;
    }
    __syncthreads();

    const T* kc = static_cast<const T*>(p.key_cache);
    const T* vc = static_cast<const T*>(p.value_cache);
    const std::uint64_t head_stride = static_cast<std::uint64_t>(bs) * kD;
    const std::uint64_t page_stride = head_stride * p.heads;

    // Element offset of this lane's slice of chunk token `t_local`, or ~0.
    auto slice_offset = [&](std::uint32_t t_local) -> std::uint64_t {
        const std::uint32_t t = static_cast<std::uint32_t>(tok_begin % bs) + t_local;
        const std::uint32_t pg = p.block_size.div(t);
        const std::uint32_t off = t - pg * bs;
        const std::uint64_t page = pages[pg];
        if (page == kNoPage) return ~0ULL;
        return page * page_stride + kvh * head_stride + static_cast<std::uint64_t>(off) * kD +
               slice * kDpl;
    };

    const std::uint32_t npasses = (ntok + kTpp - 1) / kTpp;

    // ---- phase A: scores of the chunk -> LDS
    for (std::uint32_t p0 = wave; p0 < npasses; p0 += kWaves * kUnroll) {
        std::uint32_t w[kUnroll][kWords];
        bool ok[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const std::uint32_t pass = p0 + u * kWaves;
            const std::uint32_t t_local = pass * kTpp + tsub;
            ok[u] = pass < npasses && t_local < ntok;
            std::uint64_t off = ok[u] ? slice_offset(t_local) : ~0ULL;
            ok[u] = off != ~0ULL;
            if (ok[u]) {
                load_slice<E, kDpl>(kc + off, w[u]);
            } else {
#pragma unroll
                for (int j = 0; j < kWords; ++j) w[u][j] = 0;
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const std::uint32_t pass = p0 + u * kWaves;
            if (pass >= npasses) break;  // uniform across the wave
            float k[kDpl];
            widen<E>(w[u], k, kDpl);
            float dot[kG];
#pragma unroll
            for (int g = 0; g < kG; ++g) {
                float a = 0.0f;
#pragma unroll
                for (int i = 0; i < kDpl; ++i) a = fmaf(q[g][i], k[i], a);
                dot[g] = group_sum<kLpt>(a);
            }
            const std::uint32_t t_local = pass * kTpp + tsub;
            if (slice == 0 && t_local < ntok) {
#pragma unroll
                for (int g = 0; g < kG; ++g) {
                    scores[t_local * kG + g] = ok[u] ? dot[g] : -INFINITY;
                }
            }
        }
    }
    __syncthreads();

    // ---- phase B: exact max and exp-sum of the chunk per head
    for (int g = wave; g < kG; g += kWaves) {
        float m = -INFINITY;
        for (std::uint32_t t = lane; t < ntok; t += 64) m = fmaxf(m, scores[t * kG + g]);
        m = wave_max(m);
        float l = 0.0f;
        for (std::uint32_t t = lane; t < ntok; t += 64) {
            const float e = exp2_shifted(scores[t * kG + g], m);
            scores[t * kG + g] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) {
            stats[2 * g] = m;
            stats[2 * g + 1] = l;
        }
    }
    __syncthreads();

    // ---- phase C: acc[g][:] = sum_t p[t][g] * v_t[slice]
    float acc[kG][kDpl];
#pragma unroll
    for (int g = 0; g < kG; ++g)
#pragma unroll
        for (int i = 0; i < kDpl; ++i) acc[g][i] = 0.0f;

    for (std::uint32_t p0 = wave; p0 < npasses; p0 += kWaves * kUnroll) {
        std::uint32_t w[kUnroll][kWords];
        bool ok[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const std::uint32_t pass = p0 + u * kWaves;
            const std::uint32_t t_local = pass * kTpp + tsub;
            ok[u] = pass < npasses && t_local < ntok;
            std::uint64_t off = ok[u] ? slice_offset(t_local) : ~0ULL;
            ok[u] = off != ~0ULL;
            if (ok[u]) load_slice<E, kDpl>(vc + off, w[u]);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            if (!ok[u]) continue;
            const std::uint32_t t_local = (p0 + u * kWaves) * kTpp + tsub;
            float v[kDpl];
            widen<E>(w[u], v, kDpl);
            float pw[kG];
#pragma unroll
            for (int g = 0; g < kG; ++g) pw[g] = scores[t_local * kG + g];
#pragma unroll
            for (int g = 0; g < kG; ++g)
#pragma unroll
                for (int i = 0; i < kDpl; ++i) acc[g][i] = fmaf(pw[g], v[i], acc[g][i]);
        }
    }

    // Fold token lanes within each 32-lane half, then halves and waves in LDS.
#pragma unroll
    for (int g = 0; g < kG; ++g) {
#pragma unroll
        for (int i = 0; i < kDpl; ++i) {
            float a = acc[g][i];
            if constexpr (kLpt <= 2) a += dpp<kRowRor2>(a);
            if constexpr (kLpt <= 4) a += dpp<kRowRor4>(a);
            if constexpr (kLpt <= 8) a += dpp<kRowRor8>(a);
            if constexpr (kLpt <= 16) a += swizzle_xor16(a);
            acc[g][i] = a;
        }
    }
    if ((lane & 31) < kLpt) {
        float* dst = reduce + ((wave * 2 + lane / 32) * kG) * kD + slice * kDpl;
#pragma unroll
        for (int g = 0; g < kG; ++g)
#pragma unroll
            for (int i = 0; i < kDpl; ++i) dst[g * kD + i] = acc[g][i];
    }
    __syncthreads();

    // max_chunks == 1 means no workspace was provided: never write partials.
    const bool single = len <= kChunk || p.max_chunks <= 1;
    for (int idx = tid; idx < kG * kD; idx += kThreads) {
        float sum = 0.0f;
#pragma unroll
        for (int part = 0; part < kWaves * 2; ++part) sum += reduce[part * kG * kD + idx];
        const int g = idx / kD, d = idx % kD;
        const std::uint64_t out_row = static_cast<std::uint64_t>(row) * p.query_heads + qh0 + g;
        if (single) {
            const float l = stats[2 * g + 1];
            p.output[out_row * kD + d] = l > 0.0f ? sum / l : 0.0f;
        } else {
            const std::uint64_t slot = out_row * p.max_chunks + chunk;
            p.partial_acc[slot * kD + d] = sum;
            if (d == 0) {
                p.partial_ml[2 * slot] = stats[2 * g];
                p.partial_ml[2 * slot + 1] = stats[2 * g + 1];
            }
        }
    }
}

// ---------------------------------------------------------------- MFMA QK decode
// 16-bit caches, head_size 64 or 128: the QK product of each 16-token tile
// runs on v_mfma_f32_16x16x32_{bf16,f16}. Lane l of the A operand holds
// K[token l%16][8*(l/16) + 32*kk ...] exactly as loaded (no conversion); the
// B operand holds Q split into three 16-bit parts (hi + mid + lo = q to
// FP32 precision) in columns split*G + g, so one MFMA per 32 dims gives all
// partial scores and two DPP row shifts add the parts. The softmax is online
// per wavefront (exact running max, rescale only when it grows), P*V stays on
// the VALU in the 8-lanes-per-token layout, and each wavefront double-buffers
// the K and V loads of its next tile.
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

template <typename E>
struct Mfma;
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));

template <>
struct Mfma<Bf16> {
    using Vec = bf16x8_t;
    using Elem = __bf16;
    // x = hi + mid + lo exactly up to the last 8 bits: truncating splits.
    __device__ static void split3(float x, std::uint32_t& hi, std::uint32_t& mid, std::uint32_t& lo) {
        hi = __float_as_uint(x) & 0xffff0000u;
        const float r1 = x - __uint_as_float(hi);
        mid = __float_as_uint(r1) & 0xffff0000u;
        const float r2 = r1 - __uint_as_float(mid);
        lo = __float_as_uint(r2) & 0xffff0000u;
    }
    // Packs the 16-bit payloads of four split words (upper halves).
    __device__ static i16x4_t pack(const std::uint32_t* w) {
        const std::uint32_t a = (w[0] >> 16) | (w[1] & 0xffff0000u);
        const std::uint32_t b = (w[2] >> 16) | (w[3] & 0xffff0000u);
        return __builtin_bit_cast(i16x4_t, make_uint2(a, b));
    }
    __device__ static f32x4_t mma16(const i16x4_t& a, const i16x4_t& b, const f32x4_t& c) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
    }
    __device__ static std::uint16_t split(float x, float* rest) {  // RNE to BF16
        std::uint32_t u = __float_as_uint(x);
        u += 0x7fffu + ((u >> 16) & 1u);
        const std::uint16_t h = static_cast<std::uint16_t>(u >> 16);
        *rest = x - __uint_as_float(static_cast<std::uint32_t>(h) << 16);
        return h;
    }
    __device__ static f32x4_t mma(const Vec& a, const Vec& b, const f32x4_t& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
template <>
struct Mfma<F16> {
    using Vec = f16x8_t;
    using Elem = _Float16;
    // Three FP16 parts, each holding its value in the upper 16 bits.
    __device__ static void split3(float x, std::uint32_t& hi, std::uint32_t& mid, std::uint32_t& lo) {
        const _Float16 h = static_cast<_Float16>(x);
        const float r1 = x - static_cast<float>(h);
        const _Float16 m = static_cast<_Float16>(r1);
        const _Float16 l = static_cast<_Float16>(r1 - static_cast<float>(m));
        hi = static_cast<std::uint32_t>(__builtin_bit_cast(std::uint16_t, h)) << 16;
        mid = static_cast<std::uint32_t>(__builtin_bit_cast(std::uint16_t, m)) << 16;
        lo = static_cast<std::uint32_t>(__builtin_bit_cast(std::uint16_t, l)) << 16;
    }
    __device__ static i16x4_t pack(const std::uint32_t* w) {
        const std::uint32_t a = (w[0] >> 16) | (w[1] & 0xffff0000u);
        const std::uint32_t b = (w[2] >> 16) | (w[3] & 0xffff0000u);
        return __builtin_bit_cast(i16x4_t, make_uint2(a, b));
    }
    __device__ static f32x4_t mma16(const i16x4_t& a, const i16x4_t& b, const f32x4_t& c) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a),
                                                     __builtin_bit_cast(f16x4_t, b), c, 0, 0, 0);
    }
    __device__ static std::uint16_t split(float x, float* rest) {
        const _Float16 h = static_cast<_Float16>(x);
        *rest = x - static_cast<float>(h);
        return __builtin_bit_cast(std::uint16_t, h);
    }
    __device__ static f32x4_t mma(const Vec& a, const Vec& b, const f32x4_t& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

template <int kShift>
__device__ inline std::uint32_t row_shr_u(std::uint32_t x) {  // lane i <- lane i-kShift in a row
    return static_cast<std::uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x110 + kShift, 0xf, 0xf, true));
}
template <int kShift>
__device__ inline float row_shr(float x) {
    return __uint_as_float(row_shr_u<kShift>(__float_as_uint(x)));
}

template <int kShift>
__device__ inline float row_shl(float x) {  // lane i <- lane i+kShift within a 16-lane row
    if constexpr (kShift == 0) {
        return x;
    } else {
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x100 + kShift, 0xf, 0xf, true));
    }
}

// ---------------------------------------------------------------- block_size 16 decode
// Hot path for pages of 1 to 256 tokens: head_size 64/128 with 16-bit and
// FP32 caches, head_size 256 with 16-bit caches (one workgroup per CU there,
// and for FP32 small pages at 128; up to 5 heads per item at 256):
//  * persistent workgroups walk a plan of (row, chunk, kv head) items built
//    in LDS from the row lengths (exclusive prefix of chunk counts), so no
//    workgroup is launched for an empty chunk and consecutive items read the
//    same pages for neighbouring kv heads. A chunk is 512..4096 tokens,
//    chosen per call (the largest that leaves enough items to balance the
//    persistent grid): fewer, longer items mean fewer item epilogues and
//    fewer chunk partials (4096 against 512 tokens: 1.227 against 1.37 ms
//    for 128 rows of U[1024, 32768] tokens on MI355X). Every row's first
//    chunk comes first, then the remaining chunks row by row: rows that
//    share a prefix read it at about the same time, while it is still in
//    the L2 of the XCD serving that kv head (that batch with a 2048-token
//    shared prefix fetched 1.082x its unique bytes in plain row order,
//    1.019x in this one);
//  * a 16-token tile is one page (or a contiguous 1/2, 1/4, 1/8 of one
//    kv head's rows of a 32-, 64- or 128-token page): its base offset is one
//    lane read and every K/V address is that base plus a constant lane
//    offset, and both K and V of a tile arrive as fully coalesced 16-byte
//    loads;
//  * QK^T of a tile is kD/32 MFMA 16x16x32 ops on the raw 16-bit K rows
//    against Q split into hi/mid/lo 16-bit parts (FP32-equivalent); two DPP
//    row shifts add the parts;
//  * online softmax per wavefront; the weights P are split the same way and
//    P*V runs as kD/16 MFMA 16x16x16 ops: V^T (the A operand) comes from the
//    wave's own LDS copy of the tile through the transposing ds_read_tr16_b64,
//    and P^T (the B operand) is exactly the four weights each score lane
//    holds (tokens 4*quad .. 4*quad+3 of its column);
//  * K and V of the next tile are in flight while the current one is computed;
//  * FP32 caches: QK^T is kD/4 v_mfma_f32_16x16x4_f32 on K and Q as they
//    are, and P*V 4 * kD/16 of them on V and the FP32 weights; the dims and
//    tokens each lane takes are ordered so that K, V and Q are read with
//    straight 16-byte loads (no splits, no LDS copy of V): 2.40 against
//    3.03 ms on the VALU split kernel for 128 rows of U[1024, 32768] tokens.
// V tile in LDS: row t (token) holds kD 16-bit values as kD/8 chunks of 16
// bytes; chunk c of row t is stored at slot c ^ ((kD/64) * (t % 8)), which
// makes both the row-wise 16-byte writes and the transposing 8-byte reads
// free of bank conflicts.
constexpr int kPlanRows = 4096;

// Column routing of the three split parts of a per-head value held by lanes
// col < kG of each 16-lane row: set 0 gets hi in columns [0, kG), mid in
// [kG, 2kG) and, when 3kG <= 16, lo in [2kG, 3kG); otherwise lo goes to the
// second set (columns [0, kG), handled by the caller). Lanes whose column is
// not covered keep hi (those output columns are never read). With kG a
// multiple of 4 the moves are bank-masked DPP writes of whole 4-lane banks.
template <int kShift, int kBanks>
__device__ inline std::uint32_t dpp_shr_into(std::uint32_t old, std::uint32_t src) {
    return static_cast<std::uint32_t>(__builtin_amdgcn_update_dpp(
        static_cast<int>(old), static_cast<int>(src), 0x110 + kShift, 0xf, kBanks, false));
}

// x *= a with the result tied to x's register (a plain multiply under a
// rarely taken branch makes the register allocator copy every accumulator
// on the other path).
__device__ inline void scale_in_place(f32x4_t& v, float a) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float x = v[r];
        asm volatile("v_mul_f32 %0, %0, %1" : "+v"(x) : "v"(a));
        v[r] = x;
    }
}

template <int kG, int kSets>
__device__ inline std::uint32_t route(std::uint32_t hi, std::uint32_t mid, std::uint32_t lo, int col) {
    if constexpr (kG == 4) {
        return dpp_shr_into<8, 0x4>(dpp_shr_into<4, 0x2>(hi, mid), lo);
    } else if constexpr (kG == 8) {
        static_assert(kSets == 2, "lo of 8 heads goes to the second set");
        return dpp_shr_into<8, 0xc>(hi, mid);
    } else {
        const std::uint32_t mid_up = row_shr_u<kG>(mid), lo_up = row_shr_u<2 * kG>(lo);
        return col < kG ? hi : col < 2 * kG ? mid_up : col < 3 * kG ? lo_up : hi;
    }
}

typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

// kSmall: pages of 1 to 8 tokens. A 16-token tile then spans
// 2^tile_pages_shift pages; lane j of a wave holds the offset of page slot j
// of the wave's tiles (tile j >> tile_pages_shift, page j & mask of it; the
// item size keeps them within 64), and every lane takes the page of its own
// token row from the lane holding it (a cross-lane read), where whole tiles
// take one wave-uniform page.
// One workgroup per CU (the registers of two) at head_size 256 and for FP32
// tiles gathered from small pages at head_size 128.
template <typename E, int kD, bool kSmall>
constexpr int bs16_occupancy() {
    return kD == 256 || (std::is_same<E, F32>::value && kD == 128 && kSmall) ? 1 : 2;
}
template <typename E, int kD, int kG, bool kSmall>
constexpr int bs16_occupancy_g() {
    return kG > 8 && kD == 128 && !std::is_same<E, F32>::value ? 1 : bs16_occupancy<E, kD, kSmall>();
}

template <typename E, int kD, int kG, bool kSmall>
__global__ __launch_bounds__(kThreads, (bs16_occupancy_g<E, kD, kG, kSmall>())) void paged_decode_bs16_kernel(Params p) {
    // FP32 caches: QK^T and P*V on v_mfma_f32_16x16x4_f32 with FP32 K, V, Q
    // and weights as they are (no splits, no LDS staging of V).
    constexpr bool kF32 = std::is_same<E, F32>::value;
    using M = Mfma<typename std::conditional<kF32, Bf16, E>::type>;
    using Vec = typename M::Vec;
    using T = typename E::Storage;
    constexpr int kBs = 16;
    constexpr int kF32Chunks = kD / 16;     // FP32: 16-byte K (and V) loads per lane per tile
    constexpr int kSteps = kD / 32;         // QK MFMAs per tile (32 dims each)
    constexpr int kDt = kD / 16;            // P*V MFMAs per tile (16 dims each)
    constexpr int kCpr = kD / 8;            // 16-byte chunks per token row
    constexpr int kVLoads = kD / 32;        // 16-byte V chunks per lane per tile
    constexpr int kRowStep = 64 / kCpr;     // token rows covered by one wave-wide load
    constexpr int kSwz = kCpr / 8;          // LDS slot swizzle multiplier
    // Column sets of the split Q parts: one for G <= 5 (hi, mid, lo of G heads
    // side by side), two for G = 6..8 (lo in the second), three for G = 9..16
    // (set s holds part s of every head, column = head).
    constexpr int kSets = kF32 || 3 * kG <= 16 ? 1 : kG <= 8 ? 2 : 3;
    constexpr int kRowBytes = kD * 2;
    constexpr int kQPer = (kG * kD + kThreads - 1) / kThreads;
    static_assert(kRowStep * kVLoads == kBs, "V tile covers 16 tokens");
    // Chunk of 2^chunk_shift tokens (256..4096): 16..256 tiles per item, so
    // 4..64 (even) tiles per wavefront, whose page offsets fit one lane each
    // (small pages: whose page slots fit one lane each).
    const std::uint32_t chunk_shift = p.chunk_shift;
    const std::uint32_t chunk_tokens = 1u << chunk_shift;
    const std::uint32_t tiles = chunk_tokens / kBs;  // tiles per item
    const int per_wave = static_cast<int>(tiles / kWaves);
    // ceil(len / chunk_tokens) without wrapping for len near 2^32.
    auto chunks_of = [&](std::uint32_t len) {
        return (len >> chunk_shift) + ((len & (chunk_tokens - 1)) != 0 ? 1u : 0u);
    };

    __shared__ std::uint32_t plan[kPlanRows + 1];
    __shared__ std::uint32_t lens[kPlanRows];
    __shared__ std::uint32_t scan[kThreads];
    // 16-bit caches: Q split in three 16-bit parts; FP32: Q as floats (two
    // 16-bit slots each). V tiles are staged for the transposing reads of the
    // 16-bit path only.
    __shared__ __attribute__((aligned(16))) std::uint16_t qsplit[2][(kF32 ? 2 : 3) * kG * kD];
    __shared__ __attribute__((aligned(16))) std::uint16_t vtile[kWaves][kF32 ? 8 : kBs * kD];
    __shared__ __attribute__((aligned(16))) float reduce[kWaves * kG * kD];
    __shared__ float wstats[kWaves][2 * kG];

    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int col = lane % 16, quad = lane / 16;
    // This launch's rows: p.row_base + r for r < rows (a batch of more than
    // kPlanRows rows runs as launches of kPlanRows-row slices).
    const std::uint32_t rows = p.slice_rows;

    // ---- plan: lens[r] = row length (clamped to kv_len), plan[r] = number
    // of chunks of rows < r (a zero-length row still owns one chunk so its
    // output is written).
    constexpr int kPer = kPlanRows / kThreads;
    std::uint32_t mine = 0;
    for (int i = 0; i < kPer; ++i) {
        const std::uint32_t r = tid * kPer + i;
        if (r < rows) {
            const std::uint64_t full = row_length(p, p.row_base + r);
            const std::uint32_t len = static_cast<std::uint32_t>(full < p.kv_len ? full : p.kv_len);
            lens[r] = len;
            mine += len == 0 ? 1u : chunks_of(len);
        }
    }
    scan[tid] = mine;
    __syncthreads();
    for (int off = 1; off < kThreads; off <<= 1) {
        const std::uint32_t add = tid >= off ? scan[tid - off] : 0u;
        __syncthreads();
        scan[tid] += add;
        __syncthreads();
    }
    {
        std::uint32_t run = scan[tid] - mine;
        for (int i = 0; i < kPer; ++i) {
            const std::uint32_t r = tid * kPer + i;
            if (r < rows) {
                plan[r] = run;
                run += lens[r] == 0 ? 1u : chunks_of(lens[r]);
            }
        }
        if (tid == kThreads - 1) plan[rows] = scan[tid];
    }
    __syncthreads();
    const std::uint32_t total = plan[rows] * p.heads * p.q_sets;

    const T* kc = static_cast<const T*>(p.key_cache);
    const T* vc = static_cast<const T*>(p.value_cache);
    // A page holds 2^page_tiles_shift 16-token tiles of every kv head:
    // tile t of a row is tile t % 2^shift of page t >> shift. Small pages
    // (kSmall): 2^tile_pages_shift pages per tile, one kv head's block of a
    // page being bs rows.
    const std::uint32_t tile_shift = p.page_tiles_shift;
    const std::uint32_t tps = kSmall ? p.tile_pages_shift : 0u;
    const std::uint32_t bs_shift = p.bs_shift;
    const std::uint64_t head_stride =
        kSmall ? (static_cast<std::uint64_t>(1) << bs_shift) * kD : static_cast<std::uint64_t>(kBs << tile_shift) * kD;
    const std::uint64_t page_stride = head_stride * p.heads;
    // K: lane (quad, col) loads token col, dims 8*quad + 32*kk .. +8.
    const std::uint32_t k_lane = col * kD + quad * 8;
    // V: lane loads chunk lane + 64*i of the tile (contiguous 1 KiB per load).
    const std::uint32_t v_lane = lane * 8;
    char* const my_tile = reinterpret_cast<char*>(vtile[wave]);
    std::uint32_t v_store[kVLoads];  // swizzled LDS byte offset of each loaded chunk
#pragma unroll
    for (int i = 0; i < kVLoads; ++i) {
        const int t = lane / kCpr + i * kRowStep, c = lane % kCpr;
        v_store[i] = t * kRowBytes + ((c ^ (kSwz * (t % 8))) * 16);
    }
    // Transposing read of the 16x16 block dt: lane (q, s) addresses token
    // 4q + s/4, dims 16*dt + 4*(s%4) .. +4. The swizzle acts on bits 4..6 of
    // the byte offset and dt on bits 5..7, so block dt is base ^ (dt << 5).
    std::uint32_t v_read;
    {
        const int s = lane % 16, t = 4 * quad + s / 4;
        const int c = (4 * (s % 4)) / 8;
        v_read = t * kRowBytes + ((c ^ (kSwz * (t % 8))) * 16) + (s % 2) * 8;
    }

    // ---- work items: (row, chunk, kv head), item = rc * H + kvh. rc < rows
    // is chunk 0 of row rc; rc >= rows walks the later chunks row by row
    // (the chunks after each row's first: plan[r] - r of them before row r).
    // Every global load of the item loop is unconditional (invalid tiles read
    // page 0 and are masked), so the compiler's wait counts stay exact and
    // the tile stream never drains.
    struct Item {
        std::uint32_t row, chunk, kvh, qf, ntok;  // qf: first query head of the item's head set
    };
    auto uniform = [](std::uint32_t x) { return static_cast<std::uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(x))); };
    auto locate = [&](std::uint32_t item) -> Item {
        Item it;
        // Block q = (row/chunk) * heads + kv head. Blocks go in groups of 8,
        // each group as its head sets one after another (item = group * 8 *
        // sets + set * 8 + q % 8), so the sets of a block are 8 items apart:
        // with a persistent grid that is a multiple of 8 they run on one XCD
        // at about the same time and the later ones find the pages in its L2.
        // The blocks past the last whole group take the sets in turn. With
        // one set this is item = q.
        const std::uint32_t group_items = 8u * p.q_sets;
        const std::uint32_t whole = (total / group_items) * group_items;
        std::uint32_t q, set;
        if (item < whole) {
            const std::uint32_t in_group = item % group_items;
            set = in_group / 8u;
            q = (item / group_items) * 8u + in_group % 8u;
        } else {
            const std::uint32_t tail_blocks = (total - whole) / p.q_sets;
            set = (item - whole) / tail_blocks;
            q = whole / p.q_sets + (item - whole) % tail_blocks;
        }
        it.kvh = uniform(q % p.heads);
        it.qf = uniform(set * kG);
        const std::uint32_t rc = q / p.heads;
        if (rc < rows) {
            it.row = uniform(rc);
            it.chunk = 0;
        } else {
            const std::uint32_t rx = rc - rows;
            std::uint32_t lo = 0, hi = rows;  // plan[lo] - lo <= rx < plan[hi] - hi
            while (hi - lo > 1) {
                const std::uint32_t mid = (lo + hi) / 2;
                if (plan[mid] - mid <= rx) lo = mid; else hi = mid;
            }
            it.row = uniform(lo);
            it.chunk = uniform(rx - (plan[it.row] - it.row) + 1);
        }
        const std::uint32_t len = lens[it.row];
        const std::uint32_t begin = it.chunk << chunk_shift;
        it.ntok = uniform(len > begin ? (len - begin < chunk_tokens ? len - begin : chunk_tokens) : 0u);
        return it;
    };
    // Lane j < per_wave of every wave: element offset of the page of tile
    // wave + kWaves * j, or kNoPage. Small pages: lane j < per_wave << tps
    // holds page slot j (page j & (2^tps - 1) of tile wave + kWaves * (j >> tps)).
    auto fetch_pages = [&](const Item& it) -> std::uint64_t {
        const std::uint64_t* table_row =
            p.table + (p.seq_lens ? static_cast<std::uint64_t>(p.row_base) + it.row : 0) * p.width;
        if constexpr (kSmall) {
            const std::uint32_t j = lane & ((per_wave << tps) - 1);
            const std::uint64_t tile = static_cast<std::uint64_t>(it.chunk) * tiles + wave + kWaves * (j >> tps);
            const std::uint64_t logical = (tile << tps) + (j & ((1u << tps) - 1));
            const std::uint64_t id = table_row[logical < p.width ? logical : p.width - 1];
            return logical < p.width && id < p.num_blocks ? id * page_stride : kNoPage;
        } else {
            const std::uint64_t tile = static_cast<std::uint64_t>(it.chunk) * tiles + wave + kWaves * (lane & (per_wave - 1));
            const std::uint64_t logical = tile >> tile_shift;
            const std::uint64_t id = table_row[logical < p.width ? logical : p.width - 1];
            const std::uint64_t in_page = (tile & ((1u << tile_shift) - 1)) * (kBs * kD);
            return logical < p.width && id < p.num_blocks ? id * page_stride + in_page : kNoPage;
        }
    };
    // Small pages: the offset page slot `slot` holds, read from its lane
    // (kNoPage reads page 0; such rows are masked).
    auto slot_offset = [](std::uint64_t pages, std::uint32_t slot) -> std::uint64_t {
        const auto lo32 = static_cast<std::uint32_t>(__shfl(static_cast<int>(pages), static_cast<int>(slot)));
        const auto hi32 = static_cast<std::uint32_t>(__shfl(static_cast<int>(pages >> 32), static_cast<int>(slot)));
        const std::uint64_t off = (static_cast<std::uint64_t>(hi32) << 32) | lo32;
        return off == kNoPage ? 0 : off;
    };
    // Query elements tid + kThreads * i of the item's kG heads (clamped).
    auto fetch_query = [&](const Item& it, float (&q)[kQPer]) {
        const float* base =
            p.query + ((static_cast<std::uint64_t>(p.row_base) + it.row) * p.query_heads + it.kvh * p.q_group + p.q_first +
                       it.qf) * kD;
#pragma unroll
        for (int i = 0; i < kQPer; ++i) {
            const int idx = tid + kThreads * i;
            q[i] = base[idx < kG * kD ? idx : kG * kD - 1];
        }
    };
    auto stage_query = [&](const float (&q)[kQPer], int s) {
#pragma unroll
        for (int i = 0; i < kQPer; ++i) {
            const int idx = tid + kThreads * i;
            if (idx < kG * kD) {
                const int g = idx / kD, d = idx % kD;
                const float x = q[i] * p.scale_log2;
                if constexpr (kF32) {
                    reinterpret_cast<float*>(qsplit[s])[g * kD + d] = x;
                } else {
                    float rest;
                    qsplit[s][(0 * kG + g) * kD + d] = M::split(x, &rest);
                    qsplit[s][(1 * kG + g) * kD + d] = M::split(rest, &rest);
                    qsplit[s][(2 * kG + g) * kD + d] = M::split(rest, &rest);
                }
            }
        }
    };
    auto page_of = [](std::uint64_t pages, int j) -> std::uint64_t {
        const std::uint32_t lo32 = static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(pages), j));
        const std::uint32_t hi32 = static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(pages >> 32), j));
        return (static_cast<std::uint64_t>(hi32) << 32) | lo32;
    };

    struct Tile {
        uint4 k[kF32 ? kF32Chunks : kSteps];
        uint4 v[kF32 ? kF32Chunks : kVLoads];
    };
    auto load = [&](std::uint64_t off, std::uint32_t kvh, Tile& b) {
        const std::uint64_t base = (off == kNoPage ? 0 : off) + kvh * head_stride;
        if constexpr (kF32) {
            // K: lane (quad, col) takes token col, 16-byte chunks 4m + quad
            // (two loads complete each 128-byte line). V: token 4 * quad + kk,
            // chunks 16 * mm + col (whole lines per load, streamed).
            const T* kb = kc + base + col * kD + quad * 4;
            const T* vb = vc + base + (4 * quad) * kD + col * 4;
#pragma unroll
            for (int m = 0; m < kF32Chunks; ++m) b.k[m] = *reinterpret_cast<const uint4*>(kb + 16 * m);
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                for (int mm = 0; mm < kD / 64; ++mm)
                    b.v[kk * (kD / 64) + mm] = stream_load(reinterpret_cast<const uint4*>(vb + kk * kD + 64 * mm));
            return;
        }
        const T* kb = kc + base + k_lane;
        const T* vb = vc + base + v_lane;
#pragma unroll
        for (int kk = 0; kk < kSteps; ++kk) b.k[kk] = *reinterpret_cast<const uint4*>(kb + kk * 32);
#pragma unroll
        // V rows arrive as whole 1 KiB lines per load: streamed (non-temporal).
        // K loads take 64 bytes of each of 16 token rows, so a 128-byte line
        // is completed by a second load and K keeps the default policy.
        for (int i = 0; i < kVLoads; ++i) b.v[i] = stream_load(reinterpret_cast<const uint4*>(vb + i * 512));
    };
    // Small pages: tile `jt` of the wave in `pages` (slots jt << tps ..).
    // Token t of the tile is row t & (bs - 1) of slot (jt << tps) + (t >> bs_shift).
    auto load_small = [&](std::uint64_t pages, std::uint32_t jt, std::uint32_t kvh, Tile& b) {
        const std::uint32_t first = jt << tps;
        const std::uint32_t bs_mask = (1u << bs_shift) - 1;
        const std::uint64_t head = kvh * head_stride;
        if constexpr (kF32) {
            // The lanes of load(), each token row from its own page slot.
            {
                const std::uint32_t t = static_cast<std::uint32_t>(col);
                const T* kb = kc + slot_offset(pages, first + (t >> bs_shift)) + head + (t & bs_mask) * kD + quad * 4;
#pragma unroll
                for (int m = 0; m < kF32Chunks; ++m) b.k[m] = *reinterpret_cast<const uint4*>(kb + 16 * m);
            }
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const std::uint32_t t = static_cast<std::uint32_t>(4 * quad + kk);
                const T* vb = vc + slot_offset(pages, first + (t >> bs_shift)) + head + (t & bs_mask) * kD + col * 4;
#pragma unroll
                for (int mm = 0; mm < kD / 64; ++mm)
                    b.v[kk * (kD / 64) + mm] = stream_load(reinterpret_cast<const uint4*>(vb + 64 * mm));
            }
            return;
        }
        {
            const std::uint32_t t = static_cast<std::uint32_t>(col);
            const T* kb = kc + slot_offset(pages, first + (t >> bs_shift)) + head + (t & bs_mask) * kD + quad * 8;
#pragma unroll
            for (int kk = 0; kk < kSteps; ++kk) b.k[kk] = *reinterpret_cast<const uint4*>(kb + kk * 32);
        }
#pragma unroll
        for (int i = 0; i < kVLoads; ++i) {
            const std::uint32_t t = static_cast<std::uint32_t>(lane / kCpr + i * kRowStep);
            const T* vb = vc + slot_offset(pages, first + (t >> bs_shift)) + head + (t & bs_mask) * kD + (lane % kCpr) * 8;
            b.v[i] = stream_load(reinterpret_cast<const uint4*>(vb));
        }
    };
    // Leading valid pages of tile jt (small pages): those before the tile's
    // first missing page slot, from a wave-wide ballot of missing slots.
    auto leading_pages = [&](std::uint64_t missing, std::uint32_t jt) -> std::uint32_t {
        const std::uint32_t n = 1u << tps;
        const std::uint64_t bits = (missing >> (jt << tps)) & ((n == 64 ? ~0ULL : (1ULL << n) - 1));
        return bits ? static_cast<std::uint32_t>(__builtin_ctzll(bits)) : n;
    };

    // run_max is a reference point, not always the exact maximum: it only
    // moves when a score exceeds it by more than kLazy (log2 units), so
    // weights stay <= 2^kLazy and rescales are rare. FP16 caches: FP16's
    // exponent stops at 2^-24, so an unscaled weight below that would vanish
    // from the P*V numerator while counting in the FP32 sum. There every
    // weight stays <= 1 (the reference moves with each new maximum) and the
    // split takes 2^15 times it (<= 32768): a leading part loses bits to
    // FP16's subnormals only below 2^-29 of the maximum and vanishes only
    // below 2^-39, where 2^15 such keys together weigh under 2^-24 of the
    // row. The wave totals are multiplied by 2^-15 (exact) before the block
    // combine.
    constexpr bool kF16Weights = !kF32 && std::is_same<E, F16>::value;
    constexpr float kLazy = kF16Weights ? 0.0f : 8.0f;
    constexpr float kWeightScale = kF16Weights ? 32768.0f : 1.0f;
    float run_max, run_sum, run_low;  // run_low: the low word of run_sum (compensated sum)
    f32x4_t acc[kSets][kDt];
    Vec qb[kSets][kF32 ? 1 : kSteps];
    float qf[kF32 ? kD / 4 : 1];  // FP32: Q of head col, dims 16 * (kk / 4) + 4 * quad + kk % 4

    // consume(): V of the tile into the wave's LDS slot and the QK^T MFMAs;
    // after it the tile's registers are free for the next load.
    struct Scores {
        f32x4_t s0, s1, s2;  // one per column set (s2: groups 9..16)
        std::uint32_t valid;
    };
    auto consume = [&](std::uint32_t valid, const Tile& b) -> Scores {
        Scores out;
        out.valid = valid;
        if constexpr (kF32) {
            // S^T = K Q^T over dims: MFMA kk takes, in lane (quad, col), dim
            // 16 * (kk / 4) + 4 * quad + kk % 4 of token col (K) and of head
            // col (Q, in qf[kk]); the dim order does not change the sum.
            out.s0 = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            out.s1 = out.s0;
#pragma unroll
            for (int m = 0; m < kF32Chunks; ++m) {
                const float kx[4] = {__uint_as_float(b.k[m].x), __uint_as_float(b.k[m].y), __uint_as_float(b.k[m].z),
                                     __uint_as_float(b.k[m].w)};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    out.s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(kx[j], qf[4 * m + j], out.s0, 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int i = 0; i < kVLoads; ++i) *reinterpret_cast<uint4*>(my_tile + v_store[i]) = b.v[i];
            if (valid < kBs) {  // rows past the end read as zero (0 * NaN would poison P*V)
#pragma unroll
                for (int i = 0; i < kVLoads; ++i) {
                    if (static_cast<std::uint32_t>(lane / kCpr + i * kRowStep) >= valid)
                        *reinterpret_cast<uint4*>(my_tile + v_store[i]) = make_uint4(0, 0, 0, 0);
                }
            }
            out.s0 = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            out.s1 = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            out.s2 = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kk = 0; kk < kSteps; ++kk) {
                const Vec a = __builtin_bit_cast(Vec, b.k[kk]);
                out.s0 = M::mma(a, qb[0][kk], out.s0);
                if constexpr (kSets >= 2) out.s1 = M::mma(a, qb[1][kk], out.s1);
                if constexpr (kSets == 3) out.s2 = M::mma(a, qb[2][kk], out.s2);
            }
        }
        return out;
    };

    // finish(): online softmax of the tile's scores and the P*V MFMAs.
    auto finish_f32 = [&](const Scores& in, const Tile& b) {
        const std::uint32_t valid = in.valid;
        // Lane (quad, col < kG) holds the scores of tokens 4*quad+r, head col.
        float sc[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            sc[r] = in.s0[r];
            if (valid < kBs && static_cast<std::uint32_t>(quad * 4 + r) >= valid) sc[r] = -INFINITY;
        }
        float tmax = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        tmax = fmaxf(tmax, swizzle_xor16(tmax));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const bool grow = tmax > run_max + kLazy;
        const float old_max = run_max;
        if (grow) run_max = tmax;
        const float ref = run_max == -INFINITY ? 0.0f : run_max;
        const float alpha = grow ? __builtin_amdgcn_exp2f(old_max - ref) : 1.0f;
        float pr[4];
        float psum = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            pr[r] = __builtin_amdgcn_exp2f(sc[r] - ref);
            psum += pr[r];
        }
        run_sum *= alpha;  // alpha == 1 unless the reference moved
        run_low *= alpha;
        two_sum_add(run_sum, run_low, psum);
        if (__builtin_expect(__builtin_amdgcn_ballot_w64(col < kG && grow && old_max != -INFINITY) != 0, 0)) {
#pragma unroll
            for (int dt = 0; dt < kDt; ++dt) scale_in_place(acc[0][dt], alpha);
        }
        // O^T += V^T P^T over tokens: MFMA kk takes token 4 * quad + kk in
        // lane (quad, col), the weight the lane holds in pr[kk]; block dt of
        // O^T is dims 64 * (dt / 4) + 4 * i + dt % 4, i = 0..15. V rows of
        // tokens past the end read as zero (0 * NaN would poison P*V).
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const bool live = static_cast<std::uint32_t>(4 * quad + kk) < valid;
#pragma unroll
            for (int mm = 0; mm < kD / 64; ++mm) {
                const uint4 w = b.v[kk * (kD / 64) + mm];
                const float vx[4] = {live ? __uint_as_float(w.x) : 0.0f, live ? __uint_as_float(w.y) : 0.0f,
                                     live ? __uint_as_float(w.z) : 0.0f, live ? __uint_as_float(w.w) : 0.0f};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[0][4 * mm + j] = __builtin_amdgcn_mfma_f32_16x16x4f32(vx[j], pr[kk], acc[0][4 * mm + j], 0, 0, 0);
            }
        }
    };

    auto finish = [&](const Scores& in) {
        if constexpr (!kF32) {
            const std::uint32_t valid = in.valid;
            // Lane (quad, col < kG) holds the scores of tokens 4*quad+r, head col.
            float sc[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if constexpr (kSets == 1) {
                    sc[r] = in.s0[r] + row_shl<kG>(in.s0[r]) + row_shl<2 * kG>(in.s0[r]);
                } else if constexpr (kSets == 2) {
                    sc[r] = in.s0[r] + row_shl<kG>(in.s0[r]) + in.s1[r];
                } else {
                    sc[r] = (in.s0[r] + in.s1[r]) + in.s2[r];
                }
                if (valid < kBs && static_cast<std::uint32_t>(quad * 4 + r) >= valid) sc[r] = -INFINITY;
            }
            float tmax = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
            tmax = fmaxf(tmax, swizzle_xor16(tmax));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
            const bool grow = tmax > run_max + kLazy;
            const float old_max = run_max;
            if (grow) run_max = tmax;
            const float ref = run_max == -INFINITY ? 0.0f : run_max;  // exp2(-inf - ref) = 0
            const float alpha = grow ? __builtin_amdgcn_exp2f(old_max - ref) : 1.0f;

            // Weights, split into three 16-bit parts and routed to the columns
            // (split, head): lane col < kG keeps hi, the mid and lo parts move kG
            // and 2*kG lanes up the row.
            std::uint32_t w0[4], w1[4], w2[4];
            float psum = 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pr = __builtin_amdgcn_exp2f(sc[r] - ref);
                psum += pr;
                std::uint32_t whi, wmid, wlo;
                M::split3(pr * kWeightScale, whi, wmid, wlo);
                if constexpr (kSets == 3) {
                    w0[r] = whi;
                    w1[r] = wmid;
                    w2[r] = wlo;
                } else {
                    w0[r] = route<kG, kSets>(whi, wmid, wlo, col);
                    if constexpr (kSets == 2) w1[r] = wlo;
                }
            }
            run_sum *= alpha;  // alpha == 1 unless the reference moved
            run_low *= alpha;
            two_sum_add(run_sum, run_low, psum);

            // Rescale the columns whose reference point moved (never needed while
            // nothing has been accumulated yet).
            if (__builtin_expect(__builtin_amdgcn_ballot_w64(col < kG && grow && old_max != -INFINITY) != 0, 0)) {
                if constexpr (kSets == 3) {
#pragma unroll
                    for (int m = 0; m < 3; ++m)
#pragma unroll
                        for (int dt = 0; dt < kDt; ++dt) acc[m][dt] *= alpha;
                } else {
                    const float a0 = __uint_as_float(route<kG, kSets>(__float_as_uint(alpha), __float_as_uint(alpha),
                                                                      __float_as_uint(alpha), col));
#pragma unroll
                    for (int dt = 0; dt < kDt; ++dt) acc[0][dt] *= a0;
                    if constexpr (kSets == 2) {
#pragma unroll
                        for (int dt = 0; dt < kDt; ++dt) acc[1][dt] *= alpha;
                    }
                }
            }

            const i16x4_t pb0 = M::pack(w0);
            i16x4_t pb1, pb2;
            if constexpr (kSets >= 2) pb1 = M::pack(w1);
            if constexpr (kSets == 3) pb2 = M::pack(w2);
#pragma unroll
            for (int dt = 0; dt < kDt; ++dt) {
                lds_i16x4_t* src = (lds_i16x4_t*)((__attribute__((address_space(3))) char*)(
                                           (__attribute__((address_space(3))) std::uint16_t*)vtile[wave]) +
                                       (v_read ^ (dt << 5)));
                const i16x4_t va = __builtin_amdgcn_ds_read_tr16_b64_v4i16(src);
                acc[0][dt] = M::mma16(va, pb0, acc[0][dt]);
                if constexpr (kSets >= 2) acc[1][dt] = M::mma16(va, pb1, acc[1][dt]);
                if constexpr (kSets == 3) acc[2][dt] = M::mma16(va, pb2, acc[2][dt]);
            }
        }
    };

    // ---- item loop. Wave w takes tiles w, w + 4, ... (per_wave of them) of
    // every item; its loads run two tiles ahead through item boundaries. The
    // next item's page offsets and query are fetched at the start of the
    // current one.
    std::uint32_t item = blockIdx.x;
    if (item >= total) return;  // uniform over the block
    int sel = 0;
    Item cur = locate(item);
    std::uint64_t cur_pages = fetch_pages(cur);
    {
        float q[kQPer];
        fetch_query(cur, q);
        stage_query(q, 0);
    }
    __syncthreads();
    Tile buf0, buf1;
    if constexpr (kSmall) {
        load_small(cur_pages, 0, cur.kvh, buf0);
        load_small(cur_pages, 1, cur.kvh, buf1);
    } else {
        load(page_of(cur_pages, 0), cur.kvh, buf0);
        load(page_of(cur_pages, 1), cur.kvh, buf1);
    }
    while (true) {
        const std::uint32_t next_item = item + gridDim.x;
        const bool has_next = next_item < total;
        const Item nxt = locate(has_next ? next_item : item);
        const std::uint64_t nxt_pages = fetch_pages(nxt);
        float nq[kQPer];
        fetch_query(nxt, nq);

        if constexpr (kF32) {
            const float* qs = reinterpret_cast<const float*>(qsplit[sel]) + (col < kG ? col : 0) * kD + 4 * quad;
#pragma unroll
            for (int m = 0; m < kF32Chunks; ++m) {
                const float4 x = *reinterpret_cast<const float4*>(qs + 16 * m);
                qf[4 * m] = col < kG ? x.x : 0.0f;
                qf[4 * m + 1] = col < kG ? x.y : 0.0f;
                qf[4 * m + 2] = col < kG ? x.z : 0.0f;
                qf[4 * m + 3] = col < kG ? x.w : 0.0f;
            }
        }
        // B operands from the split table: column -> (split, head). Columns
        // past the last split only feed output columns that are never read.
        if constexpr (!kF32)
#pragma unroll
        for (int m = 0; m < kSets; ++m) {
            int split = col / kG, g = col % kG;
            if (kSets == 2 && m == 1) split = 2;
            if (kSets == 3) {
                split = m;  // set m: part m of head col (columns past the group read head 0)
                g = col < kG ? col : 0;
            }
            if (split > 2) split = 2;
#pragma unroll
            for (int kk = 0; kk < kSteps; ++kk) {
                qb[m][kk] = __builtin_bit_cast(
                    Vec, *reinterpret_cast<const uint4*>(&qsplit[sel][(split * kG + g) * kD + kk * 32 + quad * 8]));
            }
        }
        run_max = -INFINITY;
        run_sum = 0.0f;
        run_low = 0.0f;
#pragma unroll
        for (int m = 0; m < kSets; ++m)
#pragma unroll
            for (int dt = 0; dt < kDt; ++dt) acc[m][dt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

        const std::uint64_t cur_missing = kSmall ? __builtin_amdgcn_ballot_w64(cur_pages == kNoPage) : 0;
        auto valid_of = [&](int j) -> std::uint32_t {
            const std::uint32_t t = wave + kWaves * j;
            const std::uint32_t begin = t * kBs;
            const std::uint32_t n = cur.ntok > begin ? (cur.ntok - begin < kBs ? cur.ntok - begin : kBs) : 0u;
            if constexpr (kSmall) {
                const std::uint32_t ok = leading_pages(cur_missing, static_cast<std::uint32_t>(j)) << bs_shift;
                return n < ok ? n : ok;
            } else {
                return page_of(cur_pages, j) == kNoPage ? 0u : n;
            }
        };
        auto issue = [&](int j, Tile& b) {  // stream position j: this item's tile j or the next item's j - per_wave
            if constexpr (kSmall) {
                if (j < per_wave) {
                    load_small(cur_pages, static_cast<std::uint32_t>(j), cur.kvh, b);
                } else {
                    load_small(nxt_pages, static_cast<std::uint32_t>(j - per_wave), nxt.kvh, b);
                }
            } else if (j < per_wave) {
                load(page_of(cur_pages, j), cur.kvh, b);
            } else {
                load(page_of(nxt_pages, j - per_wave), nxt.kvh, b);
            }
        };
        // Two tiles per step, unrolled once more: a full unroll of 64 tiles
        // would spill. FP32 keeps V in the tile's registers until P*V, so a
        // buffer is reloaded after its tile is finished.
        if constexpr (kF32) {
#pragma unroll 1
            for (int j = 0; j < per_wave; j += 2) {
                finish_f32(consume(valid_of(j), buf0), buf0);
                issue(j + 2, buf0);
                finish_f32(consume(valid_of(j + 1), buf1), buf1);
                issue(j + 3, buf1);
            }
        } else {
#pragma unroll 2
            for (int j = 0; j < per_wave; j += 2) {
                const Scores s0 = consume(valid_of(j), buf0);
                issue(j + 2, buf0);
                finish(s0);
                const Scores s1 = consume(valid_of(j + 1), buf1);
                issue(j + 3, buf1);
                finish(s1);
            }
        }
        if (has_next) stage_query(nq, sel ^ 1);

        // Wave totals: add the split columns (lane col < kG then holds head
        // col, dims 16*dt + 4*quad + r), then the block combine through LDS.
        run_sum += run_low;
        run_sum += swizzle_xor16(run_sum);
        run_sum += __shfl_xor(run_sum, 32);
        if (lane < kG) {
            wstats[wave][2 * lane] = run_max;
            wstats[wave][2 * lane + 1] = run_sum;
        }
        if constexpr (kF32) {
            // acc[0][4 * mm + j][r] is dim 64 * mm + 16 * quad + 4 * r + j of head col.
#pragma unroll
            for (int mm = 0; mm < kD / 64; ++mm)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float4 o = make_float4(acc[0][4 * mm][r], acc[0][4 * mm + 1][r], acc[0][4 * mm + 2][r],
                                                 acc[0][4 * mm + 3][r]);
                    if (col < kG)
                        *reinterpret_cast<float4*>(reduce + (wave * kG + col) * kD + 64 * mm + 16 * quad + 4 * r) = o;
                }
        } else {
#pragma unroll
            for (int dt = 0; dt < kDt; ++dt) {
                float4 o;
                float* op = reinterpret_cast<float*>(&o);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float x = acc[0][dt][r];
                    if constexpr (kSets == 1) {
                        op[r] = x + row_shl<kG>(x) + row_shl<2 * kG>(x);
                    } else if constexpr (kSets == 2) {
                        op[r] = x + row_shl<kG>(x) + acc[1][dt][r];
                    } else {
                        op[r] = (x + acc[1][dt][r]) + acc[2][dt][r];
                    }
                    op[r] *= 1.0f / kWeightScale;  // a power of two: exact
                }
                if (col < kG) *reinterpret_cast<float4*>(reduce + (wave * kG + col) * kD + dt * 16 + quad * 4) = o;
            }
        }
        __syncthreads();

        const bool single = lens[cur.row] <= chunk_tokens || p.max_chunks <= 1;
        const std::uint32_t qh0 = cur.kvh * p.q_group + p.q_first + cur.qf;
        // The thread index is opaque here, so the epilogue's addresses are
        // formed per item rather than hoisted and held through the tile loop
        // (at D = 128, G = 6 and 7 with FP16 they would not fit the registers).
        int first_idx = tid;
        asm volatile("" : "+v"(first_idx));
        for (int idx = first_idx; idx < kG * kD; idx += kThreads) {
            const int g = idx / kD, d = idx % kD;
            float m = -INFINITY;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) m = fmaxf(m, wstats[w][2 * g]);
            float l = 0.0f, sum = 0.0f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float f = exp2_shifted(wstats[w][2 * g], m);
                l += wstats[w][2 * g + 1] * f;
                sum += reduce[w * kG * kD + idx] * f;
            }
            const std::uint64_t out_row = (static_cast<std::uint64_t>(p.row_base) + cur.row) * p.query_heads + qh0 + g;
            if (single) {
                p.output[out_row * kD + d] = l > 0.0f ? sum / l : 0.0f;
            } else {
                const std::uint64_t slot = out_row * p.max_chunks + cur.chunk;
                p.partial_acc[slot * kD + d] = sum;
                if (d == 0) {
                    p.partial_ml[2 * slot] = m;
                    p.partial_ml[2 * slot + 1] = l;
                }
            }
        }
        if (!has_next) break;
        __syncthreads();  // reduce, wstats and qsplit[sel] are reused
        item = next_item;
        cur = nxt;
        cur_pages = nxt_pages;
        sel ^= 1;
    }
}

// Combines the chunk partials of every (row, query head) with more than one
// chunk. One 128-thread block per (row, query head): the chunk weights
// exp2(m_c - m) of 128 chunks at a time go to LDS, then every thread sums its
// dimensions over those chunks with independent loads. All sums run in
// ascending chunk order, so results are deterministic.
constexpr int kCombineThreads = 128;
constexpr int kCombineMaxD = 256;  // largest head_size of the kernels that write partials

__global__ __launch_bounds__(kCombineThreads) void paged_attention_combine_kernel(Params p, std::uint32_t head_dim,
                                                                                   std::uint32_t chunk_tokens) {
    __shared__ float weight[kCombineThreads];
    __shared__ float wave_max_of[kCombineThreads / 64];
    const std::uint32_t row = p.row_base + blockIdx.x / p.query_heads;
    const std::uint32_t qh = blockIdx.x % p.query_heads;
    const std::uint64_t len = row_length(p, row);
    const std::uint64_t needed = (len + chunk_tokens - 1) / chunk_tokens;
    const std::uint32_t nchunks =
        needed < p.max_chunks ? static_cast<std::uint32_t>(needed) : p.max_chunks;
    if (nchunks <= 1) return;  // uniform over the block
    const int tid = threadIdx.x;
    const std::uint64_t out_row = static_cast<std::uint64_t>(row) * p.query_heads + qh;
    const float* ml = p.partial_ml + out_row * p.max_chunks * 2;
    const float* acc = p.partial_acc + out_row * p.max_chunks * head_dim;

    float m = -INFINITY;
    for (std::uint32_t c = tid; c < nchunks; c += kCombineThreads) m = fmaxf(m, ml[2 * c]);
    m = wave_max(m);
    if (tid % 64 == 0) wave_max_of[tid / 64] = m;
    __syncthreads();
    m = fmaxf(wave_max_of[0], wave_max_of[1]);

    constexpr int kDims = kCombineMaxD / kCombineThreads;
    float o[kDims];
#pragma unroll
    for (int j = 0; j < kDims; ++j) o[j] = 0.0f;
    float l = 0.0f;
    for (std::uint32_t c0 = 0; c0 < nchunks; c0 += kCombineThreads) {
        const std::uint32_t n = nchunks - c0 < kCombineThreads ? nchunks - c0 : kCombineThreads;
        __syncthreads();  // the previous tile's weights are no longer read
        if (static_cast<std::uint32_t>(tid) < n) weight[tid] = exp2_shifted(ml[2 * (c0 + tid)], m);
        __syncthreads();
        for (std::uint32_t c = 0; c < n; ++c) l = fmaf(ml[2 * (c0 + c) + 1], weight[c], l);
#pragma unroll
        for (int j = 0; j < kDims; ++j) {
            const std::uint32_t d = tid + kCombineThreads * j;
            if (d < head_dim) {
                const float* src = acc + static_cast<std::uint64_t>(c0) * head_dim + d;
                float sum = o[j];
                std::uint32_t c = 0;
                for (; c + 8 <= n; c += 8) {
                    float v[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) v[u] = src[static_cast<std::uint64_t>(c + u) * head_dim];
#pragma unroll
                    for (int u = 0; u < 8; ++u) sum = fmaf(v[u], weight[c + u], sum);
                }
                for (; c < n; ++c) sum = fmaf(src[static_cast<std::uint64_t>(c) * head_dim], weight[c], sum);
                o[j] = sum;
            }
        }
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int j = 0; j < kDims; ++j) {
        const std::uint32_t d = tid + kCombineThreads * j;
        if (d < head_dim) p.output[out_row * head_dim + d] = o[j] * inv;
    }
}

// Fallback for head sizes / group sizes without a tuned instantiation:
// one wavefront per (row, query head), online softmax over 64-token blocks.
constexpr int kGenericMaxD = 512;

template <typename E>
__global__ __launch_bounds__(64) void paged_attention_generic_kernel(Params p, std::uint32_t head_dim) {
    using T = typename E::Storage;
    __shared__ float qs[kGenericMaxD];
    __shared__ float probs[64];
    const std::uint32_t row = p.row_base + blockIdx.x / p.query_heads;
    const std::uint32_t qh = blockIdx.x % p.query_heads;
    const std::uint32_t group = p.query_heads / p.heads;
    const std::uint32_t kvh = qh / group;
    const std::uint64_t len = row_length(p, row);
    const std::uint32_t bs = p.block_size.divisor;
    const int lane = threadIdx.x;
    const std::uint64_t out_row = static_cast<std::uint64_t>(row) * p.query_heads + qh;
    for (std::uint32_t d = lane; d < head_dim; d += 64) qs[d] = p.query[out_row * head_dim + d] * p.scale_log2;
    __syncthreads();
    const std::uint64_t* table_row = p.table + (p.seq_lens ? row : 0) * p.width;
    const T* kc = static_cast<const T*>(p.key_cache);
    const T* vc = static_cast<const T*>(p.value_cache);
    const std::uint64_t head_stride = static_cast<std::uint64_t>(bs) * head_dim;
    const std::uint64_t page_stride = head_stride * p.heads;

    constexpr int kPer = kGenericMaxD / 64;
    float acc[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) acc[j] = 0.0f;
    float m = -INFINITY, l = 0.0f;

    auto row_offset = [&](std::uint64_t t) -> std::uint64_t {
        const std::uint64_t logical = t / bs;
        const std::uint64_t id = logical < p.width ? table_row[logical] : kNoPage;
        if (id >= p.num_blocks) return ~0ULL;
        return id * page_stride + kvh * head_stride + (t % bs) * head_dim;
    };

    for (std::uint64_t t0 = 0; t0 < len; t0 += 64) {
        const std::uint64_t t = t0 + lane;
        float s = -INFINITY;
        if (t < len) {
            const std::uint64_t off = row_offset(t);
            if (off != ~0ULL) {
                float a = 0.0f;
                for (std::uint32_t d = 0; d < head_dim; ++d) a = fmaf(qs[d], to_float<E>(kc[off + d]), a);
                s = a;
            }
        }
        const float m_new = fmaxf(m, wave_max(s));
        const float e = exp2_shifted(s, m_new);
        const float pr = (t < len && s != -INFINITY) ? e : 0.0f;
        const float alpha = exp2_shifted(m, m_new);
        l = l * alpha + wave_sum(pr);
        probs[lane] = pr;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kPer; ++j) acc[j] *= alpha;
        const std::uint32_t n = len - t0 < 64 ? static_cast<std::uint32_t>(len - t0) : 64;
        for (std::uint32_t j = 0; j < n; ++j) {
            const float w = probs[j];
            if (w == 0.0f) continue;  // uniform: every lane reads the same value
            const std::uint64_t off = row_offset(t0 + j);
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                const std::uint32_t d = lane + 64 * k;
                if (d < head_dim) acc[k] = fmaf(w, to_float<E>(vc[off + d]), acc[k]);
            }
        }
        __syncthreads();
        m = m_new;
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const std::uint32_t d = lane + 64 * k;
        if (d < head_dim) p.output[out_row * head_dim + d] = acc[k] * inv;
    }
}

// ---------------------------------------------------------------- dispatch
//
// A call is planned first and launched second. The plan fixes the kernel
// family, the GQA sub-group of the block-size-16 kernel, its work-item size
// and so the number of chunk partials per (row, query head), which is the
// stride of the partial arrays. Both entry points (caller workspace, static
// scratch) launch the same plan.

// Resident workgroups of one kernel on one device (CUs x occupancy), queried
// once per (kernel, device). Devices past kMaxDevices are queried per call.
constexpr int kMaxDevices = 64;

template <typename E, int kD, int kG, bool kSmall>
int resident_slots(int* out) {
    static std::atomic<int> cache[kMaxDevices];
    int device = 0;
    int status = hip_status(hipGetDevice(&device), "hipGetDevice");
    if (status != KVFLUX_OK) return status;
    if (device >= 0 && device < kMaxDevices) {
        const int known = cache[device].load(std::memory_order_relaxed);
        if (known > 0) {
            *out = known;
            return KVFLUX_OK;
        }
    }
    int cus = 0, per_cu = 0;
    status = hip_status(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device),
                        "hipDeviceGetAttribute");
    if (status == KVFLUX_OK)
        status = hip_status(hipOccupancyMaxActiveBlocksPerMultiprocessor(
                                &per_cu, paged_decode_bs16_kernel<E, kD, kG, kSmall>, kThreads, 0),
                            "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    if (status != KVFLUX_OK) return status;
    const int slots = (cus > 0 ? cus : 1) * (per_cu > 0 ? per_cu : 1);
    if (device >= 0 && device < kMaxDevices) cache[device].store(slots, std::memory_order_relaxed);
    *out = slots;
    return KVFLUX_OK;
}

enum class Family { Bs16, Split, Generic };

struct Plan {
    Family family = Family::Generic;
    std::uint32_t sub = 0;     // Bs16: heads per item; Split: heads per launch (divides the group)
    bool small = false;        // Bs16: pages of 1 to 8 tokens
    std::uint32_t shift = 9;   // Bs16: log2(tokens per work item)
    unsigned grid = 0;         // Bs16: persistent grid
    std::uint64_t chunks = 0;  // partial slots per (row, query head); <= 1: no partials
    std::uint32_t rest = 0;    // Bs16: heads past the last whole set (a second launch), 0 if none
    unsigned rest_grid = 0;    // Bs16: persistent grid of that launch
};

template <typename E, int kD, bool kSmall>
int resident_slots_for(std::uint32_t sub, int* out) {
    switch (sub) {
    case 1: return resident_slots<E, kD, 1, kSmall>(out);
    case 2: return resident_slots<E, kD, 2, kSmall>(out);
    case 3: return resident_slots<E, kD, 3, kSmall>(out);
    case 4: return resident_slots<E, kD, 4, kSmall>(out);
    case 5: return resident_slots<E, kD, 5, kSmall>(out);
    default: break;
    }
    if constexpr ((kSmall && kD == 128 && !std::is_same<E, F32>::value) || kD == 256) {
        return fail(KVFLUX_ERR_UNSUPPORTED, "paged attention: a sub-group of %u", sub);
    } else {
        switch (sub) {
        case 6: return resident_slots<E, kD, 6, kSmall>(out);
        case 7: return resident_slots<E, kD, 7, kSmall>(out);
        case 8: return resident_slots<E, kD, 8, kSmall>(out);
        default: break;
        }
        if constexpr (!kSmall) {
            switch (sub) {
            case 10: return resident_slots<E, kD, 10, kSmall>(out);
            case 12: return resident_slots<E, kD, 12, kSmall>(out);
            case 16: return resident_slots<E, kD, 16, kSmall>(out);
            default: break;
            }
        }
        return fail(KVFLUX_ERR_UNSUPPORTED, "paged attention: a sub-group of %u", sub);
    }
}

// log2 of a power of two.
inline std::uint32_t log2_pow2(std::uint64_t x) {
    std::uint32_t l = 0;
    while ((std::uint64_t{1} << l) < x) ++l;
    return l;
}

// Work-item tokens of the block-size-16 kernel: 2^shift with shift in
// [9, 12] (32..256 tiles per item); pages of bs < 16 tokens cap it at
// 4096 * bs / 16 (the item's page slots fit one per lane of a wave), down to
// 256 tokens at bs = 1.
inline std::uint32_t min_item_shift(std::uint32_t bs) { return bs >= 2 ? 9u : 8u; }
inline std::uint32_t max_item_shift(std::uint32_t bs) { return bs >= 16 ? 12u : 8u + log2_pow2(bs); }

constexpr std::uint32_t kSmallMaxGroup128 = 5;

// The VALU kernels: split at head_size 64/128/256, as launches of the
// largest power of two up to 8 (4 at 256) dividing the group, or generic.
inline int plan_fallback(std::uint64_t head_dim, std::uint64_t group, std::uint64_t max_chunks, Plan* plan) {
    if (head_dim == 64 || head_dim == 128 || head_dim == 256 || head_dim == 96 || head_dim == 80) {
        std::uint64_t sub = head_dim == 256 ? 4 : head_dim == 96 ? 2 : head_dim == 80 ? 1 : 8;
        while (group % sub != 0) sub /= 2;
        plan->family = Family::Split;
        plan->sub = static_cast<std::uint32_t>(sub);
        plan->chunks = max_chunks;
    } else {
        plan->family = Family::Generic;
        plan->chunks = 0;
    }
    return KVFLUX_OK;
}

// max_chunks: ceil(kv_len / kChunk), the partial count at 512-token items.
template <typename E, int kD>
int plan_group(const Params& p, std::uint64_t rows, std::uint64_t group, std::uint64_t max_chunks,
               Plan* plan) {
    if constexpr (kD == 64 || kD == 128 || (kD == 256 && !std::is_same<E, F32>::value)) {
        // The kernel counts work items in 32 bits (at most 512-token chunks);
        // rows <= kPlanRows keeps the product below 2^51.
        const std::uint32_t bs = p.block_size.divisor;
        const bool small = bs == 1 || bs == 2 || bs == 4 || bs == 8;
        // Items are counted in 32 bits; at most 2 * max_chunks of them.
        if ((small || bs == 16 || bs == 32 || bs == 64 || bs == 128 || bs == 256) && p.width > 0 &&
            2 * rows * max_chunks * p.heads <= 0xffffffffULL) {
            // A group above 8 is served as head sets of a sub-group (the
            // largest divisor of the group up to 8), each set a work item of
            // its own in the same launch; the sets of one (row, chunk, kv
            // head) run on one XCD at about the same time, so the later ones
            // read the pages from its L2 (group 16, 128 query / 8 kv heads:
            // 1.98-2.07 ms, against 2.49-2.52 ms as one launch per set reading
            // K/V again). Group 8 at
            // kD = 128 takes 251 VGPRs (no spills, two workgroups per CU):
            // 1.27 against 3.10 ms on the VALU split kernel for 128 rows of
            // U[1024, 32768] tokens with 64 query / 8 kv heads.
            // Small pages at head_size 128 take sub-groups up to 5 (the
            // per-lane page addresses of larger ones exceed the registers).
            // Head size 256 (one workgroup per CU) takes sub-groups up to 5
            // as well; FP32 tiles need no split columns, so any sub-group up
            // to 8 fits.
            const auto g = static_cast<std::uint32_t>(group);
            constexpr bool kF32Cache = std::is_same<E, F32>::value;
            const std::uint32_t cap = (small && kD == 128 && !kF32Cache) || kD == 256 ? kSmallMaxGroup128 : 8u;
            std::uint32_t sub = g < cap ? g : cap;
            while (g % sub != 0) --sub;
            // Pages of 16 tokens or more at head_size 64/128 also take items
            // of 10, 12 or 16 heads (16-bit caches: three column sets; one
            // workgroup per CU at 128), so groups 10, 12 and 16 (and their
            // multiples) read each page once.
            if (!small && kD != 256 && g > 8) {
                for (const std::uint32_t wide : {16u, 12u, 10u}) {
                    if (g % wide == 0) {
                        sub = wide;
                        break;
                    }
                }
            }
            // A group whose largest divisor that fits is small (a prime above
            // 8, say) takes sets of 16 (or 8) heads plus one launch for the
            // heads past the last set, rather than many narrow sets.
            std::uint32_t rest = 0;
            if (!small && kD != 256 && g > 8 && sub < 4) {
                sub = g > 16 && g % 16 <= 8 ? 16u : 8u;
                rest = g % sub;
            }
            const std::uint64_t sets = g / sub;  // head sets per kv head, each its own work items
            if (2 * rows * max_chunks * p.heads * sets > 0xffffffffULL) return plan_fallback(kD, group, max_chunks, plan);
            int rest_slots = 0;
            if (rest > 0) {
                const int st = resident_slots_for<E, kD, false>(rest, &rest_slots);
                if (st != KVFLUX_OK) return st;
            }
            int slots = 0;
            int status = KVFLUX_OK;
            status = small ? resident_slots_for<E, kD, true>(sub, &slots) : resident_slots_for<E, kD, false>(sub, &slots);
            if (status != KVFLUX_OK) return status;
            // Work item size: the largest chunk (up to 4096 tokens, less for
            // small pages) that still gives at least 8 items per resident
            // workgroup when every row is kv_len long.
            std::uint32_t shift = min_item_shift(bs);
            while (shift < max_item_shift(bs)) {
                const std::uint64_t wider =
                    ((p.kv_len + (std::uint64_t{2} << shift) - 1) >> (shift + 1)) * rows * p.heads * sets;
                if (wider < 8 * static_cast<std::uint64_t>(slots)) break;
                ++shift;
            }
            const std::uint64_t chunks = (p.kv_len + (std::uint64_t{1} << shift) - 1) >> shift;
            const std::uint64_t items = rows * chunks * p.heads * sets;  // upper bound of the real count
            plan->family = Family::Bs16;
            plan->sub = sub;
            plan->small = small;
            plan->shift = shift;
            plan->grid = static_cast<unsigned>(items == 0 ? 1 : items < static_cast<std::uint64_t>(slots) ? items : slots);
            plan->chunks = chunks;
            plan->rest = rest;
            const std::uint64_t rest_items = rows * chunks * p.heads;
            plan->rest_grid = static_cast<unsigned>(
                rest_items == 0 ? 1 : rest_items < static_cast<std::uint64_t>(rest_slots) ? rest_items : rest_slots);
            return KVFLUX_OK;
        }
    }
    return plan_fallback(kD, group, max_chunks, plan);
}

template <typename E>
int plan_call(const Params& p, std::uint64_t rows, std::uint64_t head_dim, std::uint64_t group,
              std::uint64_t max_chunks, Plan* plan) {
    switch (head_dim) {
    case 64: return plan_group<E, 64>(p, rows, group, max_chunks, plan);
    case 128: return plan_group<E, 128>(p, rows, group, max_chunks, plan);
    case 256: return plan_group<E, 256>(p, rows, group, max_chunks, plan);
    case 96:
    case 80: return plan_fallback(head_dim, group, max_chunks, plan);
    default: break;
    }
    plan->family = Family::Generic;
    plan->chunks = 0;
    return KVFLUX_OK;
}

int launch_combine(Params p, std::uint32_t head_dim, std::uint32_t chunk_tokens, hipStream_t s) {
    const std::uint64_t per_launch = 0x7fffffffULL / p.query_heads;
    for (std::uint64_t base = 0; base < p.num_rows; base += per_launch) {
        const std::uint64_t n = p.num_rows - base < per_launch ? p.num_rows - base : per_launch;
        p.row_base = static_cast<std::uint32_t>(base);
        hipLaunchKernelGGL(paged_attention_combine_kernel, dim3(static_cast<unsigned>(n * p.query_heads)),
                           dim3(kCombineThreads), 0, s, p, head_dim, chunk_tokens);
        const int status = launch_status("paged_attention_combine_kernel");
        if (status != KVFLUX_OK) return status;
    }
    return KVFLUX_OK;
}

template <typename E, int kD, int kG>
int launch_split_pass(const Params& p, std::uint64_t n, hipStream_t s) {
    hipLaunchKernelGGL((paged_attention_split_kernel<E, kD, kG>),
                       dim3(p.max_chunks > 0 ? p.max_chunks : 1u, static_cast<unsigned>(n * p.heads)),
                       dim3(kThreads), 0, s, p);
    return launch_status("paged_attention_split_kernel");
}

// The split kernel over every row: one launch per `sub` query heads of each
// kv head (sub divides the group), then one combine over all heads.
template <typename E, int kD>
int run_split(Params p, std::uint64_t rows, std::uint32_t sub, hipStream_t s) {
    const std::uint64_t rows_per_launch = 65535 / p.heads;
    for (std::uint64_t base = 0; base < rows; base += rows_per_launch) {
        const std::uint64_t n = rows - base < rows_per_launch ? rows - base : rows_per_launch;
        p.row_base = static_cast<std::uint32_t>(base);
        for (std::uint32_t first = 0; first < p.q_group; first += sub) {
            p.q_first = first;
            int status = KVFLUX_OK;
            if constexpr (kD == 80) {
                status = launch_split_pass<E, kD, 1>(p, n, s);
            } else if constexpr (kD == 96) {
                status = sub == 2 ? launch_split_pass<E, kD, 2>(p, n, s) : launch_split_pass<E, kD, 1>(p, n, s);
            } else {
                switch (sub) {
                case 1: status = launch_split_pass<E, kD, 1>(p, n, s); break;
                case 2: status = launch_split_pass<E, kD, 2>(p, n, s); break;
                case 4: status = launch_split_pass<E, kD, 4>(p, n, s); break;
                default:
                    if constexpr (kD != 256) {
                        status = launch_split_pass<E, kD, 8>(p, n, s);
                    } else {
                        status = fail(KVFLUX_ERR_UNSUPPORTED, "paged attention: split sub-group %u", sub);
                    }
                    break;
                }
            }
            if (status != KVFLUX_OK) return status;
        }
        if (p.max_chunks > 1) {
            hipLaunchKernelGGL(paged_attention_combine_kernel,
                               dim3(static_cast<unsigned>(n * p.query_heads)), dim3(kCombineThreads), 0, s,
                               p, static_cast<std::uint32_t>(kD), static_cast<std::uint32_t>(kChunk));
            const int status = launch_status("paged_attention_combine_kernel");
            if (status != KVFLUX_OK) return status;
        }
    }
    return KVFLUX_OK;
}

template <typename E>
int launch_generic(Params p, std::uint64_t rows, std::uint64_t head_dim, hipStream_t s) {
    const std::uint64_t rows_per_launch = 0x7fffffffULL / p.query_heads;
    for (std::uint64_t base = 0; base < rows; base += rows_per_launch) {
        const std::uint64_t n = rows - base < rows_per_launch ? rows - base : rows_per_launch;
        p.row_base = static_cast<std::uint32_t>(base);
        hipLaunchKernelGGL(paged_attention_generic_kernel<E>,
                           dim3(static_cast<unsigned>(n * p.query_heads)), dim3(64), 0, s, p,
                           static_cast<std::uint32_t>(head_dim));
        const int status = launch_status("paged_attention_generic_kernel");
        if (status != KVFLUX_OK) return status;
    }
    return KVFLUX_OK;
}

template <typename E, int kD, int kG>
int launch_bs16_slice(const Params& p, const Plan& plan, hipStream_t s) {
    if (plan.small) {
        if constexpr (kG <= 8 &&
                      (kD == 64 || (kD == 128 && (std::is_same<E, F32>::value || kG <= static_cast<int>(kSmallMaxGroup128))) ||
                       (kD == 256 && kG <= static_cast<int>(kSmallMaxGroup128)))) {
            hipLaunchKernelGGL((paged_decode_bs16_kernel<E, kD, kG, true>), dim3(plan.grid), dim3(kThreads), 0, s, p);
        } else {
            return fail(KVFLUX_ERR_UNSUPPORTED, "paged attention: small pages with a group of %d", kG);
        }
    } else if constexpr (kD != 256 || kG <= static_cast<int>(kSmallMaxGroup128)) {
        hipLaunchKernelGGL((paged_decode_bs16_kernel<E, kD, kG, false>), dim3(plan.grid), dim3(kThreads), 0, s, p);
    } else {
        return fail(KVFLUX_ERR_UNSUPPORTED, "paged attention: head_size 256 with a group of %d", kG);
    }
    return launch_status("paged_decode_bs16_kernel");
}

// A batch of more than kPlanRows rows runs as launches of kPlanRows-row slices.
template <typename E, int kD, int kG>
int launch_bs16(Params p, const Plan& plan, hipStream_t s) {
    for (std::uint64_t base = 0; base < p.num_rows; base += kPlanRows) {
        p.row_base = static_cast<std::uint32_t>(base);
        p.slice_rows = static_cast<std::uint32_t>(p.num_rows - base < kPlanRows ? p.num_rows - base : kPlanRows);
        const int status = launch_bs16_slice<E, kD, kG>(p, plan, s);
        if (status != KVFLUX_OK) return status;
    }
    return KVFLUX_OK;
}

template <typename E, int kD>
int run_bs16(Params p, const Plan& plan, hipStream_t s) {
    const std::uint32_t bs = p.block_size.divisor;
    p.page_tiles_shift = bs <= 16 ? 0u : log2_pow2(bs) - 4u;
    p.tile_pages_shift = bs < 16 ? 4u - log2_pow2(bs) : 0u;
    p.bs_shift = log2_pow2(bs);
    p.chunk_shift = plan.shift;
    // One launch: a group above 8 is served as head sets of the sub-group,
    // each a work item of its own (and the heads past the last whole set, if
    // any, by a second launch).
    p.q_first = 0;
    p.q_sets = p.q_group / plan.sub;
    int status = KVFLUX_OK;
    if (plan.rest > 0) {
        Params r = p;
        r.q_first = plan.sub * p.q_sets;
        r.q_sets = 1;
        Plan rp = plan;
        rp.grid = plan.rest_grid;
        switch (plan.rest) {
        case 1: status = launch_bs16<E, kD, 1>(r, rp, s); break;
        case 2: status = launch_bs16<E, kD, 2>(r, rp, s); break;
        case 3: status = launch_bs16<E, kD, 3>(r, rp, s); break;
        case 4: status = launch_bs16<E, kD, 4>(r, rp, s); break;
        case 5: status = launch_bs16<E, kD, 5>(r, rp, s); break;
        case 6: status = launch_bs16<E, kD, 6>(r, rp, s); break;
        case 7: status = launch_bs16<E, kD, 7>(r, rp, s); break;
        default: status = launch_bs16<E, kD, 8>(r, rp, s); break;
        }
        if (status != KVFLUX_OK) return status;
    }
    switch (plan.sub) {
    case 1: status = launch_bs16<E, kD, 1>(p, plan, s); break;
    case 2: status = launch_bs16<E, kD, 2>(p, plan, s); break;
    case 3: status = launch_bs16<E, kD, 3>(p, plan, s); break;
    case 4: status = launch_bs16<E, kD, 4>(p, plan, s); break;
    case 5: status = launch_bs16<E, kD, 5>(p, plan, s); break;
    case 6: status = launch_bs16<E, kD, 6>(p, plan, s); break;
    case 7: status = launch_bs16<E, kD, 7>(p, plan, s); break;
    case 8: status = launch_bs16<E, kD, 8>(p, plan, s); break;
    case 10: status = launch_bs16<E, kD, 10>(p, plan, s); break;
    case 12: status = launch_bs16<E, kD, 12>(p, plan, s); break;
    default: status = launch_bs16<E, kD, 16>(p, plan, s); break;
    }
    if (status != KVFLUX_OK) return status;
    if (p.max_chunks > 1) return launch_combine(p, kD, 1u << plan.shift, s);
    return KVFLUX_OK;
}


template <typename E>
int run_plan(Params p, const Plan& plan, std::uint64_t rows, std::uint64_t head_dim, std::uint64_t group,
             hipStream_t s) {
    switch (plan.family) {
    case Family::Bs16:
        if (head_dim == 64) return run_bs16<E, 64>(p, plan, s);
        if constexpr (!std::is_same<E, F32>::value) {
            if (head_dim == 256) return run_bs16<E, 256>(p, plan, s);
        }
        return run_bs16<E, 128>(p, plan, s);
    case Family::Split:
        if (head_dim == 64) return run_split<E, 64>(p, rows, plan.sub, s);
        if (head_dim == 128) return run_split<E, 128>(p, rows, plan.sub, s);
        if (head_dim == 96) return run_split<E, 96>(p, rows, plan.sub, s);
        if (head_dim == 80) return run_split<E, 80>(p, rows, plan.sub, s);
        return run_split<E, 256>(p, rows, plan.sub, s);
    case Family::Generic: break;
    }
    return launch_generic<E>(p, rows, head_dim, s);
}

// Whether a call may write chunk partials (and so needs the workspace): the
// block-size-16 and split kernels at head_size 64/128/256, any group.
bool uses_split(std::uint64_t head_dim, std::uint64_t group) {
    return (head_dim == 64 || head_dim == 128 || head_dim == 256 || head_dim == 96 || head_dim == 80) && group >= 1;
}

// Bytes of the partial arrays for `chunks` slots per (row, query head):
// accumulators first, then (m, l) pairs, both 256-byte aligned.
struct PartialLayout {
    std::uint64_t acc_bytes = 0, total = 0;
};

PartialLayout partial_layout(std::uint64_t rows, std::uint64_t query_heads, std::uint64_t chunks,
                             std::uint64_t head_size) {
    PartialLayout out;
    if (chunks <= 1) return out;
    const std::uint64_t acc = rows * query_heads * chunks * head_size * sizeof(float);
    const std::uint64_t ml = rows * query_heads * chunks * 2 * sizeof(float);
    out.acc_bytes = (acc + 255) & ~std::uint64_t{255};
    out.total = out.acc_bytes + ((ml + 255) & ~std::uint64_t{255});
    return out;
}

// Argument checks shared by both entry points; fills `p` and `plan`.
// *empty = true when there is nothing to do (no rows).
int prepare(const void* key_cache, const void* value_cache, uint64_t num_blocks, uint64_t num_kv_heads,
            uint64_t block_size, uint64_t head_size, int dtype, const uint64_t* block_table,
            uint64_t max_blocks_per_seq, const uint64_t* seq_lens, uint64_t kv_len, uint64_t num_rows,
            uint64_t query_heads, const float* query, float* output, Params* p, Plan* plan) {
    if (dtype_bytes(dtype) == 0) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
    if (!key_cache || !value_cache || !block_table || !query || !output) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged attention: null pointer");
    }
    if (num_blocks == 0 || num_kv_heads == 0 || block_size == 0 || head_size == 0 ||
        query_heads == 0 || query_heads % num_kv_heads != 0) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged attention: invalid shape");
    }
    if (!seq_lens && num_rows > kv_len) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged attention: more queries than tokens");
    }
    if (num_rows > 0xffffffffULL || query_heads > 0xffffffffULL || num_kv_heads > 65535 ||
        block_size > 0xffffffffULL || kv_len > 0xffffffffULL) {
        return fail(KVFLUX_ERR_UNSUPPORTED, "paged attention: dimension too large");
    }
    const std::uint64_t group = query_heads / num_kv_heads;
    if (!uses_split(head_size, group) && head_size > kGenericMaxD) {
        return fail(KVFLUX_ERR_UNSUPPORTED, "paged attention: head_size %llu > %d",
                    static_cast<unsigned long long>(head_size), kGenericMaxD);
    }
    const std::uint64_t max_chunks = (kv_len + kChunk - 1) / kChunk;
    *p = Params{};
    p->key_cache = key_cache;
    p->value_cache = value_cache;
    p->num_blocks = num_blocks;
    p->heads = static_cast<std::uint32_t>(num_kv_heads);
    p->block_size = FastDiv(static_cast<std::uint32_t>(block_size));
    p->table = block_table;
    p->width = max_blocks_per_seq;
    p->seq_lens = seq_lens;
    p->kv_len = kv_len;
    p->num_rows = static_cast<std::uint32_t>(num_rows);
    p->query_heads = static_cast<std::uint32_t>(query_heads);
    p->query = query;
    p->output = output;
    p->q_group = static_cast<std::uint32_t>(group);
    p->q_first = 0;
    p->q_sets = 1;
    p->row_base = 0;
    p->slice_rows = static_cast<std::uint32_t>(num_rows);
    p->scale_log2 = static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(head_size)));
    int status = KVFLUX_OK;
    switch (dtype) {
    case KVFLUX_DTYPE_BF16: status = plan_call<Bf16>(*p, num_rows, head_size, group, max_chunks, plan); break;
    case KVFLUX_DTYPE_F16: status = plan_call<F16>(*p, num_rows, head_size, group, max_chunks, plan); break;
    default: status = plan_call<F32>(*p, num_rows, head_size, group, max_chunks, plan); break;
    }
    if (status != KVFLUX_OK) return status;
    // The partial arrays' stride; 1 (or 0) tells the kernels that no
    // partials are written.
    p->max_chunks = static_cast<std::uint32_t>(plan->chunks);
    return KVFLUX_OK;
}

int launch_prepared(Params p, const Plan& plan, int dtype, std::uint64_t head_size, hipStream_t s) {
    const std::uint64_t group = p.q_group;
    switch (dtype) {
    case KVFLUX_DTYPE_BF16: return run_plan<Bf16>(p, plan, p.num_rows, head_size, group, s);
    case KVFLUX_DTYPE_F16: return run_plan<F16>(p, plan, p.num_rows, head_size, group, s);
    default: return run_plan<F32>(p, plan, p.num_rows, head_size, group, s);
    }
}

} // namespace
} // namespace kvflux_hip

using namespace kvflux_hip;

extern "C" int kvflux_paged_attention_workspace_size(uint64_t num_rows, uint64_t kv_len,
                                                     uint64_t num_kv_heads, uint64_t query_heads,
                                                     uint64_t block_size, uint64_t head_size,
                                                     size_t* bytes) {
    if (!bytes) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "bytes is null");
    *bytes = 0;
    if (num_kv_heads == 0 || query_heads == 0 || query_heads % num_kv_heads != 0) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "invalid attention head counts");
    }
    if (!uses_split(head_size, query_heads / num_kv_heads)) return KVFLUX_OK;
    // Partials of the smallest work item any kernel uses for this call:
    // 512 tokens, 256 on pages of one token.
    const std::uint64_t item = block_size == 1 ? std::uint64_t{1} << min_item_shift(1) : kChunk;
    const std::uint64_t chunks = (kv_len + item - 1) / item;
    if (chunks <= 1) return KVFLUX_OK;
    const long double need = static_cast<long double>(num_rows) * query_heads * chunks *
                             (head_size + 2) * sizeof(float);
    if (need > static_cast<long double>(~std::size_t{0} / 2)) {
        return fail(KVFLUX_ERR_OVERFLOW, "attention workspace size overflow");
    }
    *bytes = partial_layout(num_rows, query_heads, chunks, head_size).total;
    return KVFLUX_OK;
}

extern "C" int kvflux_paged_attention(const void* key_cache, const void* value_cache,
                                      uint64_t num_blocks, uint64_t num_kv_heads,
                                      uint64_t block_size, uint64_t head_size, int dtype,
                                      const uint64_t* block_table, uint64_t max_blocks_per_seq,
                                      const uint64_t* seq_lens, uint64_t kv_len, uint64_t num_rows,
                                      uint64_t query_heads, const float* query, float* output,
                                      void* workspace, size_t workspace_bytes, void* stream) {
    if (num_rows == 0) return KVFLUX_OK;
    Params p;
    Plan plan;
    int status = prepare(key_cache, value_cache, num_blocks, num_kv_heads, block_size, head_size, dtype,
                         block_table, max_blocks_per_seq, seq_lens, kv_len, num_rows, query_heads, query,
                         output, &p, &plan);
    if (status != KVFLUX_OK) return status;
    // The documented size (partials of 512-token items) bounds every plan.
    std::size_t need = 0;
    status = kvflux_paged_attention_workspace_size(num_rows, kv_len, num_kv_heads, query_heads, block_size,
                                                   head_size, &need);
    if (status != KVFLUX_OK) return status;
    if (need > 0 && (!workspace || workspace_bytes < need)) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged attention: workspace needs %zu bytes", need);
    }
    const PartialLayout layout = partial_layout(num_rows, query_heads, plan.chunks, head_size);
    if (layout.total > 0) {
        p.partial_acc = static_cast<float*>(workspace);
        p.partial_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + layout.acc_bytes);
    }
    return launch_prepared(p, plan, dtype, head_size, as_stream(stream));
}

// ---------------------------------------------------------------- no-allocation entry
//
// kvflux_paged_attention_noalloc runs the same plan as kvflux_paged_attention
// with the chunk partials in `scratch`, a file-scope device array of
// KVFLUX_NOALLOC_SCRATCH_BYTES that every device holds from module load until
// the process ends. Host code never passes the array's name to a kernel: its
// device address comes from hipGetSymbolAddress, taken once per device (with
// that device current) at the first call there and kept in scratch_base.
// Every call on one device shares that device's array (its contents are
// whatever the last call left; the kernels need no initialisation), so calls
// that overlap on one device race.
namespace kvflux_hip {

__device__ __attribute__((aligned(256))) unsigned char scratch[KVFLUX_NOALLOC_SCRATCH_BYTES];

namespace {

std::mutex scratch_mutex;
void* scratch_base[kMaxDevices] = {};

// Device address of the current device's copy of `scratch`.
int scratch_address(void** out) {
    int device = 0;
    int status = hip_status(hipGetDevice(&device), "hipGetDevice");
    if (status != KVFLUX_OK) return status;
    const bool cached = device >= 0 && device < kMaxDevices;
    if (cached) {
        std::lock_guard<std::mutex> lock(scratch_mutex);
        if (scratch_base[device]) {
            *out = scratch_base[device];
            return KVFLUX_OK;
        }
    }
    void* ptr = nullptr;
    status = hip_status(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress");
    if (status != KVFLUX_OK) return status;
    if (!ptr) return fail(KVFLUX_ERR_RUNTIME, "hipGetSymbolAddress returned no address for the scratch array");
    if (cached) {
        std::lock_guard<std::mutex> lock(scratch_mutex);
        scratch_base[device] = ptr;
    }
    *out = ptr;
    return KVFLUX_OK;
}

} // namespace
} // namespace kvflux_hip

extern "C" int kvflux_paged_attention_noalloc(const void* key_cache, const void* value_cache,
                                              uint64_t num_blocks, uint64_t num_kv_heads,
                                              uint64_t block_size, uint64_t head_size, int dtype,
                                              const uint64_t* block_table, uint64_t max_blocks_per_seq,
                                              const uint64_t* seq_lens, uint64_t kv_len, uint64_t num_rows,
                                              uint64_t query_heads, const float* query, float* output,
                                              void* stream) {
    if (num_rows == 0) return KVFLUX_OK;
    Params p;
    Plan plan;
    int status = prepare(key_cache, value_cache, num_blocks, num_kv_heads, block_size, head_size, dtype,
                         block_table, max_blocks_per_seq, seq_lens, kv_len, num_rows, query_heads, query,
                         output, &p, &plan);
    if (status != KVFLUX_OK) return status;
    const PartialLayout layout = partial_layout(num_rows, query_heads, plan.chunks, head_size);
    if (layout.total > KVFLUX_NOALLOC_SCRATCH_BYTES) {
        return fail(KVFLUX_ERR_UNSUPPORTED,
                    "paged attention (no allocation): this call needs %llu bytes of chunk partials, "
                    "more than the %llu-byte static scratch; use kvflux_paged_attention with a workspace",
                    static_cast<unsigned long long>(layout.total),
                    static_cast<unsigned long long>(KVFLUX_NOALLOC_SCRATCH_BYTES));
    }
    if (layout.total > 0) {
        void* base = nullptr;
        status = scratch_address(&base);
        if (status != KVFLUX_OK) return status;
        p.partial_acc = static_cast<float*>(base);
        p.partial_ml = reinterpret_cast<float*>(static_cast<char*>(base) + layout.acc_bytes);
    }
    return launch_prepared(p, plan, dtype, head_size, as_stream(stream));
}
