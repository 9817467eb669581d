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
    static constexpr int kDpl = (kD == 64 || kG >= 8) ? 8 : 16;
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
    std::uint32_t max_chunks;
    std::uint32_t row_base;  // first row of this launch slice
    float scale_log2;        // log2(e) / sqrt(D)
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
    const std::uint32_t qh0 = kvh * kG;
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
template <>
struct Mfma<Bf16> {
    using Vec = bf16x8_t;
    using Elem = __bf16;
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
__device__ inline float row_shl(float x) {  // lane i <- lane i+kShift within a 16-lane row
    if constexpr (kShift == 0) {
        return x;
    } else {
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x100 + kShift, 0xf, 0xf, true));
    }
}

// ---------------------------------------------------------------- block_size 16 decode
// Hot path for 16-token pages, 16-bit caches, head_size 64/128:
//  * persistent workgroups walk a plan of (row, 512-token chunk, kv head)
//    items built in LDS from the row lengths (exclusive prefix of chunk
//    counts), so no workgroup is launched for an empty chunk and consecutive
//    items read the same pages for neighbouring kv heads;
//  * a 16-token tile is exactly one page: its id is one uniform LDS read and
//    every K/V address is that page's base plus a constant lane offset;
//  * QK^T of a tile is kD/32 MFMA 16x16x32 ops on the raw 16-bit K rows
//    against Q split into hi/mid/lo 16-bit parts (FP32-equivalent); two DPP
//    row shifts add the parts;
//  * online softmax per wavefront, P*V on the VALU (8 lanes per token row),
//    K and V of the next tile in flight while the current one is computed.
constexpr int kPlanRows = 4096;

template <typename E, int kD, int kG>
__global__ __launch_bounds__(kThreads, 2) void paged_decode_bs16_kernel(Params p) {
    using M = Mfma<E>;
    using Vec = typename M::Vec;
    using T = typename E::Storage;
    constexpr int kBs = 16;
    constexpr int kSteps = kD / 32;
    constexpr int kDpl = kD == 64 ? 8 : 16;
    constexpr int kLpt = kD / kDpl;
    constexpr int kTpp = 64 / kLpt;
    constexpr int kPasses = kBs / kTpp;
    constexpr int kVWords = kDpl / 2;
    constexpr int kMfmas = 3 * kG <= 16 ? 1 : 2;
    constexpr int kTiles = kChunk / kBs;
    static_assert(kLpt == 8 && kTpp == 8 && kPasses == 2, "V lane layout");

    __shared__ std::uint32_t plan[kPlanRows + 1];
    __shared__ std::uint32_t scan[kThreads];
    __shared__ std::uint64_t pages[kTiles];
    __shared__ __attribute__((aligned(16))) std::uint16_t qsplit[3 * kG * kD];
    __shared__ __attribute__((aligned(16))) float probs[kWaves][kBs * kG];
    __shared__ float reduce[kWaves * 2 * kG * kD];
    __shared__ float wstats[kWaves][2 * kG];

    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int col = lane % 16, quad = lane / 16;
    const int tsub = lane / kLpt, slice = lane % kLpt;
    const std::uint32_t rows = p.num_rows;

    // ---- plan: plan[r] = number of chunks of rows < r (a zero-length row
    // still owns one chunk so its output is written).
    constexpr int kPer = kPlanRows / kThreads;
    std::uint32_t mine = 0;
    for (int i = 0; i < kPer; ++i) {
        const std::uint32_t r = tid * kPer + i;
        if (r < rows) {
            const std::uint64_t len = row_length(p, r);
            mine += len == 0 ? 1u : static_cast<std::uint32_t>((len + kChunk - 1) / kChunk);
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
                const std::uint64_t len = row_length(p, r);
                run += len == 0 ? 1u : static_cast<std::uint32_t>((len + kChunk - 1) / kChunk);
            }
        }
        if (tid == kThreads - 1) plan[rows] = scan[tid];
    }
    __syncthreads();
    const std::uint32_t total = plan[rows] * p.heads;

    const T* kc = static_cast<const T*>(p.key_cache);
    const T* vc = static_cast<const T*>(p.value_cache);
    const std::uint64_t head_stride = static_cast<std::uint64_t>(kBs) * kD;
    const std::uint64_t page_stride = head_stride * p.heads;
    // Lane offsets inside one page-head block [16 tokens][kD].
    const std::uint32_t k_lane = col * kD + quad * 8;
    const std::uint32_t v_lane = tsub * kD + slice * kDpl;
    float* my_probs = probs[wave];

    for (std::uint32_t item = blockIdx.x; item < total; item += gridDim.x) {
        const std::uint32_t kvh = item % p.heads;
        const std::uint32_t rc = item / p.heads;
        std::uint32_t lo = 0, hi = rows;  // plan[lo] <= rc < plan[hi]
        while (hi - lo > 1) {
            const std::uint32_t mid = (lo + hi) / 2;
            if (plan[mid] <= rc) lo = mid; else hi = mid;
        }
        const std::uint32_t row = lo;
        const std::uint32_t chunk = rc - plan[row];
        const std::uint64_t len = row_length(p, row);
        const std::uint64_t tok_begin = static_cast<std::uint64_t>(chunk) * kChunk;
        const std::uint32_t ntok =
            len > tok_begin ? static_cast<std::uint32_t>(len - tok_begin < kChunk ? len - tok_begin : kChunk) : 0;
        const std::uint32_t ntiles = (ntok + kBs - 1) / kBs;
        const std::uint64_t* table_row = p.table + (p.seq_lens ? row : 0) * p.width;
        const std::uint64_t first_page = tok_begin / kBs;
        for (std::uint32_t i = tid; i < ntiles; i += kThreads) {
            const std::uint64_t logical = first_page + i;
            const std::uint64_t id = logical < p.width ? table_row[logical] : kNoPage;
            pages[i] = id < p.num_blocks ? id : kNoPage;
        }
        const std::uint32_t qh0 = kvh * kG;
        for (int idx = tid; idx < kG * kD; idx += kThreads) {
            const int g = idx / kD, d = idx % kD;
            float rest;
            const float x = p.query[(static_cast<std::uint64_t>(row) * p.query_heads + qh0 + g) * kD + d] * p.scale_log2;
            qsplit[(0 * kG + g) * kD + d] = M::split(x, &rest);
            qsplit[(1 * kG + g) * kD + d] = M::split(rest, &rest);
            qsplit[(2 * kG + g) * kD + d] = M::split(rest, &rest);
        }
        __syncthreads();

        // B operands from the split table: column -> (split, head).
        Vec qb[kMfmas][kSteps];
#pragma unroll
        for (int m = 0; m < kMfmas; ++m) {
            int split = col / kG, g = col % kG;
            bool used = col < 3 * kG;
            if (kMfmas == 2 && m == 1) {
                split = 2;
                g = col;
                used = col < kG;
            }
#pragma unroll
            for (int kk = 0; kk < kSteps; ++kk) {
                const uint4 raw = used ? *reinterpret_cast<const uint4*>(qsplit + (split * kG + g) * kD + kk * 32 + quad * 8)
                                       : make_uint4(0, 0, 0, 0);
                qb[m][kk] = __builtin_bit_cast(Vec, raw);
            }
        }

        struct Tile {
            uint4 k[kSteps];
            uint4 v[kPasses][kVWords / 4];
        };
        auto load = [&](std::uint32_t t, Tile& b) {
            const std::uint64_t page = pages[t];
            if (page != kNoPage) {
                const T* kb = kc + page * page_stride + kvh * head_stride;
                const T* vb = vc + page * page_stride + kvh * head_stride;
#pragma unroll
                for (int kk = 0; kk < kSteps; ++kk) b.k[kk] = *reinterpret_cast<const uint4*>(kb + k_lane + kk * 32);
#pragma unroll
                for (int u = 0; u < kPasses; ++u)
#pragma unroll
                    for (int w = 0; w < kVWords / 4; ++w)
                        b.v[u][w] = *reinterpret_cast<const uint4*>(vb + v_lane + u * kTpp * kD + w * 8);
            } else {
#pragma unroll
                for (int kk = 0; kk < kSteps; ++kk) b.k[kk] = make_uint4(0, 0, 0, 0);
#pragma unroll
                for (int u = 0; u < kPasses; ++u)
#pragma unroll
                    for (int w = 0; w < kVWords / 4; ++w) b.v[u][w] = make_uint4(0, 0, 0, 0);
            }
        };

        float run_max = -INFINITY, run_sum = 0.0f;
        float acc[kG][kDpl];
#pragma unroll
        for (int g = 0; g < kG; ++g)
#pragma unroll
            for (int i = 0; i < kDpl; ++i) acc[g][i] = 0.0f;

        auto compute = [&](std::uint32_t t, Tile& b) {
            const std::uint32_t valid = pages[t] == kNoPage ? 0u
                                        : (ntok - t * kBs < kBs ? ntok - t * kBs : kBs);  // uniform
            f32x4_t s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kk = 0; kk < kSteps; ++kk) {
                const Vec a = __builtin_bit_cast(Vec, b.k[kk]);
                s0 = M::mma(a, qb[0][kk], s0);
                if constexpr (kMfmas == 2) s1 = M::mma(a, qb[1][kk], s1);
            }
            float sc[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if constexpr (kMfmas == 1) {
                    sc[r] = s0[r] + row_shl<kG>(s0[r]) + row_shl<2 * kG>(s0[r]);
                } else {
                    sc[r] = s0[r] + row_shl<kG>(s0[r]) + s1[r];
                }
            }
            if (valid < kBs) {  // partial or unreadable tile (uniform)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (static_cast<std::uint32_t>(quad * 4 + r) >= valid) sc[r] = -INFINITY;
                }
#pragma unroll
                for (int u = 0; u < kPasses; ++u) {
                    if (static_cast<std::uint32_t>(u * kTpp + tsub) >= valid) {
#pragma unroll
                        for (int w = 0; w < kVWords / 4; ++w) b.v[u][w] = make_uint4(0, 0, 0, 0);
                    }
                }
            }
            float tmax = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
            tmax = fmaxf(tmax, swizzle_xor16(tmax));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
            const float new_max = fmaxf(run_max, tmax);
            const float alpha = exp2_shifted(run_max, new_max);
            run_max = new_max;
            float psum = 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pr = exp2_shifted(sc[r], new_max);
                psum += pr;
                if (col < kG) my_probs[(quad * 4 + r) * kG + col] = pr;
            }
            run_sum = run_sum * alpha + psum;
#pragma unroll
            for (int g = 0; g < kG; ++g) {
                const float a_g = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), g));
                if (a_g != 1.0f) {
#pragma unroll
                    for (int i = 0; i < kDpl; ++i) acc[g][i] *= a_g;
                }
            }
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int u = 0; u < kPasses; ++u) {
                const std::uint32_t* words = reinterpret_cast<const std::uint32_t*>(b.v[u]);
                float v[kDpl];
                widen<E>(words, v, kDpl);
                float pw[kG];
#pragma unroll
                for (int g = 0; g < kG; ++g) pw[g] = my_probs[(u * kTpp + tsub) * kG + g];
#pragma unroll
                for (int g = 0; g < kG; ++g)
#pragma unroll
                    for (int i = 0; i < kDpl; ++i) acc[g][i] = fmaf(pw[g], v[i], acc[g][i]);
            }
            __builtin_amdgcn_wave_barrier();
        };

        Tile buf0, buf1;
        std::uint32_t t0 = wave;
        if (t0 < ntiles) load(t0, buf0);
        for (; t0 < ntiles; t0 += 2 * kWaves) {
            const std::uint32_t t1 = t0 + kWaves;
            if (t1 < ntiles) load(t1, buf1);
            compute(t0, buf0);
            if (t1 >= ntiles) break;
            if (t1 + kWaves < ntiles) load(t1 + kWaves, buf0);
            compute(t1, buf1);
        }

        // Wave totals, then the block combine through LDS.
        run_sum += swizzle_xor16(run_sum);
        run_sum += __shfl_xor(run_sum, 32);
        if (lane < kG) {
            wstats[wave][2 * lane] = run_max;
            wstats[wave][2 * lane + 1] = run_sum;
        }
#pragma unroll
        for (int g = 0; g < kG; ++g) {
#pragma unroll
            for (int i = 0; i < kDpl; ++i) {
                float a = acc[g][i];
                a += dpp<kRowRor8>(a);
                a += swizzle_xor16(a);
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

        const bool single = len <= kChunk || p.max_chunks <= 1;
        for (int idx = tid; idx < kG * kD; idx += kThreads) {
            const int g = idx / kD, d = idx % kD;
            float m = -INFINITY;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) m = fmaxf(m, wstats[w][2 * g]);
            float l = 0.0f, sum = 0.0f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float f = exp2_shifted(wstats[w][2 * g], m);
                l += wstats[w][2 * g + 1] * f;
                sum += (reduce[(w * 2) * kG * kD + idx] + reduce[(w * 2 + 1) * kG * kD + idx]) * f;
            }
            const std::uint64_t out_row = static_cast<std::uint64_t>(row) * p.query_heads + qh0 + g;
            if (single) {
                p.output[out_row * kD + d] = l > 0.0f ? sum / l : 0.0f;
            } else {
                const std::uint64_t slot = out_row * p.max_chunks + chunk;
                p.partial_acc[slot * kD + d] = sum;
                if (d == 0) {
                    p.partial_ml[2 * slot] = m;
                    p.partial_ml[2 * slot + 1] = l;
                }
            }
        }
        __syncthreads();  // LDS is reused by the next item
    }
}

// Combines the chunk partials of every (row, query head) with more than one
// chunk, in ascending chunk order.
__global__ __launch_bounds__(64) void paged_attention_combine_kernel(Params p, std::uint32_t head_dim) {
    const std::uint32_t row = p.row_base + blockIdx.x / p.query_heads;
    const std::uint32_t qh = blockIdx.x % p.query_heads;
    const std::uint64_t len = row_length(p, row);
    const std::uint64_t needed = (len + kChunk - 1) / kChunk;
    const std::uint32_t nchunks =
        needed < p.max_chunks ? static_cast<std::uint32_t>(needed) : p.max_chunks;
    if (nchunks <= 1) return;
    const std::uint64_t out_row = static_cast<std::uint64_t>(row) * p.query_heads + qh;
    const float* ml = p.partial_ml + out_row * p.max_chunks * 2;
    float m = -INFINITY;
    for (std::uint32_t c = 0; c < nchunks; ++c) m = fmaxf(m, ml[2 * c]);
    float l = 0.0f;
    for (std::uint32_t c = 0; c < nchunks; ++c) l += ml[2 * c + 1] * exp2_shifted(ml[2 * c], m);
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    for (std::uint32_t d = threadIdx.x; d < head_dim; d += 64) {
        float o = 0.0f;
        for (std::uint32_t c = 0; c < nchunks; ++c) {
            o = fmaf(p.partial_acc[(out_row * p.max_chunks + c) * head_dim + d],
                     exp2_shifted(ml[2 * c], m), o);
        }
        p.output[out_row * head_dim + d] = o * inv;
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
template <typename E, int kD, int kG>
int launch_split(Params p, std::uint64_t rows, std::uint64_t max_chunks, hipStream_t s) {
    const std::uint64_t rows_per_launch = 65535 / p.heads;
    for (std::uint64_t base = 0; base < rows; base += rows_per_launch) {
        const std::uint64_t n = rows - base < rows_per_launch ? rows - base : rows_per_launch;
        p.row_base = static_cast<std::uint32_t>(base);
        hipLaunchKernelGGL((paged_attention_split_kernel<E, kD, kG>),
                           dim3(static_cast<unsigned>(max_chunks), static_cast<unsigned>(n * p.heads)),
                           dim3(kThreads), 0, s, p);
        int status = launch_status("paged_attention_split_kernel");
        if (status != KVFLUX_OK) return status;
        if (max_chunks > 1) {
            hipLaunchKernelGGL(paged_attention_combine_kernel,
                               dim3(static_cast<unsigned>(n * p.query_heads)), dim3(64), 0, s, p,
                               static_cast<std::uint32_t>(kD));
            status = launch_status("paged_attention_combine_kernel");
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

// Persistent grid: every resident workgroup slot gets one workgroup.
template <typename E, int kD, int kG>
int launch_bs16(Params p, std::uint64_t max_chunks, hipStream_t s) {
    static int slots = 0;  // resident workgroups per device (queried once)
    if (slots == 0) {
        int device = 0, cus = 0, per_cu = 0;
        int status = hip_status(hipGetDevice(&device), "hipGetDevice");
        if (status == KVFLUX_OK)
            status = hip_status(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device),
                                "hipDeviceGetAttribute");
        if (status == KVFLUX_OK)
            status = hip_status(hipOccupancyMaxActiveBlocksPerMultiprocessor(
                                    &per_cu, paged_decode_bs16_kernel<E, kD, kG>, kThreads, 0),
                                "hipOccupancyMaxActiveBlocksPerMultiprocessor");
        if (status != KVFLUX_OK) return status;
        slots = cus * (per_cu > 0 ? per_cu : 1);
    }
    const std::uint64_t items = static_cast<std::uint64_t>(p.num_rows) * max_chunks * p.heads;
    const unsigned grid = static_cast<unsigned>(items < static_cast<std::uint64_t>(slots) ? items : slots);
    p.row_base = 0;
    hipLaunchKernelGGL((paged_decode_bs16_kernel<E, kD, kG>), dim3(grid), dim3(kThreads), 0, s, p);
    int status = launch_status("paged_decode_bs16_kernel");
    if (status != KVFLUX_OK) return status;
    if (max_chunks > 1) {
        for (std::uint64_t base = 0; base < p.num_rows; base += 0x7fffffffULL / p.query_heads) {
            const std::uint64_t n = p.num_rows - base < 0x7fffffffULL / p.query_heads
                                        ? p.num_rows - base : 0x7fffffffULL / p.query_heads;
            p.row_base = static_cast<std::uint32_t>(base);
            hipLaunchKernelGGL(paged_attention_combine_kernel, dim3(static_cast<unsigned>(n * p.query_heads)),
                               dim3(64), 0, s, p, static_cast<std::uint32_t>(kD));
            status = launch_status("paged_attention_combine_kernel");
            if (status != KVFLUX_OK) return status;
        }
    }
    return KVFLUX_OK;
}

template <typename E, int kD>
int dispatch_group(Params p, std::uint64_t rows, std::uint64_t group, std::uint64_t max_chunks,
                   hipStream_t s) {
    if constexpr (!std::is_same<E, F32>::value && (kD == 64 || kD == 128)) {
        if (p.block_size.divisor == 16 && rows <= kPlanRows) {
            switch (group) {
            case 1: return launch_bs16<E, kD, 1>(p, max_chunks, s);
            case 2: return launch_bs16<E, kD, 2>(p, max_chunks, s);
            case 4: return launch_bs16<E, kD, 4>(p, max_chunks, s);
            case 8:
                // D=128 with 8 heads per group needs 128 accumulators per
                // lane: the FP32 split kernel (8 dims per lane) fits better.
                if constexpr (kD == 64) return launch_bs16<E, kD, 8>(p, max_chunks, s);
                break;
            default: break;
            }
        }
    }
    switch (group) {
    case 1: return launch_split<E, kD, 1>(p, rows, max_chunks, s);
    case 2: return launch_split<E, kD, 2>(p, rows, max_chunks, s);
    case 4: return launch_split<E, kD, 4>(p, rows, max_chunks, s);
    case 8: return launch_split<E, kD, 8>(p, rows, max_chunks, s);
    default: return launch_generic<E>(p, rows, kD, s);
    }
}

template <typename E>
int dispatch(Params p, std::uint64_t rows, std::uint64_t head_dim, std::uint64_t group,
             std::uint64_t max_chunks, hipStream_t s) {
    switch (head_dim) {
    case 64: return dispatch_group<E, 64>(p, rows, group, max_chunks, s);
    case 128: return dispatch_group<E, 128>(p, rows, group, max_chunks, s);
    case 256:
        if (group <= 4) return dispatch_group<E, 256>(p, rows, group, max_chunks, s);
        return launch_generic<E>(p, rows, head_dim, s);
    default: return launch_generic<E>(p, rows, head_dim, s);
    }
}

bool uses_split(std::uint64_t head_dim, std::uint64_t group) {
    const bool g_ok = group == 1 || group == 2 || group == 4 || group == 8;
    if (head_dim == 64 || head_dim == 128) return g_ok;
    if (head_dim == 256) return g_ok && group <= 4;
    return false;
}

} // namespace
} // namespace kvflux_hip

using namespace kvflux_hip;

extern "C" int kvflux_paged_attention_workspace_size(uint64_t num_rows, uint64_t kv_len,
                                                     uint64_t num_kv_heads, uint64_t query_heads,
                                                     uint64_t block_size, uint64_t head_size,
                                                     size_t* bytes) {
    (void)block_size;
    if (!bytes) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "bytes is null");
    *bytes = 0;
    if (num_kv_heads == 0 || query_heads == 0 || query_heads % num_kv_heads != 0) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "invalid attention head counts");
    }
    if (!uses_split(head_size, query_heads / num_kv_heads)) return KVFLUX_OK;
    const std::uint64_t chunks = (kv_len + kChunk - 1) / kChunk;
    if (chunks <= 1) return KVFLUX_OK;
    const long double need = static_cast<long double>(num_rows) * query_heads * chunks *
                             (head_size + 2) * sizeof(float);
    if (need > static_cast<long double>(~std::size_t{0} / 2)) {
        return fail(KVFLUX_ERR_OVERFLOW, "attention workspace size overflow");
    }
    // Accumulators first, then (m, l) pairs; both 256-byte aligned.
    const std::uint64_t acc = num_rows * query_heads * chunks * head_size * sizeof(float);
    const std::uint64_t ml = num_rows * query_heads * chunks * 2 * sizeof(float);
    *bytes = ((acc + 255) & ~std::uint64_t{255}) + ((ml + 255) & ~std::uint64_t{255});
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
    std::size_t need = 0;
    int status = kvflux_paged_attention_workspace_size(num_rows, kv_len, num_kv_heads, query_heads,
                                                       block_size, head_size, &need);
    if (status != KVFLUX_OK) return status;
    if (need > 0 && (!workspace || workspace_bytes < need)) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged attention: workspace needs %zu bytes", need);
    }
    const std::uint64_t chunks = (kv_len + kChunk - 1) / kChunk;
    Params p{};
    p.key_cache = key_cache;
    p.value_cache = value_cache;
    p.num_blocks = num_blocks;
    p.heads = static_cast<std::uint32_t>(num_kv_heads);
    p.block_size = FastDiv(static_cast<std::uint32_t>(block_size));
    p.table = block_table;
    p.width = max_blocks_per_seq;
    p.seq_lens = seq_lens;
    p.kv_len = kv_len;
    p.num_rows = static_cast<std::uint32_t>(num_rows);
    p.query_heads = static_cast<std::uint32_t>(query_heads);
    p.query = query;
    p.output = output;
    p.max_chunks = static_cast<std::uint32_t>(chunks);
    p.scale_log2 = static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(head_size)));
    if (need > 0) {
        const std::uint64_t acc = num_rows * query_heads * chunks * head_size * sizeof(float);
        p.partial_acc = static_cast<float*>(workspace);
        p.partial_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                                ((acc + 255) & ~std::uint64_t{255}));
    }
    const hipStream_t s = as_stream(stream);
    switch (dtype) {
    case KVFLUX_DTYPE_BF16: return dispatch<Bf16>(p, num_rows, head_size, group, chunks, s);
    case KVFLUX_DTYPE_F16: return dispatch<F16>(p, num_rows, head_size, group, chunks, s);
    default: return dispatch<F32>(p, num_rows, head_size, group, chunks, s);
    }
}
