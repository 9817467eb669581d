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

template <typename E, int kD>
int dispatch_group(Params p, std::uint64_t rows, std::uint64_t group, std::uint64_t max_chunks,
                   hipStream_t s) {
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
