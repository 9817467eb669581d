// Causal paged prefill on MFMA (gfx950): BF16/FP16 caches, head_size 64/128.
//
// One workgroup (8 wavefronts, two per SIMD) owns one kv head and a block of 256 rows,
// a row being a (query token, query head) pair of that kv head's group:
// 256 / G tokens x G heads. Wavefront w owns row blocks 2w, 2w+1 of 16 rows
// (row block b = head b % G, tokens 16 * (b / G) ..). Keys stream through
// LDS in tiles of 64 (K and V, staged through registers so the next tile's
// loads overlap this tile's MFMAs), processed as two halves of 32 keys:
//   S^T = K Q^T    v_mfma_f32_16x16x32 (A = K rows from LDS, B = Q rows held
//                  in registers, rounded to the cache dtype with the
//                  softmax scale folded in)
//   online softmax per row (reference point moved only when a score exceeds
//                  it by 2^8), weights rounded to the cache dtype
//   O^T += V^T P^T v_mfma_f32_16x16x32 (A = V^T through ds_read_b64_tr_b16,
//                  B = the weights exactly as the S^T output lanes hold them)
// The S^T output layout (lane (q, c) holds keys 4q..4q+3 of row c) is the
// P^T operand of the second product once keys are ordered as
// {4q..4q+3, 16+4q..16+4q+3} per 32-key step; V^T is read in that order.
#include "common.h"

#include <cmath>
#include <type_traits>

namespace kvflux_hip {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 pf_bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 pf_f16x8_t;
typedef __attribute__((ext_vector_type(4))) float pf_f32x4_t;
typedef short pf_i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) pf_i16x4_t pf_lds_i16x4_t;

typedef __attribute__((ext_vector_type(2))) float pf_f32x2_t;
typedef __attribute__((ext_vector_type(2))) __bf16 pf_bf16x2_t;
typedef __attribute__((ext_vector_type(2))) _Float16 pf_f16x2_t;

// pack(a, b): a in the low half, b in the high half, each rounded to nearest
// even (one v_cvt_pk_{bf16,f16}_f32).
struct PfBf16 {
    using Vec = pf_bf16x8_t;
    __device__ static std::uint32_t pack(float a, float b) {
        return __builtin_bit_cast(std::uint32_t, __builtin_convertvector(pf_f32x2_t{a, b}, pf_bf16x2_t));
    }
    __device__ static pf_f32x4_t mma(const Vec& a, const Vec& b, const pf_f32x4_t& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
struct PfF16 {
    using Vec = pf_f16x8_t;
    __device__ static std::uint32_t pack(float a, float b) {
        return __builtin_bit_cast(std::uint32_t, __builtin_convertvector(pf_f32x2_t{a, b}, pf_f16x2_t));
    }
    __device__ static pf_f32x4_t mma(const Vec& a, const Vec& b, const pf_f32x4_t& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

// NaN-propagating maximum of three (one v_maximum3_f32).
__device__ inline float max3(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}
// Maximum over the four lanes l, l^16, l^32, l^48 (the four quads of a
// column) with two cross-row lane swaps, no LDS round trip.
__device__ inline float max_across_quads(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __builtin_elementwise_maximum(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __builtin_elementwise_maximum(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ inline float sum_across_quads(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

constexpr int kPfThreads = 512;   // 8 wavefronts, two per SIMD
constexpr int kPfWaves = kPfThreads / 64;
constexpr int kPfRows = 256;      // rows per workgroup
constexpr int kPfNt = kPfRows / 16 / kPfWaves;  // 16-row blocks per wavefront
constexpr int kPfTile = 64;       // keys per LDS tile
constexpr int kPfTableMax = 2048; // page ids held in LDS (kv_len <= 2048 * block_size)
// Marks a missing page (table shorter than the tile, or an id >= num_blocks):
// its K and V read as zeros.
constexpr std::uint32_t kPfNoPage = 0xffffffffu;

struct PrefillParams {
    const void* key_cache;
    const void* value_cache;
    std::uint64_t num_blocks;
    std::uint32_t heads;      // kv heads
    std::uint32_t bs_shift;   // log2(block_size)
    const std::uint64_t* table;
    std::uint32_t table_len;
    std::uint32_t kv_len;
    std::uint32_t tq;         // query tokens (the last tq of kv_len)
    std::uint32_t query_heads;
    std::uint32_t qblocks;    // ceil(tq / tokens per workgroup)
    const float* query;       // [tq][query_heads][D]
    float* output;            // [tq][query_heads][D]
    float scale_log2;         // log2(e) / sqrt(D)
};

template <typename E, int kD, int kG>
__global__ __launch_bounds__(kPfThreads) void paged_prefill_kernel(PrefillParams p) {
    using M = E;
    using Vec = typename M::Vec;
    constexpr int kSteps = kD / 32;            // K-dim steps of S^T
    constexpr int kDt = kD / 16;               // dim blocks of O^T
    constexpr int kCpr = kD / 8;               // 16-byte chunks per key row
    constexpr int kRowBytes = kD * 2;
    constexpr int kTileChunks = kPfTile * kCpr;
    constexpr int kChunksPerThread = kTileChunks / kPfThreads;
    constexpr int kTok = kPfRows / kG;         // query tokens per workgroup
    constexpr int kVSwz = kCpr / 8;            // V slot swizzle multiplier
    constexpr float kLazy = 8.0f;
    static_assert(kChunksPerThread >= 1 && kTileChunks % kPfThreads == 0, "tile split");

    __shared__ __attribute__((aligned(16))) std::uint16_t ktile[kPfTile * kD];
    __shared__ __attribute__((aligned(16))) std::uint16_t vtile[kPfTile * kD];
    __shared__ std::uint32_t pages[kPfTableMax];

    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int col = lane % 16, quad = lane / 16;
    // Heaviest query blocks (most keys) first.
    const std::uint32_t kvh = blockIdx.x % p.heads;
    const std::uint32_t qb = p.qblocks - 1 - blockIdx.x / p.heads;
    const std::uint32_t t0 = qb * kTok;
    const std::uint32_t t_end = t0 + kTok < p.tq ? t0 + kTok : p.tq;
    const std::uint32_t past = p.kv_len - p.tq;  // keys before the first query
    const std::uint32_t last_key = past + t_end - 1;
    const std::uint32_t ntiles = last_key / kPfTile + 1;
    const std::uint32_t npages = ((ntiles * kPfTile - 1) >> p.bs_shift) + 1;
    for (std::uint32_t i = tid; i < npages; i += kPfThreads) {
        const std::uint64_t id = i < p.table_len ? p.table[i] : kPfNoPage;
        pages[i] = id < p.num_blocks ? static_cast<std::uint32_t>(id) : kPfNoPage;  // never dereferenced
    }

    // Q rows of this wave: B operands [row block][K step], already scaled.
    Vec qb_op[kPfNt][kSteps];
    std::uint32_t row_token[kPfNt];
#pragma unroll
    for (int n = 0; n < kPfNt; ++n) {
        const int b = wave * kPfNt + n;
        const int g = b % kG;
        const std::uint32_t token = t0 + 16 * (b / kG) + col;
        row_token[n] = token;
        const std::uint32_t tq_safe = token < p.tq ? token : p.tq - 1;
        const float* src = p.query + (static_cast<std::uint64_t>(tq_safe) * p.query_heads + kvh * kG + g) * kD;
#pragma unroll
        for (int kk = 0; kk < kSteps; ++kk) {
            const float4 lo = *reinterpret_cast<const float4*>(src + kk * 32 + quad * 8);
            const float4 hi = *reinterpret_cast<const float4*>(src + kk * 32 + quad * 8 + 4);
            const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            std::uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                w[e] = M::pack(v[2 * e] * p.scale_log2, v[2 * e + 1] * p.scale_log2);
            }
            qb_op[n][kk] = __builtin_bit_cast(Vec, make_uint4(w[0], w[1], w[2], w[3]));
        }
    }
    __syncthreads();  // pages[] ready

    // Tile staging: chunk id = tid + kPfThreads * i; row = id / kCpr, c = id % kCpr.
    const std::uint16_t* kc = static_cast<const std::uint16_t*>(p.key_cache);
    const std::uint16_t* vc = static_cast<const std::uint16_t*>(p.value_cache);
    const std::uint64_t head_stride = static_cast<std::uint64_t>(kD) << p.bs_shift;
    const std::uint64_t page_stride = head_stride * p.heads;
    const std::uint32_t bs_mask = (1u << p.bs_shift) - 1;
    auto k_slot = [](int row, int c) {  // conflict-free for 16-row ds_read_b128
        return kCpr == 16 ? (c ^ (row & 15)) : (c ^ ((row >> 1) & 7));
    };
    auto v_slot = [](int row, int c) { return c ^ (kVSwz * (row & 7)); };
    struct Staged {
        uint4 k[kChunksPerThread], v[kChunksPerThread];
    };
    auto fetch = [&](std::uint32_t tile, Staged& st) {
#pragma unroll
        for (int i = 0; i < kChunksPerThread; ++i) {
            const int id = tid + kPfThreads * i;
            const int row = id / kCpr, c = id % kCpr;
            const std::uint32_t key = tile * kPfTile + row;
            const std::uint32_t page = key < p.kv_len ? pages[key >> p.bs_shift] : kPfNoPage;
            if (page != kPfNoPage) {
                const std::uint64_t off = static_cast<std::uint64_t>(page) * page_stride +
                                          kvh * head_stride + static_cast<std::uint64_t>(key & bs_mask) * kD + c * 8;
                st.k[i] = *reinterpret_cast<const uint4*>(kc + off);
                st.v[i] = *reinterpret_cast<const uint4*>(vc + off);
            } else {
                st.k[i] = make_uint4(0, 0, 0, 0);
                st.v[i] = make_uint4(0, 0, 0, 0);
            }
        }
    };
    auto stage = [&](const Staged& st) {
        char* kb = reinterpret_cast<char*>(ktile);
        char* vb = reinterpret_cast<char*>(vtile);
#pragma unroll
        for (int i = 0; i < kChunksPerThread; ++i) {
            const int id = tid + kPfThreads * i;
            const int row = id / kCpr, c = id % kCpr;
            *reinterpret_cast<uint4*>(kb + row * kRowBytes + k_slot(row, c) * 16) = st.k[i];
            *reinterpret_cast<uint4*>(vb + row * kRowBytes + v_slot(row, c) * 16) = st.v[i];
        }
    };
    // Transposing V^T reads: lane (q, s) addresses key row 4q + s/4 (+16 for
    // the second half of the operand), dims 16*dt + 4*(s%4).
    std::uint32_t v_read0;
    {
        const int s = lane % 16, r = 4 * quad + s / 4;
        const int c = (4 * (s % 4)) / 8;
        v_read0 = r * kRowBytes + (v_slot(r, c) * 16) + (s % 2) * 8;
    }

    pf_f32x4_t acc[kDt][kPfNt];
#pragma unroll
    for (int dt = 0; dt < kDt; ++dt)
#pragma unroll
        for (int n = 0; n < kPfNt; ++n) acc[dt][n] = pf_f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float run_max[kPfNt], run_sum[kPfNt];
#pragma unroll
    for (int n = 0; n < kPfNt; ++n) {
        run_max[n] = -INFINITY;
        run_sum[n] = 0.0f;
    }
    const std::uint32_t min_limit = past + t0;  // smallest causal limit of the block

    // Tiles alternate between two register sets, loaded two tiles ahead.
    auto compute_tile = [&](std::uint32_t tile) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const std::uint32_t k0 = tile * kPfTile + 32 * h;
            if (k0 > last_key) break;  // uniform
            // S^T for keys k0 .. k0+31: two 16-key tiles x 4 row blocks.
            pf_f32x4_t s[2][kPfNt];
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                const int row = 32 * h + 16 * kt + col;
                Vec a[kSteps];
#pragma unroll
                for (int kk = 0; kk < kSteps; ++kk) {
                    const int c = quad + 4 * kk;
                    a[kk] = __builtin_bit_cast(
                        Vec, *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(ktile) + row * kRowBytes +
                                                             k_slot(row, c) * 16));
                }
#pragma unroll
                for (int n = 0; n < kPfNt; ++n) {
                    pf_f32x4_t x = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int kk = 0; kk < kSteps; ++kk) x = M::mma(a[kk], qb_op[n][kk], x);
                    s[kt][n] = x;
                }
            }
            const bool edge = k0 + 31 > min_limit;  // uniform: causal mask needed
            Vec pb[kPfNt];
#pragma unroll
            for (int n = 0; n < kPfNt; ++n) {
                if (edge) {  // keys past the row's causal limit (select, no branch)
                    const std::int32_t room = static_cast<std::int32_t>(past + row_token[n] - k0 - 4 * quad);
#pragma unroll
                    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                        for (int r = 0; r < 4; ++r) s[kt][n][r] = 16 * kt + r > room ? -INFINITY : s[kt][n][r];
                }
                float tmax = max3(max3(s[0][n][0], s[0][n][1], s[0][n][2]), max3(s[0][n][3], s[1][n][0], s[1][n][1]),
                                  max3(s[1][n][2], s[1][n][3], -INFINITY));
                tmax = max_across_quads(tmax);
                const bool grow = tmax > run_max[n] + kLazy;
                const float old = run_max[n];
                if (grow) run_max[n] = tmax;
                const float ref = run_max[n] == -INFINITY ? 0.0f : run_max[n];
                if (grow && old != -INFINITY) {
                    const float alpha = __builtin_amdgcn_exp2f(old - ref);
                    run_sum[n] *= alpha;
#pragma unroll
                    for (int dt = 0; dt < kDt; ++dt) acc[dt][n] *= alpha;
                }
                std::uint32_t w[4];
                float psum = 0.0f;
#pragma unroll
                for (int kt = 0; kt < 2; ++kt) {
                    float e[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        e[r] = __builtin_amdgcn_exp2f(s[kt][n][r] - ref);
                        psum += e[r];
                    }
                    w[2 * kt] = M::pack(e[0], e[1]);
                    w[2 * kt + 1] = M::pack(e[2], e[3]);
                }
                run_sum[n] += psum;
                pb[n] = __builtin_bit_cast(Vec, make_uint4(w[0], w[1], w[2], w[3]));
            }
            // O^T += V^T P^T for the 32 keys of this half.
            const auto* vbase = (__attribute__((address_space(3))) char*)(
                (__attribute__((address_space(3))) std::uint16_t*)vtile);
#pragma unroll
            for (int dt = 0; dt < kDt; ++dt) {
                const std::uint32_t off = (v_read0 + 32 * h * kRowBytes) ^ (dt << 5);
                const pf_i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((pf_lds_i16x4_t*)(vbase + off));
                const pf_i16x4_t hi =
                    __builtin_amdgcn_ds_read_tr16_b64_v4i16((pf_lds_i16x4_t*)(vbase + off + 16 * kRowBytes));
                const Vec a = __builtin_bit_cast(Vec, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
                for (int n = 0; n < kPfNt; ++n) acc[dt][n] = M::mma(a, pb[n], acc[dt][n]);
            }
        }
    };
    Staged set0, set1;
    fetch(0, set0);
    if (ntiles > 1) fetch(1, set1);
    for (std::uint32_t tile = 0; tile < ntiles; tile += 2) {
        stage(set0);
        __syncthreads();
        if (tile + 2 < ntiles) fetch(tile + 2, set0);
        compute_tile(tile);
        __syncthreads();  // the tile is consumed before the next stage()
        if (tile + 1 >= ntiles) break;
        stage(set1);
        __syncthreads();
        if (tile + 3 < ntiles) fetch(tile + 3, set1);
        compute_tile(tile + 1);
        __syncthreads();
    }

    // Row sums across the four quads, then O = O^T / l.
#pragma unroll
    for (int n = 0; n < kPfNt; ++n) {
        const float l = sum_across_quads(run_sum[n]);
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        const int b = wave * kPfNt + n;
        const int g = b % kG;
        const std::uint32_t token = row_token[n];
        if (token < t_end) {
            float* dst = p.output + (static_cast<std::uint64_t>(token) * p.query_heads + kvh * kG + g) * kD;
#pragma unroll
            for (int dt = 0; dt < kDt; ++dt) {
                *reinterpret_cast<float4*>(dst + 16 * dt + 4 * quad) =
                    make_float4(acc[dt][n][0] * inv, acc[dt][n][1] * inv, acc[dt][n][2] * inv, acc[dt][n][3] * inv);
            }
        }
    }
}

template <typename E, int kD>
int launch_prefill_group(const PrefillParams& p, std::uint32_t group, hipStream_t s) {
    const unsigned grid_of[9] = {0, kPfRows / 1, kPfRows / 2, 0, kPfRows / 4, 0, 0, 0, kPfRows / 8};
    PrefillParams q = p;
    q.qblocks = (p.tq + grid_of[group] - 1) / grid_of[group];
    const dim3 grid(q.qblocks * p.heads);
    switch (group) {
    case 1: hipLaunchKernelGGL((paged_prefill_kernel<E, kD, 1>), grid, dim3(kPfThreads), 0, s, q); break;
    case 2: hipLaunchKernelGGL((paged_prefill_kernel<E, kD, 2>), grid, dim3(kPfThreads), 0, s, q); break;
    case 4: hipLaunchKernelGGL((paged_prefill_kernel<E, kD, 4>), grid, dim3(kPfThreads), 0, s, q); break;
    default: hipLaunchKernelGGL((paged_prefill_kernel<E, kD, 8>), grid, dim3(kPfThreads), 0, s, q); break;
    }
    return launch_status("paged_prefill_kernel");
}

} // namespace
} // namespace kvflux_hip

using namespace kvflux_hip;

extern "C" int kvflux_paged_prefill(const void* key_cache, const void* value_cache, uint64_t num_blocks,
                                    uint64_t num_kv_heads, uint64_t block_size, uint64_t head_size, int dtype,
                                    const uint64_t* block_table, uint64_t num_table_blocks, uint64_t kv_len,
                                    uint64_t query_tokens, uint64_t query_heads, const float* query,
                                    float* output, void* stream) {
    if (query_tokens == 0) return KVFLUX_OK;
    if (dtype_bytes(dtype) == 0) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
    if (!key_cache || !value_cache || !block_table || !query || !output) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged prefill: null pointer");
    }
    if (num_blocks == 0 || num_kv_heads == 0 || block_size == 0 || head_size == 0 || query_heads == 0 ||
        query_heads % num_kv_heads != 0) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged prefill: invalid shape");
    }
    if (query_tokens > kv_len) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged prefill: more queries than tokens");
    if (num_table_blocks * block_size < kv_len) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged prefill: block table shorter than kv_len");
    }
    const std::uint64_t group = query_heads / num_kv_heads;
    if (dtype == KVFLUX_DTYPE_F32 || (head_size != 64 && head_size != 128) || !is_pow2(block_size) ||
        block_size > 64 || (group != 1 && group != 2 && group != 4 && group != 8) ||
        num_blocks >= 0xffffffffULL || num_kv_heads > 65535 || kv_len > 0xffffffffULL ||
        query_heads > 0xffffffffULL) {
        return fail(KVFLUX_ERR_UNSUPPORTED, "paged prefill: shape not handled by the MFMA kernel");
    }
    const std::uint64_t pages_needed = (((kv_len + kPfTile - 1) / kPfTile) * kPfTile + block_size - 1) / block_size;
    if (pages_needed > kPfTableMax) {
        return fail(KVFLUX_ERR_UNSUPPORTED, "paged prefill: kv_len above %llu tokens",
                    static_cast<unsigned long long>(kPfTableMax / ((kPfTile + block_size - 1) / block_size) *
                                                    kPfTile));
    }
    PrefillParams p{};
    p.key_cache = key_cache;
    p.value_cache = value_cache;
    p.num_blocks = num_blocks;
    p.heads = static_cast<std::uint32_t>(num_kv_heads);
    std::uint32_t shift = 0;
    while ((std::uint64_t{1} << shift) < block_size) ++shift;
    p.bs_shift = shift;
    p.table = block_table;
    p.table_len = static_cast<std::uint32_t>(num_table_blocks < kPfTableMax ? num_table_blocks : kPfTableMax);
    p.kv_len = static_cast<std::uint32_t>(kv_len);
    p.tq = static_cast<std::uint32_t>(query_tokens);
    p.query_heads = static_cast<std::uint32_t>(query_heads);
    p.query = query;
    p.output = output;
    p.scale_log2 = static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(head_size)));
    const hipStream_t s = as_stream(stream);
    const std::uint32_t g = static_cast<std::uint32_t>(group);
    if (dtype == KVFLUX_DTYPE_BF16) {
        return head_size == 64 ? launch_prefill_group<PfBf16, 64>(p, g, s) : launch_prefill_group<PfBf16, 128>(p, g, s);
    }
    return head_size == 64 ? launch_prefill_group<PfF16, 64>(p, g, s) : launch_prefill_group<PfF16, 128>(p, g, s);
}
