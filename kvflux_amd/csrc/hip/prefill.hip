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
    static constexpr std::uint32_t kOnes = 0x3f803f80u;  // two 1.0
    __device__ static std::uint32_t pack(float a, float b) {
        return __builtin_bit_cast(std::uint32_t, __builtin_convertvector(pf_f32x2_t{a, b}, pf_bf16x2_t));
    }
    __device__ static pf_f32x4_t mma(const Vec& a, const Vec& b, const pf_f32x4_t& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
struct PfF16 {
    using Vec = pf_f16x8_t;
    static constexpr std::uint32_t kOnes = 0x3c003c00u;  // two 1.0
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

constexpr int kPfThreads = 512;   // 8 wavefronts, two per SIMD
constexpr int kPfWaves = kPfThreads / 64;
constexpr int kPfRows = 256;      // rows per workgroup
constexpr int kPfNt = kPfRows / 16 / kPfWaves;  // 16-row blocks per wavefront
constexpr int kPfTile = 64;       // keys per LDS tile
constexpr int kPfTableMax = 2048; // page ids held in LDS (kv_len <= 2048 * block_size)
// Flag bit of a missing page in the LDS page list (ids are below 2^31): it is
// loaded from page 0 (never out of bounds) and its K and V staged as zeros.
constexpr std::uint32_t kPfMissing = 0x80000000u;

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
    // Page ids of the tiles; a missing page (past the table or kv_len, or an
    // id >= num_blocks) is loaded from page 0 and zeroed before it reaches LDS.
    bool missing = false;
    for (std::uint32_t i = tid; i < npages; i += kPfThreads) {
        const std::uint64_t id = i < p.table_len ? p.table[i] : p.num_blocks;
        const bool ok = id < p.num_blocks && (static_cast<std::uint64_t>(i) << p.bs_shift) < p.kv_len;
        pages[i] = ok ? static_cast<std::uint32_t>(id) : kPfMissing;
        missing |= !ok && (static_cast<std::uint64_t>(i) << p.bs_shift) < p.kv_len;
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
    // pages[] ready; uniform: some page inside kv_len is missing
    const bool table_gaps = __syncthreads_or(missing);

    // Tile staging: chunk id = tid + kPfThreads * i; row = id / kCpr, c = id % kCpr.
    // A tile starts on a page boundary (block_size divides 64), so a thread's
    // row sits at a fixed offset in its page, and its page is entry
    // tile * (64 / block_size) + row / block_size of pages[].
    const char* kc = static_cast<const char*>(p.key_cache);
    const char* vc = static_cast<const char*>(p.value_cache);
    const std::uint32_t page_bytes = (static_cast<std::uint32_t>(kRowBytes) << p.bs_shift) * p.heads;
    const std::uint32_t tile_pages_shift = 6 - p.bs_shift;
    std::uint32_t lane_bytes[kChunksPerThread], row_page[kChunksPerThread];
#pragma unroll
    for (int i = 0; i < kChunksPerThread; ++i) {
        const int id = tid + kPfThreads * i;
        const int row = id / kCpr, c = id % kCpr;
        row_page[i] = static_cast<std::uint32_t>(row) >> p.bs_shift;
        lane_bytes[i] = ((kvh << p.bs_shift) + (static_cast<std::uint32_t>(row) & ((1u << p.bs_shift) - 1))) *
                            kRowBytes + c * 16;
    }
    auto k_slot = [](int row, int c) {  // conflict-free for 16-row ds_read_b128
        return kCpr == 16 ? (c ^ (row & 15)) : (c ^ ((row >> 1) & 7));
    };
    auto v_slot = [](int row, int c) { return c ^ (kVSwz * (row & 7)); };
    struct Staged {
        uint4 k[kChunksPerThread], v[kChunksPerThread];
    };
    // Unconditional loads (straight-line code keeps the wait counts exact).
    auto fetch = [&](std::uint32_t tile, Staged& st) {
#pragma unroll
        for (int i = 0; i < kChunksPerThread; ++i) {
            const std::uint32_t page = pages[(tile << tile_pages_shift) + row_page[i]] & ~kPfMissing;
            const std::uint64_t off = static_cast<std::uint64_t>(page) * page_bytes + lane_bytes[i];
            st.k[i] = *reinterpret_cast<const uint4*>(kc + off);
            st.v[i] = *reinterpret_cast<const uint4*>(vc + off);
        }
    };
    auto stage = [&](std::uint32_t tile, const Staged& st) {
        char* kb = reinterpret_cast<char*>(ktile);
        char* vb = reinterpret_cast<char*>(vtile);
        // Keys at or past kv_len, or on a missing page, are staged as zeros
        // (finite V under a zero weight). Uniform test: only the last tile or
        // a table with gaps takes it. The loaded registers are only read
        // here, never overwritten, so no wait is needed for the other set.
        const bool fix = table_gaps || (tile + 1) * kPfTile > p.kv_len;
#pragma unroll
        for (int i = 0; i < kChunksPerThread; ++i) {
            const int id = tid + kPfThreads * i;
            const int row = id / kCpr, c = id % kCpr;
            uint4 k = st.k[i], v = st.v[i];
            if (fix) {
                const std::uint32_t key = tile * kPfTile + row;
                const std::uint32_t missing_bit = pages[(tile << tile_pages_shift) + row_page[i]] & kPfMissing;
                const std::uint32_t keep = ((key >= p.kv_len) | (missing_bit != 0)) ? 0u : ~0u;
                k = make_uint4(k.x & keep, k.y & keep, k.z & keep, k.w & keep);
                v = make_uint4(v.x & keep, v.y & keep, v.z & keep, v.w & keep);
            }
            *reinterpret_cast<uint4*>(kb + row * kRowBytes + k_slot(row, c) * 16) = k;
            *reinterpret_cast<uint4*>(vb + row * kRowBytes + v_slot(row, c) * 16) = v;
        }
    };
    // Transposing V^T reads: lane (q, s) addresses key row 4q + s/4 (+16 for
    // the second half of the operand), dims 16*dt + 4*(s%4). The swizzle
    // acts on bits 4..6 of the byte offset and dt on bits 5..7, so block dt
    // is v_read0 ^ (dt << 5); row offsets of whole tiles are immediates.
    std::uint32_t v_rd[kDt];
    {
        const int s = lane % 16, r = 4 * quad + s / 4;
        const int c = (4 * (s % 4)) / 8;
        const std::uint32_t v_read0 = r * kRowBytes + (v_slot(r, c) * 16) + (s % 2) * 8;
#pragma unroll
        for (int dt = 0; dt < kDt; ++dt) v_rd[dt] = v_read0 ^ (dt << 5);
    }
    // K A operand of lane (quad, col) for step kk: key row 16*m + col (the
    // K swizzle depends on the row only through col), 16-byte column
    // quad + 4*kk.
    std::uint32_t k_rd[kSteps];
#pragma unroll
    for (int kk = 0; kk < kSteps; ++kk) k_rd[kk] = col * kRowBytes + k_slot(col, quad + 4 * kk) * 16;

    pf_f32x4_t acc[kDt][kPfNt];
#pragma unroll
    for (int dt = 0; dt < kDt; ++dt)
#pragma unroll
        for (int n = 0; n < kPfNt; ++n) acc[dt][n] = pf_f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // Per row block: the row sums of the rounded weights (an MFMA against a
    // matrix of ones, so every entry holds its column's sum) and minus the
    // row's reference point, broadcast: the S^T accumulators start from it,
    // so the scores arrive already shifted.
    pf_f32x4_t lsum[kPfNt], nref[kPfNt];
#pragma unroll
    for (int n = 0; n < kPfNt; ++n) {
        lsum[n] = pf_f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        nref[n] = pf_f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
    bool have_ref = false;  // uniform: false until the first half-tile sets every row's reference
    const Vec ones = __builtin_bit_cast(Vec, make_uint4(M::kOnes, M::kOnes, M::kOnes, M::kOnes));
    const std::uint32_t min_limit = past + t0;  // smallest causal limit of the block

    // Tiles alternate between two register sets, loaded two tiles ahead.
    auto compute_tile = [&](std::uint32_t tile) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const std::uint32_t k0 = tile * kPfTile + 32 * h;
            if (k0 > last_key) break;  // uniform
            // S^T - ref for keys k0 .. k0+31: two 16-key tiles x the row blocks.
            pf_f32x4_t s[2][kPfNt];
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                Vec a[kSteps];
#pragma unroll
                for (int kk = 0; kk < kSteps; ++kk) {
                    a[kk] = __builtin_bit_cast(
                        Vec, *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(ktile) +
                                                             (32 * h + 16 * kt) * kRowBytes + k_rd[kk]));
                }
#pragma unroll
                for (int n = 0; n < kPfNt; ++n) {
                    pf_f32x4_t x = nref[n];
#pragma unroll
                    for (int kk = 0; kk < kSteps; ++kk) x = M::mma(a[kk], qb_op[n][kk], x);
                    s[kt][n] = x;
                }
            }
            if (k0 + 31 > min_limit) {  // uniform; keys past the row's causal limit
#pragma unroll
                for (int n = 0; n < kPfNt; ++n) {
                    const std::int32_t room = static_cast<std::int32_t>(past + row_token[n] - k0 - 4 * quad);
#pragma unroll
                    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                        for (int r = 0; r < 4; ++r) s[kt][n][r] = 16 * kt + r > room ? -INFINITY : s[kt][n][r];
                }
            }
            // Row maxima relative to the reference (equal in the four quads of a column).
            float tmax[kPfNt];
            bool grow = !have_ref;
#pragma unroll
            for (int n = 0; n < kPfNt; ++n) {
                tmax[n] = max_across_quads(max3(max3(s[0][n][0], s[0][n][1], s[0][n][2]),
                                                max3(s[0][n][3], s[1][n][0], s[1][n][1]),
                                                max3(s[1][n][2], s[1][n][3], -INFINITY)));
                grow |= tmax[n] > kLazy;
            }
            // Rare, wave-uniform: move the reference of the rows whose maximum
            // exceeds it by more than 2^kLazy (all rows on the first half-tile)
            // and rescale what they have accumulated.
            if (__builtin_expect(__builtin_amdgcn_ballot_w64(grow) != 0, 0)) {
#pragma unroll
                for (int n = 0; n < kPfNt; ++n) {
                    const float shift = !have_ref || tmax[n] > kLazy ? tmax[n] : 0.0f;
                    // min(.., 0): on the first half-tile the accumulators are still zero
                    const float alpha = __builtin_amdgcn_exp2f(fminf(-shift, 0.0f));
                    nref[n] -= shift;
                    lsum[n] *= alpha;
#pragma unroll
                    for (int kt = 0; kt < 2; ++kt) s[kt][n] -= shift;
#pragma unroll
                    for (int dt = 0; dt < kDt; ++dt) acc[dt][n] *= alpha;
                }
                have_ref = true;
            }
            Vec pb[kPfNt];
#pragma unroll
            for (int n = 0; n < kPfNt; ++n) {
                std::uint32_t w[4];
#pragma unroll
                for (int kt = 0; kt < 2; ++kt) {
                    w[2 * kt] = M::pack(__builtin_amdgcn_exp2f(s[kt][n][0]), __builtin_amdgcn_exp2f(s[kt][n][1]));
                    w[2 * kt + 1] = M::pack(__builtin_amdgcn_exp2f(s[kt][n][2]), __builtin_amdgcn_exp2f(s[kt][n][3]));
                }
                pb[n] = __builtin_bit_cast(Vec, make_uint4(w[0], w[1], w[2], w[3]));
            }
            // O^T += V^T P^T for the 32 keys of this half; l += 1 P^T.
            const auto* vbase = (__attribute__((address_space(3))) char*)(
                (__attribute__((address_space(3))) std::uint16_t*)vtile);
#pragma unroll
            for (int dt = 0; dt < kDt; ++dt) {
                const std::uint32_t off = v_rd[dt] + 32 * h * kRowBytes;
                const pf_i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((pf_lds_i16x4_t*)(vbase + off));
                const pf_i16x4_t hi =
                    __builtin_amdgcn_ds_read_tr16_b64_v4i16((pf_lds_i16x4_t*)(vbase + off + 16 * kRowBytes));
                const Vec a = __builtin_bit_cast(Vec, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
                for (int n = 0; n < kPfNt; ++n) acc[dt][n] = M::mma(a, pb[n], acc[dt][n]);
            }
#pragma unroll
            for (int n = 0; n < kPfNt; ++n) lsum[n] = M::mma(ones, pb[n], lsum[n]);
        }
    };
    // Every fetch is issued, past the end as a reload of the last tile, so
    // the loads form one in-order stream and each stage() waits only for the
    // set it writes (the other set stays in flight).
    const std::uint32_t last_tile = ntiles - 1;
    auto clamp_tile = [last_tile](std::uint32_t t) { return t < last_tile ? t : last_tile; };
    Staged set0, set1;
    fetch(0, set0);
    fetch(clamp_tile(1), set1);
    for (std::uint32_t tile = 0; tile < ntiles; tile += 2) {
        stage(tile, set0);
        __syncthreads();
        fetch(clamp_tile(tile + 2), set0);
        compute_tile(tile);
        __syncthreads();  // the tile is consumed before the next stage()
        if (tile + 1 >= ntiles) break;
        stage(tile + 1, set1);
        __syncthreads();
        fetch(clamp_tile(tile + 3), set1);
        compute_tile(tile + 1);
        __syncthreads();
    }

    // O = O^T / l.
#pragma unroll
    for (int n = 0; n < kPfNt; ++n) {
        const float l = lsum[n][0];
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
        num_blocks > 0x7fffffffULL || num_kv_heads > 65535 || kv_len > 0xffffffffULL ||
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
