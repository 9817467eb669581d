// Causal paged prefill on MFMA (gfx950): BF16/FP16 caches, head_size 64/128/256,
// and FP32 caches, head_size 64/128 (v_mfma_f32_16x16x4_f32, see PfF32).
//
// One workgroup (8 wavefronts, two per SIMD) owns one kv head and 16 * R rows
// (R = 8 * pf_blocks row blocks of 16: 32 at head_size 64, 16 at 128, 8 at
// 256 and in the exact and FP32 variants), a row being a (query token, query
// head) pair of the G query heads
// of that kv head: row r is head r % G of token r / G, so a workgroup takes
// floor(16 * R / G) tokens of every head and at most G - 1 rows idle (a group
// above 16 * R runs as passes over sub-groups of heads). Wavefront w owns row
// blocks R/8 * w .. (rows 16 b .. 16 b + 15). A call that would not fill the GPU (short query
// blocks against a long prefix) may spread each workgroup's keys over several
// workgroups, merged by paged_prefill_combine_kernel. Keys stream through
// LDS in tiles of 64, double-buffered: K and V go from global memory straight
// into LDS (global_load_lds_dwordx4, no staging registers and no LDS write
// instructions), the next tile's loads in flight while this tile is computed
// (1.36 against 1.44 ms for 8 x 4096 tokens, 32/8 heads, D = 128 on MI355X,
// where the LDS issue rate, about one instruction per 4.5 clocks per CU, is
// a limit). Each tile is processed as two halves of 32 keys:
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
// even (one v_cvt_pk_{bf16,f16}_f32). split3(a, b): the same pair as three
// 16-bit parts whose sum is a and b (each part the rounded remainder of the
// ones before; the differences are exact in FP32), so an MFMA over the three
// parts against 16-bit cache values forms FP32-exact products.
struct PfBf16 {
    using Vec = pf_bf16x8_t;
    // Weights enter the split scaled by kWeightScale (undone exactly in the
    // epilogue); the running reference moves once a score passes it by
    // 2^kLazyLog2, so weights stay <= 2^kLazyLog2.
    static constexpr float kWeightScale = 1.0f;
    static constexpr float kLazyLog2 = 8.0f;
    static constexpr bool kExact = false;
    static constexpr bool kF32 = false;
    static constexpr std::uint32_t kOnes = 0x3f803f80u;  // two 1.0
    __device__ static std::uint32_t pack(float a, float b) {
        return __builtin_bit_cast(std::uint32_t, __builtin_convertvector(pf_f32x2_t{a, b}, pf_bf16x2_t));
    }
    __device__ static void split3(float a, float b, std::uint32_t (&w)[3]) {
        pf_f32x2_t x{a, b};
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const pf_bf16x2_t h = __builtin_convertvector(x, pf_bf16x2_t);
            w[i] = __builtin_bit_cast(std::uint32_t, h);
            x -= __builtin_convertvector(h, pf_f32x2_t);
        }
    }
    __device__ static pf_f32x4_t mma(const Vec& a, const Vec& b, const pf_f32x4_t& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
struct PfF16 {
    using Vec = pf_f16x8_t;
    static constexpr float kWeightScale = 1.0f;
    static constexpr float kLazyLog2 = 8.0f;
    static constexpr bool kExact = false;
    static constexpr bool kF32 = false;
    static constexpr std::uint32_t kOnes = 0x3c003c00u;  // two 1.0
    __device__ static std::uint32_t pack(float a, float b) {
        return __builtin_bit_cast(std::uint32_t, __builtin_convertvector(pf_f32x2_t{a, b}, pf_f16x2_t));
    }
    __device__ static void split3(float a, float b, std::uint32_t (&w)[3]) {
        pf_f32x2_t x{a, b};
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const pf_f16x2_t h = __builtin_convertvector(x, pf_f16x2_t);
            w[i] = __builtin_bit_cast(std::uint32_t, h);
            x -= __builtin_convertvector(h, pf_f32x2_t);
        }
    }
    __device__ static pf_f32x4_t mma(const Vec& a, const Vec& b, const pf_f32x4_t& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};
// The exact variants: Q and the softmax weights enter the MFMAs as three
// 16-bit parts each (FP32-exact products, FP32 accumulation), the row sums
// are FP32 sums of the weights, and a wavefront holds one row block.
struct PfBf16Exact : PfBf16 {
    static constexpr bool kExact = true;
};
// FP16's exponent stops at 2^-24: an unscaled weight below that would
// vanish from the numerator while still counting in the FP32 row sum. The
// FP16 exact variant therefore keeps every weight <= 1 (the reference moves
// with every new row maximum) and splits 2^15 times the weight (<= 32768, in
// range): a leading part loses bits to FP16's subnormals only below 2^-29
// of the row maximum and vanishes only below 2^-39, where 2^15 such keys
// together weigh under 2^-24 of the row; the epilogue multiplies by 2^-15
// (exact).
struct PfF16Exact : PfF16 {
    static constexpr bool kExact = true;
    static constexpr float kWeightScale = 32768.0f;
    static constexpr float kLazyLog2 = 0.0f;
};
// FP32 caches: K, V, Q and the weights enter v_mfma_f32_16x16x4_f32 as they
// are (exact products, FP32 accumulation), with the exact variants' FP32 row
// sums and one row block per wavefront. Vec only sizes the 16-bit operand
// arrays, which this policy leaves unused.
struct PfF32 {
    using Vec = pf_bf16x8_t;
    static constexpr float kWeightScale = 1.0f;
    static constexpr float kLazyLog2 = 8.0f;
    static constexpr bool kExact = true;
    static constexpr bool kF32 = true;
    static constexpr std::uint32_t kOnes = 0;
    __device__ static pf_f32x4_t mma4(float a, float b, const pf_f32x4_t& c) {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
};

// NaN-propagating maximum of three (one v_maximum3_f32).
__device__ inline float max3(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}
// Sum over the four lanes l, l^16, l^32, l^48, the same in all four (each
// level adds a pair in either order).
__device__ inline float sum_across_quads(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
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
// 16-row blocks per wavefront: four at head_size 64, two at 128, one at 256
// (the accumulators and Q operands of a block grow with the head size; more
// blocks share each K and V operand read: at 64, four blocks ran 18-22 %
// faster than two for 8 x 4096 tokens); one in the exact and FP32 variants
// (three Q parts, or FP32 operands; two at 64 measured no faster).
inline constexpr int pf_blocks_for(int head_size, bool exact) {
    return exact ? 1 : head_size == 64 ? 4 : head_size == 256 ? 1 : 2;
}
template <typename E, int kD>
constexpr int pf_blocks() { return pf_blocks_for(kD, E::kExact); }
constexpr int kPfTileShift = 6;
constexpr int kPfTile = 1 << kPfTileShift;  // keys per LDS tile
// Page ids held in LDS per workgroup, one window of the sequence at a time:
// 2048 (8 KiB, 32K tokens at block_size 16) beside the tiles.
template <int kD>
constexpr int pf_table_max() { return 2048; }
// Flag bit of a missing page in the LDS page list (ids are below 2^31): its
// K and V rows are loaded from pf_zero_rows instead.
constexpr std::uint32_t kPfMissing = 0x80000000u;
// The rows of one 64-key tile at head_size <= 256
// (16-bit elements): the source of missing pages, all zeros.
constexpr int kPfZeroBytes = 64 * 512;
__device__ __attribute__((aligned(16))) unsigned char pf_zero_rows[kPfZeroBytes];

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
    std::uint32_t q_group;    // query heads per kv head
    std::uint32_t q_first;    // first query head of the group this launch covers
    std::uint32_t q_pass;     // query heads this launch covers (rows: token-major, head-minor)
    std::uint32_t tok;        // query tokens per workgroup: floor(rows per workgroup / q_pass)
    std::uint32_t qblocks;    // ceil(tq / tokens per workgroup)
    const float* query;       // [tq][query_heads][D]
    float* output;            // [tq][query_heads][D]
    float scale_log2;         // log2(e) / sqrt(D)
    // Key splits: workgroup (split s) covers key tiles [s * split_tiles,
    // (s + 1) * split_tiles). With splits > 1 it writes unnormalised partials
    // (part_o [splits][tq][query_heads][D], part_ml [splits][tq][query_heads]
    // {reference point, weight sum}) for paged_prefill_combine_kernel.
    std::uint32_t splits;
    std::uint32_t split_tiles;
    float* part_o;
    float* part_ml;
    // Batch launches (num_seqs > 0): workgroup sequence (blockIdx.x / heads)
    // % num_seqs, whose table is row `seq` of `table` (table_len entries per
    // row), with seq_kv_lens[seq] tokens of which the last seq_q_lens[seq]
    // are queries, at rows seq_q_offsets[seq] .. of query/output. qblocks is
    // then the largest query block count; kv_len bounds every sequence.
    std::uint32_t num_seqs;
    const std::uint64_t* seq_kv_lens;
    const std::uint64_t* seq_q_lens;
    const std::uint64_t* seq_q_offsets;
};

// s_waitcnt immediates (gfx9 encoding): vmcnt(n) alone, lgkmcnt(0) alone.
template <int kN>
__device__ inline void wait_vm() {
    static_assert(kN >= 0 && kN < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((kN & 15) | ((kN >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ inline void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xF | (3 << 14) | (7 << 4)); }
// One 16-byte-per-lane load from global memory straight into LDS at
// m0 + lane * 16 (m0 wave-uniform). Issued as inline assembly so the
// compiler's wait-count tracking does not treat it as an LDS write (it would
// then wait for every such load before any LDS read); completion is ordered
// by the explicit vmcnt waits before the barriers.
__device__ inline void load_to_lds(const void* src, std::uint32_t lds_byte) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds_byte) : "memory");
}
__device__ inline std::uint32_t lds_address(const void* p) {
    return static_cast<std::uint32_t>(reinterpret_cast<std::uintptr_t>((__attribute__((address_space(3))) const char*)p));
}
// Workgroup barrier without the release fence of __syncthreads (which would
// also wait for the tile loads still in flight); LDS visibility is ordered by
// the explicit waits before it.
__device__ inline void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}
// Wave priority (s_setprio) pinned in place: raised while a wave issues its
// QK^T MFMAs, so a SIMD's other wave runs its softmax in the meantime.
template <short kLevel>
__device__ inline void set_priority() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(kLevel);
    __builtin_amdgcn_sched_barrier(0);
}

template <typename E, int kD>
__global__ __launch_bounds__(kPfThreads) void paged_prefill_kernel(PrefillParams p) {
    using M = E;
    using Vec = typename M::Vec;
    constexpr bool kF32 = E::kF32;
    constexpr int kSteps = kD / 32;            // K-dim steps of S^T (16-bit)
    constexpr int kQuads = kD / 16;            // 16-dim chunks of S^T (FP32: four MFMAs each)
    constexpr int kDt = kD / 16;               // dim blocks of O^T
    constexpr int kRowBytes = kD * (kF32 ? 4 : 2);
    constexpr int kCpr = kRowBytes / 16;       // 16-byte chunks per key row
    constexpr int kTileBytes = kPfTile * kRowBytes;
    constexpr int kDma = kTileBytes / (kPfThreads * 16);  // tile loads per thread per cache
    constexpr int kPfNt = pf_blocks<E, kD>();
    constexpr bool kExact = E::kExact;
    constexpr int kParts = kExact && !kF32 ? 3 : 1;  // 16-bit parts of Q and of the weights
    constexpr int kBlocks = kPfWaves * kPfNt;   // 16-row blocks per workgroup
    constexpr int kVSwz = kF32 ? 0 : kCpr / 8;  // V slot swizzle multiplier (FP32 V rows are read straight)
    constexpr float kLazy = E::kLazyLog2;
    constexpr float kWeightScale = E::kWeightScale;
    static_assert(kDma >= 1 && kTileBytes % (kPfThreads * 16) == 0, "tile split");
    static_assert(!kF32 || kD <= 128, "FP32 tiles of head_size 256 exceed the LDS");

    __shared__ __attribute__((aligned(16))) std::uint16_t ktile0[kTileBytes / 2];
    __shared__ __attribute__((aligned(16))) std::uint16_t ktile1[kTileBytes / 2];
    __shared__ __attribute__((aligned(16))) std::uint16_t vtile0[kTileBytes / 2];
    __shared__ __attribute__((aligned(16))) std::uint16_t vtile1[kTileBytes / 2];
    __shared__ std::uint32_t pages[pf_table_max<kD>()];

    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int col = lane % 16, quad = lane / 16;
    const std::uint32_t kvh = blockIdx.x % p.heads;
    // This workgroup's sequence: the launch's one, or in a batch launch
    // sequence (blockIdx.x / heads) % num_seqs (heavy query blocks of every
    // sequence first). All values wave-uniform.
    std::uint32_t split = 0, qb = 0, kv_len = p.kv_len, tq = p.tq, table_len = p.table_len;
    const std::uint64_t* table = p.table;
    const float* query = p.query;
    float* output = p.output;
    if (p.num_seqs == 0) {
        split = (blockIdx.x / p.heads) % p.splits;
        qb = p.qblocks - 1 - blockIdx.x / p.heads / p.splits;
    } else {
        const std::uint32_t seq = (blockIdx.x / p.heads) % p.num_seqs;
        qb = p.qblocks - 1 - blockIdx.x / p.heads / p.num_seqs;
        const std::uint64_t kvl = p.seq_kv_lens[seq], ql = p.seq_q_lens[seq], q0 = p.seq_q_offsets[seq];
        kv_len = static_cast<std::uint32_t>(kvl < p.kv_len ? kvl : p.kv_len);
        tq = static_cast<std::uint32_t>(ql < kv_len ? ql : kv_len);
        table = p.table + static_cast<std::uint64_t>(seq) * p.table_len;
        query = p.query + q0 * p.query_heads * kD;
        output = p.output + q0 * p.query_heads * kD;
        if (tq == 0 || static_cast<std::uint64_t>(qb) * p.tok >= tq) return;  // uniform
    }
    const std::uint32_t t0 = qb * p.tok;
    const std::uint32_t t_end = t0 + p.tok < tq ? t0 + p.tok : tq;
    const std::uint32_t past = kv_len - tq;
    const std::uint32_t last_key = past + t_end - 1;
    const std::uint32_t ntiles = last_key / kPfTile + 1;
    // This split's tiles [tile_begin, tile_end). The split holding the tile of
    // the first row's position runs to the last tile and later splits are
    // empty, so every split a workgroup runs starts at a key all its rows see
    // (each row then sets its reference point on the first half-tile).
    const std::uint32_t first_row_tile = (past + t0) / kPfTile;
    std::uint32_t tile_begin = split * p.split_tiles;
    std::uint32_t tile_end = tile_begin + p.split_tiles;
    if (tile_end > first_row_tile) tile_end = ntiles;
    if (tile_begin > first_row_tile) tile_begin = tile_end;
    const std::uint32_t npages = ((ntiles * kPfTile - 1) >> p.bs_shift) + 1;
    // Key k of the sequence lies in page k >> bs_shift, row k & (bs - 1).
    // The page list holds a window of kWin pages (whole tiles) at a time: page
    // `first` + i at pages[i]. A prompt longer than one window is restaged at
    // each window boundary of the tile loop.
    constexpr std::uint32_t kWin = pf_table_max<kD>();
    // Tiles per window - 1 (windows start at multiples of kWin pages).
    const std::uint32_t win_mask = static_cast<std::uint32_t>((static_cast<std::uint64_t>(kWin) << p.bs_shift) >> kPfTileShift) - 1;
    auto first_page = [&](std::uint32_t tile) { return (tile << kPfTileShift) >> p.bs_shift; };
    auto stage = [&](std::uint32_t first) {
        for (std::uint32_t i = tid; i < kWin && first + i < npages; i += kPfThreads) {
            const std::uint32_t pg = first + i;
            const std::uint64_t id = pg < table_len ? table[pg] : p.num_blocks;
            const bool ok = id < p.num_blocks && (static_cast<std::uint64_t>(pg) << p.bs_shift) < kv_len;
            pages[i] = ok ? static_cast<std::uint32_t>(id) : kPfMissing;
        }
    };
    // The query rows' loads go out before the page list's, so the two round
    // trips overlap; the rows are rounded to the cache dtype after.
    // 16-bit caches: float4 pairs 2kk, 2kk + 1 are dims 32kk + 8quad .. +8 of
    // the row; FP32: float4 c is dims 16c + 4quad .. +4.
    float4 qraw[kPfNt][kQuads];
    std::uint32_t row_token[kPfNt], row_head[kPfNt];
#pragma unroll
    for (int n = 0; n < kPfNt; ++n) {
        // Row 16 b + col: head (16 b + col) % G of token (16 b + col) / G.
        const std::uint32_t r = static_cast<std::uint32_t>(16 * (wave * kPfNt + n) + col);
        const std::uint32_t g = r % p.q_pass;
        const std::uint32_t token = t0 + r / p.q_pass;
        row_token[n] = token;
        row_head[n] = g;
        const std::uint32_t tq_safe = token < tq ? token : tq - 1;
        const float* src =
            query + (static_cast<std::uint64_t>(tq_safe) * p.query_heads + kvh * p.q_group + p.q_first + g) * kD;
#pragma unroll
        for (int c = 0; c < kQuads; ++c) {
            const int off = kF32 ? 16 * c + 4 * quad : 32 * (c / 2) + 8 * quad + 4 * (c % 2);
            qraw[n][c] = *reinterpret_cast<const float4*>(src + off);
        }
    }
    stage(first_page(tile_begin & ~win_mask));
    // FP32: Q * scale as it is, lane (quad, col) dims 16c + 4quad + j in qf[n][c][j].
    pf_f32x4_t qf[kF32 ? kPfNt : 1][kF32 ? kQuads : 1];
    Vec qb_op[kParts][kF32 ? 1 : kPfNt][kF32 ? 1 : kSteps];
#pragma unroll
    for (int n = 0; n < kPfNt; ++n) {
        if constexpr (kF32) {
#pragma unroll
            for (int c = 0; c < kQuads; ++c) {
                const float4 v = qraw[n][c];
                qf[n][c] = pf_f32x4_t{v.x, v.y, v.z, v.w} * p.scale_log2;
            }
        } else {
#pragma unroll
            for (int kk = 0; kk < kSteps; ++kk) {
                const float4 lo = qraw[n][2 * kk], hi = qraw[n][2 * kk + 1];
                const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                std::uint32_t w[kParts][4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if constexpr (kExact) {
                        std::uint32_t parts[3];
                        M::split3(v[2 * e] * p.scale_log2, v[2 * e + 1] * p.scale_log2, parts);
#pragma unroll
                        for (int k = 0; k < kParts; ++k) w[k][e] = parts[k];
                    } else {
                        w[0][e] = M::pack(v[2 * e] * p.scale_log2, v[2 * e + 1] * p.scale_log2);
                    }
                }
#pragma unroll
                for (int k = 0; k < kParts; ++k)
                    qb_op[k][n][kk] = __builtin_bit_cast(Vec, make_uint4(w[k][0], w[k][1], w[k][2], w[k][3]));
            }
        }
    }
    __syncthreads();  // pages[] ready (the query loads are complete as well)

    // Tile loads straight into LDS: load i of a wavefront fills bytes
    // [1 KiB * (i * waves + wave), +1 KiB) of the tile, lane l the 16 bytes
    // at l * 16 of that: LDS chunk e = row * kCpr + slot. The swizzle is set
    // by which global chunk a lane fetches: K chunk slot ^ kswz(row), V chunk
    // slot ^ vswz(row), so reads below see the swizzled layout.
    const char* kc = static_cast<const char*>(p.key_cache);
    const char* vc = static_cast<const char*>(p.value_cache);
    // Below 2^32 (the host declines larger pages).
    const std::uint32_t page_bytes = (static_cast<std::uint32_t>(kRowBytes) << p.bs_shift) * p.heads;
    const std::uint32_t head_bytes = (kvh << p.bs_shift) * kRowBytes;
    const std::uint32_t in_page_mask = (1u << p.bs_shift) - 1;
    auto kswz = [](int row) { return kCpr >= 16 ? (row & 15) : ((row >> 1) & 7); };
    auto vswz = [](int row) { return kVSwz * (row & 7); };
    auto issue = [&](std::uint32_t tile, auto buf) {
        // Key tile * 64 + row: page (tile * 64 >> bs_shift) + (row >> bs_shift)
        // and row (tile * 64 & (bs - 1)) + (row & (bs - 1)) of it, the tile's
        // terms wave-uniform (tile * 64 is a multiple of bs, or bs of 64).
        const std::uint32_t tile_page = ((tile & win_mask) << kPfTileShift) >> p.bs_shift;  // within the window
        const std::uint32_t tile_bytes = head_bytes + ((tile << kPfTileShift) & in_page_mask) * kRowBytes;
#pragma unroll
        for (int i = 0; i < kDma; ++i) {
            const int e = (i * kPfWaves + wave) * 64 + lane;
            const int row = e / kCpr, slot = e % kCpr;
            const std::uint32_t r = static_cast<std::uint32_t>(row) & in_page_mask;
            const std::uint32_t entry = pages[tile_page + (static_cast<std::uint32_t>(row) >> p.bs_shift)];
            const std::uint32_t kchunk = (slot ^ kswz(row)) * 16, vchunk = (slot ^ vswz(row)) * 16;
            const char* ks;
            const char* vs;
            if (entry & kPfMissing) {
                ks = reinterpret_cast<const char*>(pf_zero_rows) + row * kRowBytes + kchunk;
                vs = reinterpret_cast<const char*>(pf_zero_rows) + row * kRowBytes + vchunk;
            } else {
                const std::uint64_t base = static_cast<std::uint64_t>(entry) * page_bytes + tile_bytes + r * kRowBytes;
                ks = kc + base + kchunk;
                vs = vc + base + vchunk;
            }
            const std::uint32_t dst = static_cast<std::uint32_t>((i * kPfWaves + wave) * 1024);
            const std::uint32_t kdst = (decltype(buf)::value == 0 ? lds_address(ktile0) : lds_address(ktile1)) + dst;
            const std::uint32_t vdst = (decltype(buf)::value == 0 ? lds_address(vtile0) : lds_address(vtile1)) + dst;
            load_to_lds(ks, __builtin_amdgcn_readfirstlane(kdst));
            load_to_lds(vs, __builtin_amdgcn_readfirstlane(vdst));
        }
    };
    // Keys at or past kv_len of the last tile: their V rows are zeroed (a
    // finite value under a zero weight), each thread its own loaded chunks,
    // after its loads have landed.
    auto zero_tail = [&](std::uint32_t tile, std::uint16_t* vt) {
#pragma unroll
        for (int i = 0; i < kDma; ++i) {
            const int e = (i * kPfWaves + wave) * 64 + lane;
            const std::uint32_t key = tile * kPfTile + static_cast<std::uint32_t>(e / kCpr);
            if (key >= kv_len) *reinterpret_cast<uint4*>(reinterpret_cast<char*>(vt) + e * 16) = make_uint4(0, 0, 0, 0);
        }
    };

    // V^T block dt: v_read0 ^ (dt << 5); K step kk: k_read0 ^ (kk << 6)
    // (chunk quad + 4 * kk = quad ^ 4 * kk of row col; 64 * kk < kRowBytes).
    std::uint32_t v_read0;
    {
        const int s = lane % 16, r = 4 * quad + s / 4;
        const int c = (4 * (s % 4)) / 8;
        v_read0 = r * kRowBytes + ((c ^ vswz(r)) * 16) + (s % 2) * 8;
    }
    const std::uint32_t k_read0 = col * kRowBytes + (quad ^ kswz(col)) * 16;

    pf_f32x4_t acc[kDt][kPfNt];
#pragma unroll
    for (int dt = 0; dt < kDt; ++dt)
#pragma unroll
        for (int n = 0; n < kPfNt; ++n) acc[dt][n] = pf_f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // Row sums: the MFMA of the rounded weights against ones (the sum the
    // numerator uses), or in the exact variants each lane's FP32 sum of its
    // own weights of the row in lane 0 of the vector (added over the four
    // quads at the end).
    pf_f32x4_t lsum[kPfNt];
    // Minus the row's reference point, in all four accumulator lanes (the
    // seed of every QK^T chain; equal in the four quads of a column).
    pf_f32x4_t nref[kPfNt];
#pragma unroll
    for (int n = 0; n < kPfNt; ++n) {
        lsum[n] = pf_f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        nref[n] = pf_f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
    bool have_ref = false;
    const Vec ones = __builtin_bit_cast(Vec, make_uint4(M::kOnes, M::kOnes, M::kOnes, M::kOnes));
    const std::uint32_t min_limit = past + t0;

    auto compute_tile = [&](std::uint32_t tile, const std::uint16_t* kt, const std::uint16_t* vt) {
#pragma unroll
        for (int h = 0; h < kPfTile / 32; ++h) {
            const std::uint32_t k0 = tile * kPfTile + 32 * h;
            if (k0 > last_key) break;  // uniform
            pf_f32x4_t s[2][kPfNt];
            // V^T operands of the half-tile (head_size 128): read right after
            // K, so the LDS reads run under the QK^T MFMAs and the softmax;
            // P*V takes them from registers (8 x 4096 tokens, 32/8 heads:
            // 1.267 -> 1.245 ms). At 64 that measured 13% slower, and at 256
            // they would not fit the registers: there they are read inside P*V.
            const auto* vbase = (__attribute__((address_space(3))) char*)(
                (__attribute__((address_space(3))) std::uint16_t*)vt);
            auto read_v = [&](int dt) {
                const std::uint32_t off = (v_read0 ^ (dt << 5)) + 32 * h * kRowBytes;
                const pf_i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((pf_lds_i16x4_t*)(vbase + off));
                const pf_i16x4_t hi =
                    __builtin_amdgcn_ds_read_tr16_b64_v4i16((pf_lds_i16x4_t*)(vbase + off + 16 * kRowBytes));
                return __builtin_bit_cast(Vec, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            };
            constexpr bool kEarlyV = kD == 128 && !kF32;
            Vec vop[kEarlyV ? kDt : 1];
            set_priority<1>();
            if constexpr (kF32) {
                // MFMA (c, j) takes, in lane (quad, col), dim 16c + 4quad + j of
                // key col (K, one 16-byte read per c) and of row col (Q); the
                // dim order does not change the sum.
#pragma unroll
                for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
                    for (int n = 0; n < kPfNt; ++n) s[kt2][n] = nref[n];
#pragma unroll
                for (int c = 0; c < kQuads; ++c) {
                    float4 a[2];
#pragma unroll
                    for (int kt2 = 0; kt2 < 2; ++kt2)
                        a[kt2] = *reinterpret_cast<const float4*>(reinterpret_cast<const char*>(kt) +
                                                                  (32 * h + 16 * kt2) * kRowBytes + (k_read0 ^ (c << 6)));
#pragma unroll
                    for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
                        for (int n = 0; n < kPfNt; ++n) {
                            s[kt2][n] = M::mma4(a[kt2].x, qf[n][c][0], s[kt2][n]);
                            s[kt2][n] = M::mma4(a[kt2].y, qf[n][c][1], s[kt2][n]);
                            s[kt2][n] = M::mma4(a[kt2].z, qf[n][c][2], s[kt2][n]);
                            s[kt2][n] = M::mma4(a[kt2].w, qf[n][c][3], s[kt2][n]);
                        }
                }
            } else {
                Vec a[kSteps][2];
#pragma unroll
                for (int kk = 0; kk < kSteps; ++kk)
#pragma unroll
                    for (int kt2 = 0; kt2 < 2; ++kt2)
                        a[kk][kt2] = __builtin_bit_cast(
                            Vec, *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(kt) +
                                                                 (32 * h + 16 * kt2) * kRowBytes + (k_read0 ^ (kk << 6))));
#pragma unroll
                for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
                    for (int n = 0; n < kPfNt; ++n) s[kt2][n] = nref[n];
#pragma unroll
                for (int kk = 0; kk < kSteps; ++kk)
#pragma unroll
                    for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
                        for (int n = 0; n < kPfNt; ++n)
#pragma unroll
                            for (int k = 0; k < kParts; ++k) s[kt2][n] = M::mma(a[kk][kt2], qb_op[k][n][kk], s[kt2][n]);
                if constexpr (kEarlyV) {
#pragma unroll
                    for (int dt = 0; dt < kDt; ++dt) vop[dt] = read_v(dt);
                    // The K reads first, then the MFMAs, then the V reads.
                    __builtin_amdgcn_sched_group_barrier(0x100, 2 * kSteps, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 2 * kSteps * kPfNt * kParts, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 2 * kDt, 0);
                }
            }
            set_priority<0>();
            if (k0 + 31 > min_limit) {
#pragma unroll
                for (int n = 0; n < kPfNt; ++n) {
                    const std::int32_t room = static_cast<std::int32_t>(past + row_token[n] - k0 - 4 * quad);
#pragma unroll
                    for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
                        for (int r = 0; r < 4; ++r) s[kt2][n][r] = 16 * kt2 + r > room ? -INFINITY : s[kt2][n][r];
                }
            }
            // The wave rescales when some row's maximum exceeds its reference
            // by 2^kLazy: a lane's own maximum over its scores of the row
            // decides that (the row maximum, over the four quads, is needed
            // only inside the rare branch). A lane whose own maximum passes
            // while its row maximum is NaN enters with a zero shift for that
            // row, which changes nothing.
            float lmax[kPfNt];
            bool grow = !have_ref;
#pragma unroll
            for (int n = 0; n < kPfNt; ++n) {
                lmax[n] = max3(max3(s[0][n][0], s[0][n][1], s[0][n][2]), max3(s[0][n][3], s[1][n][0], s[1][n][1]),
                               max3(s[1][n][2], s[1][n][3], -INFINITY));
                grow |= lmax[n] > kLazy;
            }
            if (__builtin_expect(__builtin_amdgcn_ballot_w64(grow) != 0, 0)) {
#pragma unroll
                for (int n = 0; n < kPfNt; ++n) {
                    const float tmax = max_across_quads(lmax[n]);
                    const float shift = !have_ref || tmax > kLazy ? tmax : 0.0f;
                    const float alpha = __builtin_amdgcn_exp2f(fminf(-shift, 0.0f));
                    nref[n] -= shift;
                    lsum[n] *= alpha;
#pragma unroll
                    for (int kt2 = 0; kt2 < 2; ++kt2) s[kt2][n] -= shift;
#pragma unroll
                    for (int dt = 0; dt < kDt; ++dt) acc[dt][n] *= alpha;
                }
                have_ref = true;
            }
            if constexpr (kF32) {
                // O^T += V^T P^T over keys: MFMA (kt2, r, g, j) takes key
                // 16kt2 + 4quad + r in lane (quad, col), the weight the lane
                // holds, and V dim 64g + 4col + j (one 16-byte read of the key's
                // row per g). acc[4g + j][n][i] is then dim 64g + 16quad + 4i + j
                // of row col.
                const char* vrow = reinterpret_cast<const char*>(vt) + (32 * h + 4 * quad) * kRowBytes + 16 * col;
                // The tile's products are summed from zero and then added to
                // the running accumulator (one rounding per tile): added one
                // MFMA at a time to an accumulator dominated by one large
                // weight, small weights lose bits in the same direction at
                // every step (measured: 2.8e-5 on a row of one dominant key
                // and 4095 keys 2^-25 below it).
                pf_f32x4_t tpart[kD / 16][kPfNt];
#pragma unroll
                for (int i = 0; i < kD / 16; ++i)
#pragma unroll
                    for (int n = 0; n < kPfNt; ++n) tpart[i][n] = pf_f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int kt2 = 0; kt2 < 2; ++kt2) {
                    float pr[kPfNt][4];
#pragma unroll
                    for (int n = 0; n < kPfNt; ++n) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) pr[n][r] = __builtin_amdgcn_exp2f(s[kt2][n][r]);
                        float hi = lsum[n][0], lo = lsum[n][1];  // [1]: the sum's low word
                        two_sum_add(hi, lo, (pr[n][0] + pr[n][1]) + (pr[n][2] + pr[n][3]));
                        lsum[n][0] = hi;
                        lsum[n][1] = lo;
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r)
#pragma unroll
                        for (int g = 0; g < kD / 64; ++g) {
                            const float4 v =
                                *reinterpret_cast<const float4*>(vrow + (16 * kt2 + r) * kRowBytes + 256 * g);
#pragma unroll
                            for (int n = 0; n < kPfNt; ++n) {
                                tpart[4 * g][n] = M::mma4(v.x, pr[n][r], tpart[4 * g][n]);
                                tpart[4 * g + 1][n] = M::mma4(v.y, pr[n][r], tpart[4 * g + 1][n]);
                                tpart[4 * g + 2][n] = M::mma4(v.z, pr[n][r], tpart[4 * g + 2][n]);
                                tpart[4 * g + 3][n] = M::mma4(v.w, pr[n][r], tpart[4 * g + 3][n]);
                            }
                        }
                }
#pragma unroll
                for (int i = 0; i < kD / 16; ++i)
#pragma unroll
                    for (int n = 0; n < kPfNt; ++n) acc[i][n] += tpart[i][n];
            } else {
                Vec pb[kParts][kPfNt];
#pragma unroll
                for (int n = 0; n < kPfNt; ++n) {
                    float pr[8];
#pragma unroll
                    for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
                        for (int r = 0; r < 4; ++r) pr[4 * kt2 + r] = __builtin_amdgcn_exp2f(s[kt2][n][r]);
                    std::uint32_t w[kParts][4];
                    if constexpr (kExact) {
                        float hi = lsum[n][0], lo = lsum[n][1];  // [1]: the sum's low word
                        two_sum_add(hi, lo, ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7])));
                        lsum[n][0] = hi;
                        lsum[n][1] = lo;
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            std::uint32_t parts[3];
                            M::split3(pr[2 * j] * kWeightScale, pr[2 * j + 1] * kWeightScale, parts);
#pragma unroll
                            for (int k = 0; k < kParts; ++k) w[k][j] = parts[k];
                        }
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; ++j) w[0][j] = M::pack(pr[2 * j], pr[2 * j + 1]);
                    }
#pragma unroll
                    for (int k = 0; k < kParts; ++k) pb[k][n] = __builtin_bit_cast(Vec, make_uint4(w[k][0], w[k][1], w[k][2], w[k][3]));
                }
#pragma unroll
                for (int dt = 0; dt < kDt; ++dt) {
                    Vec a;
                    if constexpr (kEarlyV) {
                        a = vop[dt];
                    } else {
                        a = read_v(dt);
                    }
#pragma unroll
                    for (int n = 0; n < kPfNt; ++n) {
                        if constexpr (kExact) {
                            // The tile's three parts summed from zero, then
                            // one rounding into the running accumulator (see
                            // the FP32 path above).
                            pf_f32x4_t t = M::mma(a, pb[0][n], pf_f32x4_t{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
                            for (int k = 1; k < kParts; ++k) t = M::mma(a, pb[k][n], t);
                            acc[dt][n] += t;
                        } else {
#pragma unroll
                            for (int k = 0; k < kParts; ++k) acc[dt][n] = M::mma(a, pb[k][n], acc[dt][n]);
                        }
                    }
                }
                if constexpr (!kExact) {
#pragma unroll
                    for (int n = 0; n < kPfNt; ++n) lsum[n] = M::mma(ones, pb[0][n], lsum[n]);
                }
            }
        }
    };

    // Two LDS tile buffers: tile t lives in buffer t % 2. The loads of tile
    // t + 1 are issued before tile t is computed; each step waits for its own
    // tile's loads (2 * kDma per thread, issued one step earlier), then a
    // barrier publishes the tile; a second barrier frees the buffer.
    const bool tail = ntiles * kPfTile > kv_len;  // the last tile has keys past kv_len
    // Called at the top of a step, before tile `next` is issued. The barrier
    // first: every wave must be past its reads of the page list for the tiles
    // before `next` (a wave's reads are complete once it has issued that
    // tile's loads, whose addresses they give). On the first step nothing
    // else separates the split's first issue() from this restage.
    auto restage = [&](std::uint32_t next) {
        if ((next & win_mask) == 0) {  // uniform
            lds_barrier();
            stage(first_page(next));
            wait_lgkm0();
            lds_barrier();
        }
    };
    if (tile_begin < tile_end) issue(tile_begin, std::integral_constant<int, 0>{});  // uniform
    for (std::uint32_t tile = tile_begin; tile < tile_end; tile += 2) {
        if (tile + 1 < tile_end) {
            restage(tile + 1);
            issue(tile + 1, std::integral_constant<int, 1>{});
            wait_vm<2 * kDma>();
        } else {
            wait_vm<0>();
        }
        if (tail && tile + 1 == ntiles) zero_tail(tile, vtile0);
        wait_lgkm0();
        lds_barrier();
        compute_tile(tile, ktile0, vtile0);
        wait_lgkm0();
        lds_barrier();
        if (tile + 1 >= tile_end) break;
        if (tile + 2 < tile_end) {
            restage(tile + 2);
            issue(tile + 2, std::integral_constant<int, 0>{});
            wait_vm<2 * kDma>();
        } else {
            wait_vm<0>();
        }
        if (tail && tile + 2 == ntiles) zero_tail(tile + 1, vtile1);
        wait_lgkm0();
        lds_barrier();
        compute_tile(tile + 1, ktile1, vtile1);
        wait_lgkm0();
        lds_barrier();
    }

#pragma unroll
    for (int n = 0; n < kPfNt; ++n) {
        const float l = kExact ? sum_across_quads(lsum[n][0] + lsum[n][1]) : lsum[n][0];
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        const std::uint32_t token = row_token[n];
        if (token < t_end) {
            const std::uint64_t row =
                static_cast<std::uint64_t>(token) * p.query_heads + kvh * p.q_group + p.q_first + row_head[n];
            // One store path for both cases (two would hold the accumulators
            // twice): normalised rows of the output, or unnormalised partials.
            const bool whole = p.splits == 1;
            const std::uint64_t prow = static_cast<std::uint64_t>(split) * tq * p.query_heads + row;
            float* dst = whole ? output + row * kD : p.part_o + prow * kD;
            const float sc = (whole ? inv : 1.0f) * (1.0f / kWeightScale);  // kWeightScale: a power of two
            if constexpr (kF32) {
#pragma unroll
                for (int g = 0; g < kD / 64; ++g)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        *reinterpret_cast<float4*>(dst + 64 * g + 16 * quad + 4 * i) =
                            make_float4(acc[4 * g][n][i] * sc, acc[4 * g + 1][n][i] * sc, acc[4 * g + 2][n][i] * sc,
                                        acc[4 * g + 3][n][i] * sc);
            } else {
#pragma unroll
                for (int dt = 0; dt < kDt; ++dt) {
                    *reinterpret_cast<float4*>(dst + 16 * dt + 4 * quad) =
                        make_float4(acc[dt][n][0] * sc, acc[dt][n][1] * sc, acc[dt][n][2] * sc, acc[dt][n][3] * sc);
                }
            }
            // An empty split leaves l = 0; the combine skips it.
            if (!whole && quad == 0) *reinterpret_cast<float2*>(p.part_ml + 2 * prow) = make_float2(-nref[n][0], l);
        }
    }
}

// Merges the key splits of every (token, query head) row: weights
// exp2(ref_s - max ref) over the splits that saw a key, O = sum w_s O_s /
// sum w_s l_s. One wavefront per row, lane d4 holding dims 4*d4 .. +4.
template <int kD>
__global__ __launch_bounds__(256) void paged_prefill_combine_kernel(const float* __restrict__ part_o,
                                                                    const float* __restrict__ part_ml,
                                                                    float* __restrict__ output, std::uint64_t rows,
                                                                    std::uint32_t splits) {
    const std::uint64_t row = static_cast<std::uint64_t>(blockIdx.x) * 4 + threadIdx.x / 64;
    const int lane = threadIdx.x % 64;
    if (row >= rows) return;
    float m = -INFINITY;
    for (std::uint32_t sp = 0; sp < splits; ++sp) {
        const float2 ml = *reinterpret_cast<const float2*>(part_ml + 2 * (sp * rows + row));
        if (ml.y > 0.0f) m = fmaxf(m, ml.x);
    }
    constexpr int kLanes = kD / 4;
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float l = 0.0f;
    for (std::uint32_t sp = 0; sp < splits; ++sp) {
        const float2 ml = *reinterpret_cast<const float2*>(part_ml + 2 * (sp * rows + row));
        if (!(ml.y > 0.0f)) continue;  // uniform: no key of this split is visible to the row
        const float w = __builtin_amdgcn_exp2f(ml.x - m);
        l += w * ml.y;
        if (lane < kLanes) {
            const float4 x = *reinterpret_cast<const float4*>(part_o + (sp * rows + row) * kD + 4 * lane);
            o.x += w * x.x;
            o.y += w * x.y;
            o.z += w * x.z;
            o.w += w * x.w;
        }
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    if (lane < kLanes) {
        *reinterpret_cast<float4*>(output + row * kD + 4 * lane) = make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
    }
}

// One launch over the heads q_first .. q_first + q_pass - 1 of every kv head.
template <typename E, int kD>
int launch_prefill_pass(const PrefillParams& p, hipStream_t s) {
    PrefillParams q = p;
    constexpr unsigned kRows = 16 * kPfWaves * pf_blocks<E, kD>();
    q.tok = kRows / p.q_pass;
    // tq: the query tokens of the sequence, or the most of any sequence of a batch.
    q.qblocks = (p.tq + q.tok - 1) / q.tok;
    const std::uint64_t grid = static_cast<std::uint64_t>(q.qblocks) * p.heads * (p.num_seqs ? p.num_seqs : p.splits);
    if (grid > 0xffffffffULL) return fail(KVFLUX_ERR_UNSUPPORTED, "paged prefill: %llu workgroups",
                                          static_cast<unsigned long long>(grid));
    hipLaunchKernelGGL((paged_prefill_kernel<E, kD>), dim3(static_cast<unsigned>(grid)), dim3(kPfThreads), 0, s, q);
    return launch_status("paged_prefill_kernel");
}

// Query heads per launch for a GQA group with `rows` rows per workgroup (256,
// or 128 with one row block per wavefront): the whole group when it fits,
// else the largest divisor of it that does (the group then runs as
// group / sub launches over every kv head).
inline std::uint32_t prefill_sub_group(std::uint32_t group, std::uint32_t rows) {
    if (group <= rows) return group;
    for (std::uint32_t d = rows; d > 1; --d)
        if (group % d == 0) return d;
    return 1;
}

template <typename E, int kD>
int launch_prefill_group(const PrefillParams& p, std::uint32_t group, hipStream_t s) {
    constexpr std::uint32_t kRows = 16 * kPfWaves * pf_blocks<E, kD>();
    const std::uint32_t sub = prefill_sub_group(group, kRows);
    PrefillParams q = p;
    q.q_group = group;
    q.q_pass = sub;
    for (std::uint32_t first = 0; first < group; first += sub) {
        q.q_first = first;
        const int st = launch_prefill_pass<E, kD>(q, s);
        if (st != KVFLUX_OK) return st;
    }
    if (p.splits > 1) {
        const std::uint64_t rows = static_cast<std::uint64_t>(p.tq) * p.query_heads;
        hipLaunchKernelGGL(paged_prefill_combine_kernel<kD>, dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(256), 0,
                           s, p.part_o, p.part_ml, p.output, rows, p.splits);
        return launch_status("paged_prefill_combine_kernel");
    }
    return KVFLUX_OK;
}

template <typename E>
int launch_prefill_head_size(const PrefillParams& p, std::uint64_t head_size, std::uint32_t group, hipStream_t s) {
    switch (head_size) {
    case 64: return launch_prefill_group<E, 64>(p, group, s);
    case 128: return launch_prefill_group<E, 128>(p, group, s);
    default:
        if constexpr (E::kExact) {
            return fail(KVFLUX_ERR_UNSUPPORTED, "exact paged prefill: head_size %llu",
                        static_cast<unsigned long long>(head_size));
        } else {
            return launch_prefill_group<E, 256>(p, group, s);
        }
    }
}

struct PrefillPlan {
    std::uint32_t splits;       // key splits per (query block, kv head)
    std::uint32_t split_tiles;  // 64-key tiles per split
    std::uint64_t workspace;    // bytes of partials (0 when splits == 1)
};

// Key splits for a call whose launches hold fewer workgroups than about two
// per CU (short query blocks against a long prefix, as in chunked prefill):
// enough splits for ~512 workgroups, each of at least 4 tiles (256 keys), at
// most 32. Partials: [splits][tq][query_heads] rows of D floats, then the
// same rows of {reference point, weight sum}.
inline PrefillPlan prefill_plan(std::uint64_t head_size, std::uint64_t group, std::uint64_t num_kv_heads,
                                std::uint64_t kv_len, std::uint64_t query_tokens, std::uint64_t query_heads,
                                bool exact = false) {
    const std::uint64_t rows = 16 * kPfWaves * pf_blocks_for(static_cast<int>(head_size), exact);
    const std::uint64_t sub = prefill_sub_group(static_cast<std::uint32_t>(group), static_cast<std::uint32_t>(rows));
    const std::uint64_t tok = rows / sub;
    const std::uint64_t wgs = (query_tokens + tok - 1) / tok * num_kv_heads;
    const std::uint64_t tiles = (kv_len + kPfTile - 1) / kPfTile;
    std::uint64_t splits = wgs >= 512 ? 1 : (512 + wgs - 1) / wgs;
    if (splits > 32) splits = 32;
    if (splits > tiles / 4) splits = tiles / 4;
    if (splits < 1) splits = 1;
    const std::uint64_t split_tiles = (tiles + splits - 1) / splits;
    splits = (tiles + split_tiles - 1) / split_tiles;
    const std::uint64_t ws = splits > 1 ? splits * query_tokens * query_heads * (head_size + 2) * sizeof(float) : 0;
    return {static_cast<std::uint32_t>(splits), static_cast<std::uint32_t>(split_tiles), ws};
}

} // namespace
} // namespace kvflux_hip

using namespace kvflux_hip;

namespace {

int paged_prefill(const void* key_cache, const void* value_cache, uint64_t num_blocks, uint64_t num_kv_heads,
                  uint64_t block_size, uint64_t head_size, int dtype, const uint64_t* block_table,
                  uint64_t num_table_blocks, uint64_t kv_len, uint64_t query_tokens, uint64_t query_heads,
                  const float* query, float* output, void* workspace, uint64_t workspace_bytes, void* stream,
                  bool exact = false) {
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
    if ((head_size != 64 && head_size != 128 && head_size != 256) || !is_pow2(block_size) || block_size > 256 ||
        num_blocks > 0x7fffffffULL || num_kv_heads > 65535 || kv_len > 0x7fffffffULL || query_heads > 0xffffffffULL ||
        num_kv_heads * block_size * head_size * dtype_bytes(dtype) > 0xffffffffULL) {
        return fail(KVFLUX_ERR_UNSUPPORTED, "paged prefill: shape not handled by the MFMA kernel");
    }
    // FP32 caches always take the FP32 MFMAs, whose products are exact.
    if (dtype == KVFLUX_DTYPE_F32) exact = true;
    if (exact && head_size == 256) return fail(KVFLUX_ERR_UNSUPPORTED, "exact paged prefill: head_size 256");

    PrefillParams p{};
    p.key_cache = key_cache;
    p.value_cache = value_cache;
    p.num_blocks = num_blocks;
    p.heads = static_cast<std::uint32_t>(num_kv_heads);
    std::uint32_t shift = 0;
    while ((std::uint64_t{1} << shift) < block_size) ++shift;
    p.bs_shift = shift;
    p.table = block_table;
    p.table_len = static_cast<std::uint32_t>(num_table_blocks < 0xffffffffULL ? num_table_blocks : 0xffffffffULL);
    p.kv_len = static_cast<std::uint32_t>(kv_len);
    p.tq = static_cast<std::uint32_t>(query_tokens);
    p.query_heads = static_cast<std::uint32_t>(query_heads);
    p.query = query;
    p.output = output;
    p.scale_log2 = static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(head_size)));
    p.splits = 1;
    p.split_tiles = static_cast<std::uint32_t>((kv_len + kPfTile - 1) / kPfTile);
    if (workspace) {
        const PrefillPlan plan = prefill_plan(head_size, group, num_kv_heads, kv_len, query_tokens, query_heads, exact);
        if (plan.splits > 1) {
            if (workspace_bytes < plan.workspace) {
                return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged prefill: workspace of %llu bytes, %llu needed",
                            static_cast<unsigned long long>(workspace_bytes),
                            static_cast<unsigned long long>(plan.workspace));
            }
            p.splits = plan.splits;
            p.split_tiles = plan.split_tiles;
            p.part_o = static_cast<float*>(workspace);
            p.part_ml = p.part_o + static_cast<std::uint64_t>(plan.splits) * query_tokens * query_heads * head_size;
        }
    }
    const hipStream_t s = as_stream(stream);
    const std::uint32_t g = static_cast<std::uint32_t>(group);
    if (dtype == KVFLUX_DTYPE_F32) return launch_prefill_head_size<PfF32>(p, head_size, g, s);
    if (exact) {
        if (dtype == KVFLUX_DTYPE_BF16) return launch_prefill_head_size<PfBf16Exact>(p, head_size, g, s);
        return launch_prefill_head_size<PfF16Exact>(p, head_size, g, s);
    }
    if (dtype == KVFLUX_DTYPE_BF16) return launch_prefill_head_size<PfBf16>(p, head_size, g, s);
    return launch_prefill_head_size<PfF16>(p, head_size, g, s);
}

} // namespace

extern "C" int kvflux_paged_prefill(const void* key_cache, const void* value_cache, uint64_t num_blocks,
                                    uint64_t num_kv_heads, uint64_t block_size, uint64_t head_size, int dtype,
                                    const uint64_t* block_table, uint64_t num_table_blocks, uint64_t kv_len,
                                    uint64_t query_tokens, uint64_t query_heads, const float* query,
                                    float* output, void* stream) {
    return paged_prefill(key_cache, value_cache, num_blocks, num_kv_heads, block_size, head_size, dtype, block_table,
                         num_table_blocks, kv_len, query_tokens, query_heads, query, output, nullptr, 0, stream);
}

extern "C" int kvflux_paged_prefill_workspace_size(uint64_t num_kv_heads, uint64_t head_size, uint64_t kv_len,
                                                   uint64_t query_tokens, uint64_t query_heads, size_t* bytes) {
    if (!bytes) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged prefill workspace: null pointer");
    *bytes = 0;
    if (query_tokens == 0 || num_kv_heads == 0 || query_heads == 0 || query_heads % num_kv_heads != 0 ||
        (head_size != 64 && head_size != 128 && head_size != 256) || kv_len == 0 || kv_len > 0x7fffffffULL ||
        query_tokens > kv_len || query_heads > 0xffffffffULL) {
        return KVFLUX_OK;  // no split launch for such a call
    }
    // One size for every variant: the exact and FP32-cache kernels hold
    // fewer rows per workgroup than the rounded ones, so for some groups
    // (a large group with a small divisor <= 128, e.g. 131) they launch
    // fewer workgroups and plan more key splits.
    const std::uint64_t group = query_heads / num_kv_heads;
    const std::uint64_t rounded =
        prefill_plan(head_size, group, num_kv_heads, kv_len, query_tokens, query_heads, false).workspace;
    const std::uint64_t exact =
        head_size == 256 ? 0 : prefill_plan(head_size, group, num_kv_heads, kv_len, query_tokens, query_heads, true).workspace;
    *bytes = static_cast<size_t>(rounded > exact ? rounded : exact);
    return KVFLUX_OK;
}

extern "C" int kvflux_paged_prefill_split(const void* key_cache, const void* value_cache, uint64_t num_blocks,
                                          uint64_t num_kv_heads, uint64_t block_size, uint64_t head_size, int dtype,
                                          const uint64_t* block_table, uint64_t num_table_blocks, uint64_t kv_len,
                                          uint64_t query_tokens, uint64_t query_heads, const float* query,
                                          float* output, void* workspace, uint64_t workspace_bytes, void* stream) {
    return paged_prefill(key_cache, value_cache, num_blocks, num_kv_heads, block_size, head_size, dtype, block_table,
                         num_table_blocks, kv_len, query_tokens, query_heads, query, output, workspace,
                         workspace_bytes, stream);
}

extern "C" int kvflux_paged_prefill_exact(const void* key_cache, const void* value_cache, uint64_t num_blocks,
                                          uint64_t num_kv_heads, uint64_t block_size, uint64_t head_size, int dtype,
                                          const uint64_t* block_table, uint64_t num_table_blocks, uint64_t kv_len,
                                          uint64_t query_tokens, uint64_t query_heads, const float* query,
                                          float* output, void* workspace, uint64_t workspace_bytes, void* stream) {
    return paged_prefill(key_cache, value_cache, num_blocks, num_kv_heads, block_size, head_size, dtype, block_table,
                         num_table_blocks, kv_len, query_tokens, query_heads, query, output, workspace,
                         workspace_bytes, stream, true);
}

extern "C" int kvflux_paged_prefill_batch(const void* key_cache, const void* value_cache, uint64_t num_blocks,
                                          uint64_t num_kv_heads, uint64_t block_size, uint64_t head_size, int dtype,
                                          const uint64_t* block_table, uint64_t max_blocks_per_seq,
                                          const uint64_t* kv_lens, const uint64_t* query_lens,
                                          const uint64_t* query_offsets, uint64_t num_seqs, uint64_t max_query_tokens,
                                          uint64_t max_kv_len, uint64_t query_heads, const float* query, float* output,
                                          void* stream) {
    if (num_seqs == 0 || max_query_tokens == 0) return KVFLUX_OK;
    if (dtype_bytes(dtype) == 0) return fail(KVFLUX_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
    if (!key_cache || !value_cache || !block_table || !kv_lens || !query_lens || !query_offsets || !query ||
        !output) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged prefill batch: null pointer");
    }
    if (num_blocks == 0 || num_kv_heads == 0 || block_size == 0 || head_size == 0 || query_heads == 0 ||
        query_heads % num_kv_heads != 0 || max_blocks_per_seq == 0) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged prefill batch: invalid shape");
    }
    if (max_query_tokens > max_kv_len) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged prefill batch: more queries than tokens");
    }
    if (max_blocks_per_seq * block_size < max_kv_len) {
        return fail(KVFLUX_ERR_INVALID_ARGUMENT, "paged prefill batch: table rows shorter than max_kv_len");
    }
    if ((head_size != 64 && head_size != 128 && head_size != 256) || (dtype == KVFLUX_DTYPE_F32 && head_size == 256) ||
        !is_pow2(block_size) || block_size > 256 || num_blocks > 0x7fffffffULL || num_kv_heads > 65535 ||
        max_kv_len > 0x7fffffffULL || query_heads > 0xffffffffULL || num_seqs > 0xffffffffULL ||
        max_blocks_per_seq > 0xffffffffULL || num_kv_heads * block_size * head_size * dtype_bytes(dtype) > 0xffffffffULL) {
        return fail(KVFLUX_ERR_UNSUPPORTED, "paged prefill batch: shape not handled by the MFMA kernel");
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
    p.table_len = static_cast<std::uint32_t>(max_blocks_per_seq);
    p.kv_len = static_cast<std::uint32_t>(max_kv_len);
    p.tq = static_cast<std::uint32_t>(max_query_tokens);
    p.query_heads = static_cast<std::uint32_t>(query_heads);
    p.query = query;
    p.output = output;
    p.scale_log2 = static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(head_size)));
    p.splits = 1;
    p.split_tiles = static_cast<std::uint32_t>((max_kv_len + kPfTile - 1) / kPfTile);
    p.num_seqs = static_cast<std::uint32_t>(num_seqs);
    p.seq_kv_lens = kv_lens;
    p.seq_q_lens = query_lens;
    p.seq_q_offsets = query_offsets;
    const hipStream_t s = as_stream(stream);
    const std::uint32_t g = static_cast<std::uint32_t>(query_heads / num_kv_heads);
    if (dtype == KVFLUX_DTYPE_F32) return launch_prefill_head_size<PfF32>(p, head_size, g, s);
    if (dtype == KVFLUX_DTYPE_BF16) return launch_prefill_head_size<PfBf16>(p, head_size, g, s);
    return launch_prefill_head_size<PfF16>(p, head_size, g, s);
}
