/*
 * CPU oracle of the paged-KV data path -- TEST INFRASTRUCTURE ONLY.
 *
 * Plain C restatement of the reference's algorithms, used by tests/, the
 * smoke run and bench.py's CPU baseline to check the HIP kernels. Nothing in
 * the shipped library links or calls this file.
 *
 *   oracle_reference_attention  reference src/v2/reference_attention.cpp:28-91
 *   oracle_write_paged_kv       reference src/v2/paged_kv_write.cu:62-83
 *   oracle_gather_paged_kv      reference src/v2/paged_kv_read.cu:67-87
 *   oracle_paged_attention_rows reference src/v2/paged_attention.cu:73-153
 *                               (paged K/V, checked as gather + reference
 *                               attention, tests/paged_attention_test.cu:86-110)
 *   oracle_fill_random          the counter-based generator of kvflux_hip.h
 *
 * Arithmetic of the attention follows reference_attention.cpp exactly: FP32
 * inputs widened to double, dot products and the softmax in double, in the
 * same loop order, scale = 1/sqrt((double)head_size), output rounded to FP32.
 * Built with gcc -O2 for baseline x86-64 (no FMA contraction), so results
 * are bit-identical to the reference's own CPU build.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { OR_OK = 0, OR_INVALID = 1, OR_RANGE = 2, OR_OVERFLOW = 3 };
enum { OR_F16 = 0, OR_BF16 = 1, OR_F32 = 2 };

/* ------------------------------------------------------------ conversions */

float oracle_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const int exp = (h >> 10) & 0x1f;
    const uint32_t mant = h & 0x3ffu;
    float f;
    if (exp == 0) {
        f = ldexpf((float)mant, -24); /* subnormal or zero: mant * 2^-24, exact */
        uint32_t u;
        memcpy(&u, &f, 4);
        u |= sign;
        memcpy(&f, &u, 4);
        return f;
    }
    uint32_t u;
    if (exp == 31) {
        u = sign | 0x7f800000u | (mant << 13);
    } else {
        u = sign | ((uint32_t)(exp - 15 + 127) << 23) | (mant << 13);
    }
    memcpy(&f, &u, 4);
    return f;
}

/* Round-to-nearest-even FP32 -> BF16 (finite inputs). */
uint16_t oracle_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint32_t lower = u & 0xffffu;
    uint32_t upper = u >> 16;
    if (lower > 0x8000u || (lower == 0x8000u && (upper & 1u))) upper += 1;
    return (uint16_t)upper;
}

/* Round-to-nearest-even FP32 -> FP16 via the exact value: scale into the
 * FP16 grid with ldexp (exact), round with rint (current mode: nearest-even). */
uint16_t oracle_f32_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    double a = fabs((double)f);
    if (a == 0.0) return sign;
    int e;
    (void)frexp(a, &e);         /* a = m * 2^e, m in [0.5, 1) */
    int unit_exp = e - 11;      /* 11 significant bits for normals */
    if (unit_exp < -24) unit_exp = -24; /* subnormal grid 2^-24 */
    double q = rint(ldexp(a, -unit_exp));
    /* q * 2^unit_exp; renormalise if rounding carried to 2^11 */
    if (q >= 2048.0) {
        q /= 2.0;
        unit_exp += 1;
    }
    if (unit_exp == -24 && q < 1024.0) return (uint16_t)(sign | (uint16_t)q); /* subnormal */
    const int biased = unit_exp + 10 + 15;
    if (biased >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | (uint16_t)(biased << 10) | ((uint16_t)q & 0x3ffu));
}

static float load_elem(const void* base, size_t index, int dtype) {
    switch (dtype) {
    case OR_F32: return ((const float*)base)[index];
    case OR_BF16: return oracle_bf16_to_f32(((const uint16_t*)base)[index]);
    default: return oracle_f16_to_f32(((const uint16_t*)base)[index]);
    }
}

static size_t elem_bytes(int dtype) { return dtype == OR_F32 ? 4 : 2; }

/* ------------------------------------------------------------ random fill */

static uint64_t splitmix64_at(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

float oracle_random_value(uint64_t seed, uint64_t i, int distribution) {
    if (distribution == 0) {
        const uint32_t k = (uint32_t)(splitmix64_at(seed, i) >> 40);
        return (float)((double)k / 8388608.0 - 1.0); /* k * 2^-23 - 1, exact */
    }
    int32_t sum = 0;
    for (int j = 0; j < 3; ++j) {
        const uint64_t h = splitmix64_at(seed, 3 * i + (uint64_t)j);
        for (int s = 0; s < 64; s += 16) sum += (int32_t)((h >> s) & 0xffffu);
    }
    return (float)((double)(sum - 393210) / 65536.0);
}

/* Elements [first, first + count) of the stream, written from dst[0]. */
void oracle_fill_random(void* dst, uint64_t first, uint64_t count, int dtype, int distribution,
                        uint64_t seed) {
    for (uint64_t j = 0; j < count; ++j) {
        const float x = oracle_random_value(seed, first + j, distribution);
        if (dtype == OR_F32) ((float*)dst)[j] = x;
        else if (dtype == OR_BF16) ((uint16_t*)dst)[j] = oracle_f32_to_bf16(x);
        else ((uint16_t*)dst)[j] = oracle_f32_to_f16(x);
    }
}

/* ------------------------------------------------------------ write / gather */

/* Scatter: for token n, head h, the D-element row of key_new/value_new goes to
 * cache row ((slot / bs) * H + h) * bs + slot % bs (raw bytes). */
void oracle_write_paged_kv(void* key_cache, void* value_cache, size_t heads, size_t block_size,
                           size_t head_size, int dtype, const void* key_new,
                           const void* value_new, const uint64_t* slots, size_t tokens) {
    const size_t row = head_size * elem_bytes(dtype);
    for (size_t n = 0; n < tokens; ++n) {
        const uint64_t page = slots[n] / block_size, off = slots[n] % block_size;
        for (size_t h = 0; h < heads; ++h) {
            const size_t dst = ((page * heads + h) * block_size + off) * row;
            const size_t src = (n * heads + h) * row;
            memcpy((char*)key_cache + dst, (const char*)key_new + src, row);
            memcpy((char*)value_cache + dst, (const char*)value_new + src, row);
        }
    }
}

/* Gather one sequence of `tokens` tokens through its page table into
 * [token][head][dim] order (raw bytes). */
void oracle_gather_paged_kv(const void* key_cache, const void* value_cache, size_t heads,
                            size_t block_size, size_t head_size, int dtype,
                            const uint64_t* table, size_t tokens, void* key_out,
                            void* value_out) {
    const size_t row = head_size * elem_bytes(dtype);
    for (size_t t = 0; t < tokens; ++t) {
        const uint64_t page = table[t / block_size];
        for (size_t h = 0; h < heads; ++h) {
            const size_t src = ((page * heads + h) * block_size + t % block_size) * row;
            const size_t dst = (t * heads + h) * row;
            memcpy((char*)key_out + dst, (const char*)key_cache + src, row);
            memcpy((char*)value_out + dst, (const char*)value_cache + src, row);
        }
    }
}

/* ------------------------------------------------------------ attention */

static int mul_ok(size_t a, size_t b, size_t* out) {
    if (b != 0 && a > SIZE_MAX / b) return 0;
    *out = a * b;
    return 1;
}

/* One (query token, query head) output over visible tokens [0, last]. K/V
 * element (t, kvh, d) is read through `kv_at`. Loop order and double
 * arithmetic as reference_attention.cpp:51-87. */
typedef struct {
    const void* key;
    const void* value;
    int dtype;
    /* contiguous [T][H][D] when table == NULL, else paged */
    const uint64_t* table;
    size_t heads, block_size, head_size;
} KVSource;

static size_t kv_row(const KVSource* s, size_t t, size_t kvh) {
    if (!s->table) return (t * s->heads + kvh) * s->head_size;
    const uint64_t page = s->table[t / s->block_size];
    return ((page * s->heads + kvh) * s->block_size + t % s->block_size) * s->head_size;
}

static void attend_one(const KVSource* s, const float* q, size_t kvh, size_t last, double scale,
                       double* scores, float* out) {
    const size_t D = s->head_size;
    double maximum = -INFINITY;
    for (size_t t = 0; t <= last; ++t) {
        const size_t k = kv_row(s, t, kvh);
        double dot = 0.0;
        for (size_t d = 0; d < D; ++d) dot += (double)q[d] * load_elem(s->key, k + d, s->dtype);
        scores[t] = dot * scale;
        if (scores[t] > maximum) maximum = scores[t];
    }
    double denominator = 0.0;
    for (size_t t = 0; t <= last; ++t) {
        scores[t] = exp(scores[t] - maximum);
        denominator += scores[t];
    }
    for (size_t d = 0; d < D; ++d) {
        double result = 0.0;
        for (size_t t = 0; t <= last; ++t) {
            result += (scores[t] / denominator) * load_elem(s->value, kv_row(s, t, kvh) + d, s->dtype);
        }
        out[d] = (float)result;
    }
}

/* Contiguous CPU reference attention, FP32 tensors:
 * Q/O [Tq][Hq][D], K/V [Tkv][H][D]; query i sees tokens <= Tkv - Tq + i.
 * Returns OR_INVALID for bad shapes or non-finite inputs, OR_OVERFLOW when a
 * tensor size overflows. */
int oracle_reference_attention(const float* q, const float* k, const float* v, size_t q_tokens,
                               size_t kv_tokens, size_t q_heads, size_t kv_heads,
                               size_t head_size, float* out) {
    if (q_heads == 0 || kv_heads == 0 || head_size == 0 || q_heads % kv_heads != 0 ||
        q_tokens > kv_tokens) {
        return OR_INVALID;
    }
    size_t nq, nkv, tmp;
    if (!mul_ok(q_tokens, q_heads, &tmp) || !mul_ok(tmp, head_size, &nq)) return OR_OVERFLOW;
    if (!mul_ok(kv_tokens, kv_heads, &tmp) || !mul_ok(tmp, head_size, &nkv)) return OR_OVERFLOW;
    for (size_t i = 0; i < nq; ++i) if (!isfinite(q[i])) return OR_INVALID;
    for (size_t i = 0; i < nkv; ++i) if (!isfinite(k[i]) || !isfinite(v[i])) return OR_INVALID;
    for (size_t i = 0; i < nq; ++i) out[i] = 0.0f;
    if (q_tokens == 0) return OR_OK;
    const double scale = 1.0 / sqrt((double)head_size);
    const size_t group = q_heads / kv_heads;
    double* scores = (double*)malloc(sizeof(double) * kv_tokens);
    if (!scores) return OR_OVERFLOW;
    KVSource s = {k, v, OR_F32, NULL, kv_heads, 1, head_size};
    for (size_t i = 0; i < q_tokens; ++i) {
        const size_t last = kv_tokens - q_tokens + i;
        for (size_t h = 0; h < q_heads; ++h) {
            const size_t off = (i * q_heads + h) * head_size;
            attend_one(&s, q + off, h / group, last, scale, scores, out + off);
        }
    }
    free(scores);
    return OR_OK;
}

/* Paged attention over rows. Row r uses page table `tables + r * table_stride`
 * and attends to tokens [0, lens[r]). Q/O [rows][Hq][D] FP32. Work is split
 * over `threads` POSIX threads by (row, query head); each output keeps the
 * single-thread arithmetic, so the result does not depend on `threads`. */
typedef struct {
    const KVSource* src;
    const uint64_t* tables;
    size_t table_stride;
    const uint64_t* lens;
    const float* q;
    float* out;
    size_t rows, q_heads, group;
    double scale;
    size_t begin, end; /* flat (row, head) range */
    size_t max_len;
} RowsJob;

static void* rows_worker(void* arg) {
    RowsJob* job = (RowsJob*)arg;
    double* scores = (double*)malloc(sizeof(double) * (job->max_len ? job->max_len : 1));
    if (!scores) return (void*)1;
    for (size_t idx = job->begin; idx < job->end; ++idx) {
        const size_t r = idx / job->q_heads, h = idx % job->q_heads;
        KVSource s = *job->src;
        s.table = job->tables + r * job->table_stride;
        const size_t off = idx * s.head_size;
        if (job->lens[r] == 0) continue;
        attend_one(&s, job->q + off, h / job->group, job->lens[r] - 1, job->scale, scores,
                   job->out + off);
    }
    free(scores);
    return NULL;
}

int oracle_paged_attention_rows(const void* key_cache, const void* value_cache, size_t kv_heads,
                                size_t block_size, size_t head_size, int dtype,
                                const uint64_t* tables, size_t table_stride,
                                const uint64_t* lens, size_t rows, size_t q_heads,
                                const float* q, float* out, int threads) {
    if (q_heads == 0 || kv_heads == 0 || q_heads % kv_heads != 0 || head_size == 0) return OR_INVALID;
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    KVSource src = {key_cache, value_cache, dtype, NULL, kv_heads, block_size, head_size};
    size_t max_len = 0;
    for (size_t r = 0; r < rows; ++r) if (lens[r] > max_len) max_len = lens[r];
    const size_t work = rows * q_heads;
    RowsJob jobs[256];
    pthread_t tid[256];
    const size_t per = (work + (size_t)threads - 1) / (size_t)threads;
    int started = 0, failed = 0;
    for (int t = 0; t < threads; ++t) {
        RowsJob* j = &jobs[t];
        j->src = &src;
        j->tables = tables;
        j->table_stride = table_stride;
        j->lens = lens;
        j->q = q;
        j->out = out;
        j->rows = rows;
        j->q_heads = q_heads;
        j->group = q_heads / kv_heads;
        j->scale = 1.0 / sqrt((double)head_size);
        j->begin = per * (size_t)t < work ? per * (size_t)t : work;
        j->end = j->begin + per < work ? j->begin + per : work;
        j->max_len = max_len;
        if (threads == 1) {
            failed |= rows_worker(j) != NULL;
        } else if (pthread_create(&tid[t], NULL, rows_worker, j) == 0) {
            ++started;
        } else {
            failed |= rows_worker(j) != NULL;
        }
    }
    for (int t = 0; t < started; ++t) {
        void* ret = NULL;
        pthread_join(tid[t], &ret);
        failed |= ret != NULL;
    }
    return failed ? OR_OVERFLOW : OR_OK;
}

/* Trailing causal queries of one paged sequence (reference
 * paged_attention.cu:108-128): query i sees tokens <= kv_len - q_tokens + i. */
int oracle_paged_attention_causal(const void* key_cache, const void* value_cache, size_t kv_heads,
                                  size_t block_size, size_t head_size, int dtype,
                                  const uint64_t* table, size_t kv_len, size_t q_tokens,
                                  size_t q_heads, const float* q, float* out, int threads) {
    if (q_tokens > kv_len) return OR_INVALID;
    uint64_t* lens = (uint64_t*)malloc(sizeof(uint64_t) * (q_tokens ? q_tokens : 1));
    if (!lens) return OR_OVERFLOW;
    for (size_t i = 0; i < q_tokens; ++i) lens[i] = kv_len - q_tokens + i + 1;
    const int status = oracle_paged_attention_rows(key_cache, value_cache, kv_heads, block_size,
                                                   head_size, dtype, table, 0, lens, q_tokens,
                                                   q_heads, q, out, threads);
    free(lens);
    return status;
}
