/*
 * ctox_oracle.c -- CPU restatement of CTOX-LLM's scalar oracle and its CPU
 * feature-dispatched (AVX2) path for the decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see ctox_oracle.h). Citations are relative to
 * the reference tree, Q/ = models/qwen38_27b/.
 *
 * Pinning (each function is checked by tests/test_oracle_*.py):
 *   - quant: reference round-trip bounds (Q/src/quant.rs:211-257), exhaustive
 *     unpack of every byte value, A8 extreme codes.
 *   - fused matvec: reference golden fixtures (Q/src/backend/cpu.rs:751-1126,
 *     Q/src/loader.rs:532-542 closed forms) and an f64 brute force.
 *   - gated delta: golden vectors emitted by the pinned Python implementation
 *     (Q/src/reference.rs:590-627, 756-799), closed forms (beta=0 decay only;
 *     orthonormal write), and the fp16-state drift bound (:630-722).
 *   - sampler / greedy MTP: reference unit cases (Q/src/sampler.rs:176-253,
 *     Q/src/engine.rs:1213-1300).
 *   - orc_mtp_accept_sample: no crate counterpart; pinned by the invariants
 *     of speculative rejection sampling (identical distributions always
 *     accept; a Monte-Carlo check that the output law equals the target law)
 *     and by decisions its definition fixes (accept iff u q(d) < p(d) for
 *     the next draw, the residual max(p - q, 0), draws consumed in order).
 */
#include "ctox_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#if defined(__x86_64__)
#include <immintrin.h>
#endif

#define BLOCK_LEN 64
#define Q2_BLOCK_BYTES 18
#define Q4_BLOCK_BYTES 34
#define L2_EPSILON 1e-6f

/* Q/src/quant.rs:8 -- evaluated in f32 like the Rust const. */
static const float Q2_CODEBOOK[4] = {-1.0f, -1.0f / 3.0f, 1.0f / 3.0f, 1.0f};

/* ------------------------------------------------------------------ */
/* IEEE binary16 conversions with the `half` crate semantics.           */
/* ------------------------------------------------------------------ */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400) == 0);
            man &= 0x3ff;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13) | (man ? 0x400000u : 0);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xff;
    uint32_t man = x & 0x7fffff;
    if (exp == 0xff) { /* inf / nan (nan keeps a quiet payload bit) */
        if (man == 0) return (uint16_t)(sign | 0x7c00);
        return (uint16_t)(sign | 0x7e00 | (man >> 13));
    }
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00); /* overflow -> inf */
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign; /* underflow to zero */
        man |= 0x800000;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half_man = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half_man & 1))) half_man++;
        return (uint16_t)(sign | half_man);
    }
    uint32_t half_man = man >> 13;
    uint32_t rem = man & 0x1fff;
    uint32_t out = sign | ((uint32_t)e << 10) | half_man;
    if (rem > 0x1000 || (rem == 0x1000 && (half_man & 1))) out++; /* carries into exp ok */
    return (uint16_t)out;
}

static int finite_f(float v) { return isfinite(v); }

/* Rust f32::total_cmp ordering key. */
static int32_t total_key(float v) {
    int32_t b;
    memcpy(&b, &v, 4);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}
static int total_cmp(float a, float b) {
    int32_t ka = total_key(a), kb = total_key(b);
    return (ka > kb) - (ka < kb);
}

/* ------------------------------------------------------------------ */
/* quant.rs                                                            */
/* ------------------------------------------------------------------ */
static int require_block(const float *v) {
    for (int i = 0; i < BLOCK_LEN; i++)
        if (!finite_f(v[i])) return ORC_ERR_INVALID_ARTIFACT;
    return ORC_OK;
}

static float fold_max_abs(const float *v) {
    float m = 0.0f;
    for (int i = 0; i < BLOCK_LEN; i++) m = fmaxf(m, fabsf(v[i]));
    return m;
}

/* Q/src/quant.rs:74-105 */
int orc_q2_quantize(const float *values, uint8_t out[18]) {
    int st = require_block(values);
    if (st) return st;
    memset(out, 0, 18);
    float scale = fold_max_abs(values);
    if (scale == 0.0f) return ORC_OK;
    for (int i = 0; i < BLOCK_LEN; i++) {
        float n = values[i] / scale;
        int best = 0;
        for (int c = 1; c < 4; c++) /* min_by keeps the first minimum */
            if (total_cmp(fabsf(n - Q2_CODEBOOK[c]), fabsf(n - Q2_CODEBOOK[best])) < 0) best = c;
        out[2 + i / 4] |= (uint8_t)(best << ((i % 4) * 2));
    }
    uint16_t h = orc_f32_to_f16(scale);
    out[0] = h & 0xff;
    out[1] = h >> 8;
    return ORC_OK;
}

/* Q/src/quant.rs:144-168 */
int orc_q4_quantize(const float *values, uint8_t out[34]) {
    int st = require_block(values);
    if (st) return st;
    memset(out, 0, 34);
    float scale = fold_max_abs(values);
    if (scale == 0.0f) return ORC_OK;
    for (int i = 0; i < BLOCK_LEN; i++) {
        float n = values[i] / scale;
        n = n < -1.0f ? -1.0f : (n > 1.0f ? 1.0f : n);
        float r = roundf((n * 7.5f) + 7.5f); /* half away from zero */
        r = r < 0.0f ? 0.0f : (r > 15.0f ? 15.0f : r);
        out[2 + i / 2] |= (uint8_t)(((uint8_t)r) << ((i % 2) * 4));
    }
    uint16_t h = orc_f32_to_f16(scale);
    out[0] = h & 0xff;
    out[1] = h >> 8;
    return ORC_OK;
}

/* Q/src/quant.rs:47-61 */
int orc_a8_quantize(const float *values, float *scale_out, int8_t codes[64]) {
    int st = require_block(values);
    if (st) return st;
    float m = fold_max_abs(values);
    memset(codes, 0, 64);
    if (m == 0.0f) { *scale_out = 0.0f; return ORC_OK; }
    float scale = m / 127.0f;
    for (int i = 0; i < BLOCK_LEN; i++) {
        float r = rintf(values[i] / scale);
        r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
        codes[i] = (int8_t)r;
    }
    *scale_out = scale;
    return ORC_OK;
}

/* Q/src/quant.rs:123-140, 187-204: decode only rejects non-finite scales. */
int orc_q2_decode_check(const uint8_t b[18]) {
    return finite_f(orc_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)))) ? ORC_OK : ORC_ERR_INVALID_ARTIFACT;
}
int orc_q4_decode_check(const uint8_t b[34]) {
    return finite_f(orc_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)))) ? ORC_OK : ORC_ERR_INVALID_ARTIFACT;
}

/* Q/src/quant.rs:107-111 */
float orc_q2_value(const uint8_t b[18], size_t i) {
    unsigned code = (b[2 + i / 4] >> ((i % 4) * 2)) & 3u;
    return orc_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))) * Q2_CODEBOOK[code];
}
/* Q/src/quant.rs:171-175 */
float orc_q4_value(const uint8_t b[34], size_t i) {
    unsigned code = (b[2 + i / 2] >> ((i % 2) * 4)) & 0xfu;
    float n = ((float)code - 7.5f) / 7.5f;
    return orc_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))) * n;
}

/* ------------------------------------------------------------------ */
/* backend/cpu.rs                                                      */
/* ------------------------------------------------------------------ */
/* Q/src/backend/mod.rs:91-111 */
static int scale_value(orc_scale s, size_t index, float *out) {
    if (index >= s.len) return ORC_ERR_SHAPE;
    float v;
    if (s.kind == ORC_SCALE_F32) {
        v = ((const float *)s.data)[index];
    } else {
        const uint8_t *b = (const uint8_t *)s.data;
        v = orc_f16_to_f32((uint16_t)(b[2 * index] | (b[2 * index + 1] << 8)));
    }
    if (!finite_f(v)) return ORC_ERR_INVALID_ARTIFACT;
    *out = v;
    return ORC_OK;
}

/* Q/src/backend/cpu.rs:41-173 (same check order and error kinds). */
int orc_validate(const orc_matvec_op *op, size_t *bpr) {
    if (op->columns == 0 || op->rows == 0 || op->columns % BLOCK_LEN != 0) return ORC_ERR_SHAPE;
    if (op->input_len != op->columns) return ORC_ERR_SHAPE;
    if (op->s_in.kind != ORC_SCALE_NONE && op->s_in.len != op->columns) return ORC_ERR_SHAPE;
    if (op->s_out.kind != ORC_SCALE_NONE && op->s_out.len != op->rows) return ORC_ERR_SHAPE;
    if (op->bias && op->bias_len != op->rows) return ORC_ERR_SHAPE;
    size_t blocks = op->columns / BLOCK_LEN;
    size_t block_bytes;
    if (op->dtype == ORC_Q2B64) block_bytes = Q2_BLOCK_BYTES;
    else if (op->dtype == ORC_Q4B64) block_bytes = Q4_BLOCK_BYTES;
    else if (op->dtype == ORC_MIXED) block_bytes = 0;
    else return ORC_ERR_UNSUPPORTED_DTYPE;
    if (block_bytes) {
        if (op->n_segments) return ORC_ERR_INVALID_ARTIFACT;
        if (op->weights_len != op->rows * blocks * block_bytes) return ORC_ERR_SHAPE;
        *bpr = blocks;
        return ORC_OK;
    }
    if (op->n_segments == 0) return ORC_ERR_INVALID_ARTIFACT;
    uint64_t exp_row = 0, exp_off = 0;
    for (size_t g = 0; g < op->n_segments; g++) {
        const orc_segment *s = &op->segments[g];
        if (s->group_index != g || s->row_start != exp_row || s->row_end <= s->row_start ||
            s->row_end > op->rows || s->offset != exp_off)
            return ORC_ERR_INVALID_ARTIFACT;
        size_t sb;
        if (s->dtype == ORC_Q2B64) sb = Q2_BLOCK_BYTES;
        else if (s->dtype == ORC_Q4B64) sb = Q4_BLOCK_BYTES;
        else return ORC_ERR_INVALID_ARTIFACT;
        if (s->length != (s->row_end - s->row_start) * blocks * sb) return ORC_ERR_INVALID_ARTIFACT;
        exp_row = s->row_end;
        exp_off += s->length;
    }
    if (exp_row != op->rows || exp_off != op->weights_len) return ORC_ERR_SHAPE;
    *bpr = blocks;
    return ORC_OK;
}

/* Q/src/backend/cpu.rs:558-565 */
static float scalar_q2_dot(float scale, const uint8_t *codes, const float *x) {
    float sum = 0.0f;
    for (int i = 0; i < BLOCK_LEN; i++) {
        unsigned code = (codes[i / 4] >> ((i % 4) * 2)) & 3u;
        sum += scale * Q2_CODEBOOK[code] * x[i];
    }
    return sum;
}

/* Q/src/backend/cpu.rs:567-575 */
static float scalar_q4_dot(float scale, const uint8_t *codes, const float *x) {
    float sum = 0.0f;
    for (int i = 0; i < BLOCK_LEN; i++) {
        unsigned code = (codes[i / 2] >> ((i % 2) * 4)) & 0xfu;
        float n = ((float)code - 7.5f) / 7.5f;
        sum += scale * n * x[i];
    }
    return sum;
}

#if defined(__x86_64__)
/* Horizontal sum in lane order, as Q/src/backend/cpu.rs:577-584. */
__attribute__((target("avx2"))) static float hsum8(__m256 v) {
    float lanes[8];
    _mm256_storeu_ps(lanes, v);
    float s = 0.0f;
    for (int i = 0; i < 8; i++) s += lanes[i];
    return s;
}

/* Same arithmetic as Q/src/backend/cpu.rs:595-621: value = (2c-3)*(scale/3),
 * 8 lanes, lane i takes codes 16w+i and 16w+8+i of code word w. */
__attribute__((target("avx2"))) static float avx2_q2_dot(float scale, const uint8_t *codes, const float *x) {
    const __m256 factor = _mm256_set1_ps(scale / 3.0f);
    const __m256i three = _mm256_set1_epi32(3);
    const __m256i mask = _mm256_set1_epi32(3);
    const __m256i sh_lo = _mm256_setr_epi32(0, 2, 4, 6, 8, 10, 12, 14);
    const __m256i sh_hi = _mm256_setr_epi32(16, 18, 20, 22, 24, 26, 28, 30);
    __m256 acc = _mm256_setzero_ps();
    for (int w = 0; w < 4; w++) {
        int32_t word;
        memcpy(&word, codes + 4 * w, 4);
        __m256i bw = _mm256_set1_epi32(word);
        for (int half = 0; half < 2; half++) {
            __m256i c = _mm256_and_si256(_mm256_srlv_epi32(bw, half ? sh_hi : sh_lo), mask);
            __m256i centred = _mm256_sub_epi32(_mm256_add_epi32(c, c), three);
            __m256 val = _mm256_mul_ps(_mm256_cvtepi32_ps(centred), factor);
            __m256 xv = _mm256_loadu_ps(x + 16 * w + 8 * half);
            acc = _mm256_add_ps(acc, _mm256_mul_ps(val, xv));
        }
    }
    return hsum8(acc);
}

/* Same arithmetic as Q/src/backend/cpu.rs:633-658: value = (2c-15)*(scale/15),
 * lane i of group g takes element 16g+2i (low nibble) then 16g+2i+1. */
__attribute__((target("avx2"))) static float avx2_q4_dot(float scale, const uint8_t *codes, const float *x) {
    const __m256 factor = _mm256_set1_ps(scale / 15.0f);
    const __m256i fifteen = _mm256_set1_epi32(15);
    const __m128i nib = _mm_set1_epi8(0x0f);
    const __m256i fix = _mm256_setr_epi32(0, 1, 4, 5, 2, 3, 6, 7);
    __m256 acc = _mm256_setzero_ps();
    for (int g = 0; g < 4; g++) {
        __m128i bytes = _mm_loadl_epi64((const __m128i *)(codes + 8 * g));
        __m256i even = _mm256_cvtepu8_epi32(_mm_and_si128(bytes, nib));
        __m256i odd = _mm256_cvtepu8_epi32(_mm_and_si128(_mm_srli_epi16(bytes, 4), nib));
        __m256 lo = _mm256_loadu_ps(x + 16 * g);
        __m256 hi = _mm256_loadu_ps(x + 16 * g + 8);
        __m256 xe = _mm256_permutevar8x32_ps(_mm256_shuffle_ps(lo, hi, 0x88), fix);
        __m256 xo = _mm256_permutevar8x32_ps(_mm256_shuffle_ps(lo, hi, 0xdd), fix);
        __m256i cs[2] = {even, odd};
        __m256 xs[2] = {xe, xo};
        for (int p = 0; p < 2; p++) {
            __m256i centred = _mm256_sub_epi32(_mm256_add_epi32(cs[p], cs[p]), fifteen);
            __m256 val = _mm256_mul_ps(_mm256_cvtepi32_ps(centred), factor);
            acc = _mm256_add_ps(acc, _mm256_mul_ps(val, xs[p]));
        }
    }
    return hsum8(acc);
}
#endif

int orc_avx2_available(void) {
#if defined(__x86_64__)
    return __builtin_cpu_supports("avx2");
#else
    return 0;
#endif
}

float orc_packed_q2_dot(int profile, float scale, const uint8_t codes[16], const float x[64]) {
#if defined(__x86_64__)
    if (profile == ORC_PROFILE_AVX2) return avx2_q2_dot(scale, codes, x);
#endif
    return scalar_q2_dot(scale, codes, x);
}
float orc_packed_q4_dot(int profile, float scale, const uint8_t codes[32], const float x[64]) {
#if defined(__x86_64__)
    if (profile == ORC_PROFILE_AVX2) return avx2_q4_dot(scale, codes, x);
#endif
    return scalar_q4_dot(scale, codes, x);
}

/* Q/src/backend/cpu.rs:180-226 */
static int row_sum(int profile, int32_t dtype, const uint8_t *row, size_t blocks, const float *x,
                   float *out) {
    float sum = 0.0f;
    size_t bb = dtype == ORC_Q2B64 ? Q2_BLOCK_BYTES : Q4_BLOCK_BYTES;
    for (size_t b = 0; b < blocks; b++) {
        const uint8_t *blk = row + b * bb;
        float scale = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        if (!finite_f(scale)) return ORC_ERR_INVALID_ARTIFACT;
        sum += dtype == ORC_Q2B64 ? orc_packed_q2_dot(profile, scale, blk + 2, x + b * BLOCK_LEN)
                                  : orc_packed_q4_dot(profile, scale, blk + 2, x + b * BLOCK_LEN);
    }
    *out = sum;
    return ORC_OK;
}

/* Q/src/backend/mod.rs:58-66 */
static float activate(int32_t act, float v) { return act == 1 ? v / (1.0f + expf(-v)) : v; }

/* Q/src/backend/cpu.rs:228-240 */
static int corrected_input(const orc_matvec_op *op, float **out) {
    *out = NULL;
    if (op->s_in.kind == ORC_SCALE_NONE) return ORC_OK;
    float *c = (float *)malloc(op->columns * sizeof(float));
    for (size_t i = 0; i < op->columns; i++) {
        float s;
        int st = scale_value(op->s_in, i, &s);
        if (st) { free(c); return st; }
        c[i] = op->input[i] * s;
    }
    *out = c;
    return ORC_OK;
}

/* finish_row, Q/src/backend/cpu.rs:249-257 */
static int finish_row(const orc_matvec_op *op, size_t row, float sum, float *out) {
    sum += op->bias ? op->bias[row] : 0.0f;
    float so = 1.0f;
    if (op->s_out.kind != ORC_SCALE_NONE) {
        int st = scale_value(op->s_out, row, &so);
        if (st) return st;
    }
    sum *= so;
    *out = activate(op->activation, sum);
    return ORC_OK;
}

/* Q/src/backend/cpu.rs:242-310, restricted to rows [r0, r1). */
static int execute_rows(int profile, const orc_matvec_op *op, size_t blocks, const float *x,
                        float *output, size_t r0, size_t r1) {
    if (op->dtype != ORC_MIXED) {
        size_t rb = blocks * (op->dtype == ORC_Q2B64 ? Q2_BLOCK_BYTES : Q4_BLOCK_BYTES);
        for (size_t r = r0; r < r1; r++) {
            float s;
            int st = row_sum(profile, op->dtype, op->weights + r * rb, blocks, x, &s);
            if (!st) st = finish_row(op, r, s, &output[r]);
            if (st) return st;
        }
        return ORC_OK;
    }
    for (size_t g = 0; g < op->n_segments; g++) {
        const orc_segment *seg = &op->segments[g];
        size_t rb = blocks * (seg->dtype == ORC_Q2B64 ? Q2_BLOCK_BYTES : Q4_BLOCK_BYTES);
        const uint8_t *payload = op->weights + seg->offset;
        for (size_t r = seg->row_start; r < seg->row_end; r++) {
            if (r < r0 || r >= r1) continue;
            float s;
            int st = row_sum(profile, seg->dtype, payload + (r - seg->row_start) * rb, blocks, x, &s);
            if (!st) st = finish_row(op, r, s, &output[r]);
            if (st) return st;
        }
    }
    return ORC_OK;
}

/* Q/src/backend/cpu.rs:432-442 */
int orc_fused_matvec(int profile, const orc_matvec_op *op, float *output) {
    size_t blocks;
    int st = orc_validate(op, &blocks);
    if (st) return st;
    float *c;
    st = corrected_input(op, &c);
    if (st) return st;
    st = execute_rows(profile, op, blocks, c ? c : op->input, output, 0, op->rows);
    free(c);
    return st;
}

typedef struct {
    int profile;
    const orc_matvec_op *op;
    size_t blocks;
    const float *x;
    float *out;
    size_t r0, r1;
    int status;
} worker_arg;

static void *worker(void *p) {
    worker_arg *a = (worker_arg *)p;
    a->status = execute_rows(a->profile, a->op, a->blocks, a->x, a->out, a->r0, a->r1);
    return NULL;
}

int orc_fused_matvec_threads(int profile, const orc_matvec_op *op, float *output, int threads) {
    if (threads <= 1) return orc_fused_matvec(profile, op, output);
    size_t blocks;
    int st = orc_validate(op, &blocks);
    if (st) return st;
    float *c;
    st = corrected_input(op, &c);
    if (st) return st;
    pthread_t *tid = (pthread_t *)calloc((size_t)threads, sizeof(pthread_t));
    worker_arg *args = (worker_arg *)calloc((size_t)threads, sizeof(worker_arg));
    size_t per = (op->rows + (size_t)threads - 1) / (size_t)threads;
    for (int t = 0; t < threads; t++) {
        size_t r0 = (size_t)t * per, r1 = r0 + per;
        if (r0 > op->rows) r0 = op->rows;
        if (r1 > op->rows) r1 = op->rows;
        args[t] = (worker_arg){profile, op, blocks, c ? c : op->input, output, r0, r1, 0};
        pthread_create(&tid[t], NULL, worker, &args[t]);
    }
    for (int t = 0; t < threads; t++) {
        pthread_join(tid[t], NULL);
        if (args[t].status && !st) st = args[t].status;
    }
    free(tid);
    free(args);
    free(c);
    return st;
}

/* Q/src/backend/cpu.rs:373-380 */
static int same_scale(orc_scale a, orc_scale b) {
    if (a.kind != b.kind) return 0;
    if (a.kind == ORC_SCALE_NONE) return 1;
    if (a.len != b.len) return 0;
    size_t bytes = a.len * (a.kind == ORC_SCALE_F32 ? 4 : 2);
    return memcmp(a.data, b.data, bytes) == 0;
}

/* Q/src/backend/cpu.rs:444-472 */
int orc_fused_matvec_fanout(int profile, const orc_matvec_op *ops, size_t n,
                            float *const *outputs) {
    if (n == 0) return ORC_ERR_SHAPE;
    int share = 1;
    for (size_t i = 0; i < n; i++)
        if (ops[i].input_len != ops[0].input_len || ops[i].input != ops[0].input ||
            !same_scale(ops[i].s_in, ops[0].s_in))
            share = 0;
    if (!share) {
        for (size_t i = 0; i < n; i++) {
            int st = orc_fused_matvec(profile, &ops[i], outputs[i]);
            if (st) return st;
        }
        return ORC_OK;
    }
    size_t *blocks = (size_t *)malloc(n * sizeof(size_t));
    for (size_t i = 0; i < n; i++) {
        int st = orc_validate(&ops[i], &blocks[i]);
        if (st) { free(blocks); return st; }
    }
    float *c;
    int st = corrected_input(&ops[0], &c);
    for (size_t i = 0; !st && i < n; i++)
        st = execute_rows(profile, &ops[i], blocks[i], c ? c : ops[0].input, outputs[i], 0, ops[i].rows);
    free(c);
    free(blocks);
    return st;
}

/* Q/src/backend/cpu.rs:312-370 */
int orc_recovered_row(int32_t dtype, const uint8_t *w, size_t wlen, size_t columns, orc_scale s_in,
                      float s_out, float *output) {
    if (columns == 0 || columns % BLOCK_LEN) return ORC_ERR_SHAPE;
    if (s_in.len != columns || !finite_f(s_out)) return ORC_ERR_SHAPE;
    size_t bb;
    if (dtype == ORC_Q2B64) bb = Q2_BLOCK_BYTES;
    else if (dtype == ORC_Q4B64) bb = Q4_BLOCK_BYTES;
    else return ORC_ERR_UNSUPPORTED_DTYPE;
    if (wlen != columns / BLOCK_LEN * bb) return ORC_ERR_SHAPE;
    for (size_t b = 0; b < columns / BLOCK_LEN; b++) {
        const uint8_t *blk = w + b * bb;
        float scale = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        if (!finite_f(scale)) return ORC_ERR_INVALID_ARTIFACT;
        for (size_t lc = 0; lc < BLOCK_LEN; lc++) {
            float n;
            if (dtype == ORC_Q2B64) {
                n = Q2_CODEBOOK[(blk[2 + lc / 4] >> ((lc % 4) * 2)) & 3];
            } else {
                uint8_t p = blk[2 + lc / 2];
                unsigned code = (lc % 2 == 0) ? (p & 0x0f) : (p >> 4);
                n = ((float)code - 7.5f) / 7.5f;
            }
            size_t col = b * BLOCK_LEN + lc;
            float si;
            int st = scale_value(s_in, col, &si);
            if (st) return st;
            output[col] = scale * n * si * s_out;
        }
    }
    return ORC_OK;
}

/* Q/src/backend/cpu.rs:478-497 */
int orc_recovered_row_matvec(int profile, int32_t dtype, const uint8_t *w, size_t wlen,
                             const float *x, size_t len, float s_out, float *result) {
    if (len == 0 || len % BLOCK_LEN || !finite_f(s_out)) return ORC_ERR_SHAPE;
    for (size_t i = 0; i < len; i++)
        if (!finite_f(x[i])) return ORC_ERR_SHAPE;
    if (dtype != ORC_Q2B64 && dtype != ORC_Q4B64) return ORC_ERR_UNSUPPORTED_DTYPE;
    size_t bb = dtype == ORC_Q2B64 ? Q2_BLOCK_BYTES : Q4_BLOCK_BYTES;
    /* Rust slices the row by chunks_exact; a short buffer panics there. */
    if (wlen < len / BLOCK_LEN * bb) return ORC_ERR_SHAPE;
    float s;
    int st = row_sum(profile, dtype, w, len / BLOCK_LEN, x, &s);
    if (st) return st;
    *result = s * s_out;
    return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* reference.rs                                                        */
/* ------------------------------------------------------------------ */
static float silu(float v) { return v / (1.0f + expf(-v)); }

/* Q/src/reference.rs:18-34 */
static int matrix_contract(const float *v, size_t len, size_t rows, size_t cols) {
    if (rows == 0 || cols == 0 || len != rows * cols) return ORC_ERR_SHAPE;
    for (size_t i = 0; i < len; i++)
        if (!finite_f(v[i])) return ORC_ERR_INVALID_ARTIFACT;
    return ORC_OK;
}


/* Q/src/reference.rs:230-297 */
int orc_gated_delta_step(const float *q, const float *k, const float *v, const float *log_decay,
                         const float *beta, float *state, size_t heads, size_t kd, size_t vd,
                         float *out) {
    int st;
    if ((st = matrix_contract(q, heads * kd, heads, kd))) return st;
    if ((st = matrix_contract(k, heads * kd, heads, kd))) return st;
    if ((st = matrix_contract(v, heads * vd, heads, vd))) return st;
    size_t n = heads * kd * vd;
    for (size_t i = 0; i < n; i++)
        if (!finite_f(state[i])) return ORC_ERR_SHAPE;
    for (size_t h = 0; h < heads; h++)
        if (!finite_f(log_decay[h]) || !finite_f(beta[h])) return ORC_ERR_SHAPE;
    const float qscale = 1.0f / sqrtf((float)kd);
    for (size_t h = 0; h < heads; h++) {
        const float *qh = q + h * kd, *kh = k + h * kd, *vh = v + h * vd;
        float sq = 0.0f, sk = 0.0f;
        for (size_t i = 0; i < kd; i++) sq += qh[i] * qh[i];
        for (size_t i = 0; i < kd; i++) sk += kh[i] * kh[i];
        float qinv = 1.0f / sqrtf(sq + L2_EPSILON);
        float kinv = 1.0f / sqrtf(sk + L2_EPSILON);
        float *S = state + h * kd * vd;
        float decay = expf(log_decay[h]);
        for (size_t i = 0; i < kd * vd; i++) S[i] *= decay;
        for (size_t j = 0; j < vd; j++) {
            float mem = 0.0f;
            for (size_t i = 0; i < kd; i++) mem += S[i * vd + j] * kh[i] * kinv;
            float delta = (vh[j] - mem) * beta[h];
            for (size_t i = 0; i < kd; i++) S[i * vd + j] += kh[i] * kinv * delta;
        }
        for (size_t j = 0; j < vd; j++) {
            float o = 0.0f;
            for (size_t i = 0; i < kd; i++) o += S[i * vd + j] * qh[i] * qinv * qscale;
            out[h * vd + j] = o;
        }
    }
    return ORC_OK;
}

/* Q/src/reference.rs:302-373 */
int orc_gated_delta_step_f16_state(const float *q, const float *k, const float *v,
                                   const float *log_decay, const float *beta, uint16_t *state,
                                   size_t heads, size_t kd, size_t vd, float *out) {
    int st;
    if ((st = matrix_contract(q, heads * kd, heads, kd))) return st;
    if ((st = matrix_contract(k, heads * kd, heads, kd))) return st;
    if ((st = matrix_contract(v, heads * vd, heads, vd))) return st;
    size_t n = heads * kd * vd;
    for (size_t i = 0; i < n; i++)
        if (!finite_f(orc_f16_to_f32(state[i]))) return ORC_ERR_SHAPE;
    for (size_t h = 0; h < heads; h++)
        if (!finite_f(log_decay[h]) || !finite_f(beta[h])) return ORC_ERR_SHAPE;
    const float qscale = 1.0f / sqrtf((float)kd);
    for (size_t h = 0; h < heads; h++) {
        const float *qh = q + h * kd, *kh = k + h * kd, *vh = v + h * vd;
        float sq = 0.0f, sk = 0.0f;
        for (size_t i = 0; i < kd; i++) sq += qh[i] * qh[i];
        for (size_t i = 0; i < kd; i++) sk += kh[i] * kh[i];
        float qinv = 1.0f / sqrtf(sq + L2_EPSILON);
        float kinv = 1.0f / sqrtf(sk + L2_EPSILON);
        uint16_t *S = state + h * kd * vd;
        float decay = expf(log_decay[h]);
        for (size_t i = 0; i < kd * vd; i++) S[i] = orc_f32_to_f16(orc_f16_to_f32(S[i]) * decay);
        for (size_t j = 0; j < vd; j++) {
            float mem = 0.0f;
            for (size_t i = 0; i < kd; i++) mem += orc_f16_to_f32(S[i * vd + j]) * kh[i] * kinv;
            float delta = (vh[j] - mem) * beta[h];
            for (size_t i = 0; i < kd; i++)
                S[i * vd + j] = orc_f32_to_f16(orc_f16_to_f32(S[i * vd + j]) + kh[i] * kinv * delta);
        }
        for (size_t j = 0; j < vd; j++) {
            float o = 0.0f;
            for (size_t i = 0; i < kd; i++) o += orc_f16_to_f32(S[i * vd + j]) * qh[i] * qinv * qscale;
            out[h * vd + j] = o;
        }
    }
    return ORC_OK;
}

/* Q/src/reference.rs:377-415 */
int orc_gated_delta_sequence(const float *q, const float *k, const float *v, const float *log_decay,
                             const float *beta, float *state, size_t tokens, size_t heads,
                             size_t kd, size_t vd, float *out) {
    int st;
    if ((st = matrix_contract(q, tokens * heads * kd, tokens, heads * kd))) return st;
    if ((st = matrix_contract(k, tokens * heads * kd, tokens, heads * kd))) return st;
    if ((st = matrix_contract(v, tokens * heads * vd, tokens, heads * vd))) return st;
    if ((st = matrix_contract(log_decay, tokens * heads, tokens, heads))) return st;
    if ((st = matrix_contract(beta, tokens * heads, tokens, heads))) return st;
    for (size_t t = 0; t < tokens; t++) {
        st = orc_gated_delta_step(q + t * heads * kd, k + t * heads * kd, v + t * heads * vd,
                                  log_decay + t * heads, beta + t * heads, state, heads, kd, vd,
                                  out + t * heads * vd);
        if (st) return st;
    }
    return ORC_OK;
}

/* Q/src/reference.rs:38-62 */
int orc_rms_norm_1p_weight(const float *x, size_t rows, size_t cols, const float *w, float eps,
                           float *out) {
    int st = matrix_contract(x, rows * cols, rows, cols);
    if (st) return st;
    if (!finite_f(eps) || eps <= 0.0f) return ORC_ERR_SHAPE;
    for (size_t r = 0; r < rows; r++) {
        const float *row = x + r * cols;
        float var = 0.0f;
        for (size_t c = 0; c < cols; c++) var += row[c] * row[c];
        var = var / (float)cols;
        float inv = 1.0f / sqrtf(var + eps);
        for (size_t c = 0; c < cols; c++) out[r * cols + c] = row[c] * inv * (1.0f + w[c]);
    }
    return ORC_OK;
}

/* Q/src/reference.rs:66-93 */
int orc_rms_norm_gated(const float *x, const float *gate, size_t rows, size_t cols, const float *w,
                       float eps, float *out) {
    int st = matrix_contract(x, rows * cols, rows, cols);
    if (!st) st = matrix_contract(gate, rows * cols, rows, cols);
    if (st) return st;
    if (!finite_f(eps) || eps <= 0.0f) return ORC_ERR_SHAPE;
    for (size_t r = 0; r < rows; r++) {
        const float *row = x + r * cols;
        float var = 0.0f;
        for (size_t c = 0; c < cols; c++) var += row[c] * row[c];
        var = var / (float)cols;
        float inv = 1.0f / sqrtf(var + eps);
        for (size_t c = 0; c < cols; c++)
            out[r * cols + c] = row[c] * inv * w[c] * silu(gate[r * cols + c]);
    }
    return ORC_OK;
}

/* Q/src/reference.rs:96-112 */
int orc_swiglu(const float *gate, const float *up, size_t n, float *out) {
    if (n == 0) return ORC_ERR_SHAPE;
    for (size_t i = 0; i < n; i++)
        if (!finite_f(gate[i]) || !finite_f(up[i])) return ORC_ERR_SHAPE;
    for (size_t i = 0; i < n; i++) out[i] = silu(gate[i]) * up[i];
    return ORC_OK;
}

/* Q/src/reference.rs:159-187 */
int orc_causal_conv_silu_update(const float *input, float *state, const float *weight,
                                size_t channels, size_t kernel, float *out) {
    int st = matrix_contract(state, channels * kernel, channels, kernel);
    if (!st) st = matrix_contract(weight, channels * kernel, channels, kernel);
    if (st) return st;
    for (size_t c = 0; c < channels; c++)
        if (!finite_f(input[c])) return ORC_ERR_SHAPE;
    for (size_t c = 0; c < channels; c++) {
        float *s = state + c * kernel;
        memmove(s, s + 1, (kernel - 1) * sizeof(float));
        s[kernel - 1] = input[c];
        float sum = 0.0f;
        for (size_t i = 0; i < kernel; i++) sum += s[i] * weight[c * kernel + i];
        out[c] = silu(sum);
    }
    return ORC_OK;
}

/* Q/src/reference.rs:115-155 */
int orc_apply_partial_rope(float *q, float *k, size_t qh, size_t kh, size_t hd, size_t rd,
                           uint64_t position, float theta) {
    int st = matrix_contract(q, qh * hd, qh, hd);
    if (!st) st = matrix_contract(k, kh * hd, kh, hd);
    if (st) return st;
    if (rd == 0 || rd > hd || rd % 2 || !finite_f(theta) || theta <= 0.0f) return ORC_ERR_SHAPE;
    size_t half = rd / 2;
    float *cs = (float *)malloc(half * sizeof(float)), *sn = (float *)malloc(half * sizeof(float));
    for (size_t i = 0; i < half; i++) {
        float invf = powf(theta, -((float)(2 * i)) / (float)rd);
        float angle = (float)position * invf;
        cs[i] = cosf(angle);
        sn[i] = sinf(angle);
    }
    float *arrs[2] = {q, k};
    size_t nh[2] = {qh, kh};
    for (int a = 0; a < 2; a++)
        for (size_t h = 0; h < nh[a]; h++) {
            float *head = arrs[a] + h * hd;
            for (size_t i = 0; i < half; i++) {
                float l = head[i], r = head[i + half];
                head[i] = l * cs[i] - r * sn[i];
                head[i + half] = r * cs[i] + l * sn[i];
            }
        }
    free(cs);
    free(sn);
    return ORC_OK;
}

/* Q/src/reference.rs:420-499 */
int orc_grouped_query_attention(const float *q, const float *k, const float *v, size_t qh,
                                size_t kvh, size_t qt, size_t kvt, size_t hd, size_t q0,
                                float *out) {
    int st = matrix_contract(q, qh * qt * hd, qh, qt * hd);
    if (!st) st = matrix_contract(k, kvh * kvt * hd, kvh, kvt * hd);
    if (!st) st = matrix_contract(v, kvh * kvt * hd, kvh, kvt * hd);
    if (st) return st;
    if (kvh == 0 || qh % kvh || q0 + qt > kvt) return ORC_ERR_SHAPE;
    size_t groups = qh / kvh;
    float scale = 1.0f / sqrtf((float)hd);
    memset(out, 0, qt * qh * hd * sizeof(float));
    float *scores = (float *)malloc(kvt * sizeof(float));
    for (size_t t = 0; t < qt; t++) {
        size_t avail = q0 + t + 1;
        for (size_t h = 0; h < qh; h++) {
            size_t kvhh = h / groups;
            const float *qr = q + (h * qt + t) * hd;
            for (size_t j = 0; j < avail; j++) {
                const float *kr = k + (kvhh * kvt + j) * hd;
                float s = 0.0f;
                for (size_t d = 0; d < hd; d++) s += qr[d] * kr[d];
                scores[j] = s * scale;
            }
            float m = -INFINITY;
            for (size_t j = 0; j < avail; j++) m = fmaxf(m, scores[j]);
            float den = 0.0f;
            for (size_t j = 0; j < avail; j++) { scores[j] = expf(scores[j] - m); den += scores[j]; }
            if (!finite_f(den) || den <= 0.0f) { free(scores); return ORC_ERR_INVALID_ARTIFACT; }
            float *o = out + (t * qh + h) * hd;
            for (size_t j = 0; j < avail; j++) {
                const float *vr = v + (kvhh * kvt + j) * hd;
                for (size_t d = 0; d < hd; d++) o[d] += scores[j] / den * vr[d];
            }
        }
    }
    free(scores);
    return ORC_OK;
}

/* Q/src/reference.rs:502-515 */
int orc_sigmoid_gate(float *values, const float *gate, size_t n) {
    if (n == 0) return ORC_ERR_SHAPE;
    for (size_t i = 0; i < n; i++)
        if (!finite_f(values[i]) || !finite_f(gate[i])) return ORC_ERR_SHAPE;
    for (size_t i = 0; i < n; i++) values[i] *= 1.0f / (1.0f + expf(-gate[i]));
    return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* decoder.rs glue                                                     */
/* ------------------------------------------------------------------ */
/* Q/src/decoder.rs:29-35 */
float orc_softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

/* Q/src/decoder.rs:47-65 */
int orc_repeat_heads(const float *values, size_t heads, size_t dim, size_t repeats, float *out) {
    if (heads == 0 || dim == 0 || repeats == 0) return ORC_ERR_SHAPE;
    for (size_t h = 0; h < heads; h++)
        for (size_t r = 0; r < repeats; r++)
            memcpy(out + (h * repeats + r) * dim, values + h * dim, dim * sizeof(float));
    return ORC_OK;
}

/* Q/src/decoder.rs:881-902 */
void orc_gdn_gates(const float *a, const float *b, const float *a_log, const float *dt_bias,
                   size_t heads, float *log_decay, float *beta) {
    for (size_t h = 0; h < heads; h++) {
        beta[h] = 1.0f / (1.0f + expf(-b[h]));
        log_decay[h] = -expf(a_log[h]) * orc_softplus(a[h] + dt_bias[h]);
    }
}

/* ------------------------------------------------------------------ */
/* sampler.rs                                                          */
/* ------------------------------------------------------------------ */
/* Q/src/sampler.rs:149-174 */
uint32_t orc_pcg32_next_u32(orc_pcg32 *g) {
    uint64_t old = g->state;
    g->state = old * 6364136223846793005ULL + 1442695040888963407ULL;
    uint32_t shifted = (uint32_t)(((old >> 18) ^ old) >> 27);
    uint32_t rot = (uint32_t)(old >> 59);
    return (shifted >> rot) | (shifted << ((32 - rot) & 31));
}
void orc_pcg32_init(orc_pcg32 *g, uint64_t seed) {
    g->state = seed + 0x853c49e6748fea9bULL;
    (void)orc_pcg32_next_u32(g);
}
float orc_pcg32_next_f32(orc_pcg32 *g) {
    return (float)((double)orc_pcg32_next_u32(g) / ((double)UINT32_MAX + 1.0));
}

/* argmax with total_cmp, later index wins (Q/src/engine.rs:906-913). */
int orc_greedy_token(const float *logits, size_t n, uint32_t *token) {
    if (n == 0) return ORC_ERR_INVALID_ARTIFACT;
    size_t best = 0;
    for (size_t i = 1; i < n; i++)
        if (total_cmp(logits[i], logits[best]) >= 0) best = i;
    *token = (uint32_t)best;
    return ORC_OK;
}

typedef struct { size_t token; float value; } cand;
static int cand_cmp(const void *a, const void *b) {
    const cand *l = (const cand *)a, *r = (const cand *)b;
    int c = total_cmp(r->value, l->value); /* descending value */
    if (c) return c;
    return (r->token > l->token) - (r->token < l->token); /* later token first */
}

/* Q/src/sampler.rs:65-144 */
int orc_sample_with_draw(const float *logits, size_t n, float temperature, size_t top_k,
                         float top_p, float draw, size_t *token) {
    if (n == 0) return ORC_ERR_INVALID_ARTIFACT;
    for (size_t i = 0; i < n; i++)
        if (!finite_f(logits[i])) return ORC_ERR_INVALID_ARTIFACT;
    if (!finite_f(draw) || !(draw >= 0.0f && draw < 1.0f)) return ORC_ERR_INVALID_ARTIFACT;
    if (temperature == 0.0f) {
        uint32_t t;
        orc_greedy_token(logits, n, &t);
        *token = t;
        return ORC_OK;
    }
    float invt = 1.0f / temperature;
    if (!finite_f(invt)) return ORC_ERR_INVALID_ARTIFACT;
    cand *c = (cand *)malloc(n * sizeof(cand));
    for (size_t i = 0; i < n; i++) {
        c[i].token = i;
        c[i].value = logits[i] * invt;
        if (!finite_f(c[i].value)) { free(c); return ORC_ERR_INVALID_ARTIFACT; }
    }
    qsort(c, n, sizeof(cand), cand_cmp);
    size_t len = n;
    if (top_k > 0 && top_k < len) len = top_k;
    float m = c[0].value, norm = 0.0f;
    for (size_t i = 0; i < len; i++) { c[i].value = expf(c[i].value - m); norm += c[i].value; }
    if (!finite_f(norm) || norm <= 0.0f) { free(c); return ORC_ERR_INVALID_ARTIFACT; }
    float cum = 0.0f;
    size_t nuc = len;
    for (size_t i = 0; i < len; i++) {
        cum += c[i].value;
        if (cum >= top_p * norm) { nuc = i + 1; break; }
    }
    float total = 0.0f;
    for (size_t i = 0; i < nuc; i++) total += c[i].value;
    float thr = draw * total;
    cum = 0.0f;
    for (size_t i = 0; i < nuc; i++) {
        cum += c[i].value;
        if (thr <= cum) { *token = c[i].token; free(c); return ORC_OK; }
    }
    *token = c[nuc - 1].token;
    free(c);
    return ORC_OK;
}

/* Q/src/engine.rs:915-963 (full-logits branch). */
int orc_verify_greedy_mtp(const float *draft, const float *target, const float *bonus,
                          size_t drafts, size_t vocab, uint32_t *next_token, uint32_t *verified,
                          uint32_t *accepted, uint32_t *n_accepted) {
    uint32_t nacc = 0, ver = 0;
    for (size_t i = 0; i < drafts; i++) {
        uint32_t d, t;
        int st = orc_greedy_token(draft + i * vocab, vocab, &d);
        if (!st) st = orc_greedy_token(target + i * vocab, vocab, &t);
        if (st) return st;
        ver++;
        if (d != t) {
            *next_token = t;
            *verified = ver;
            *n_accepted = nacc;
            return ORC_OK;
        }
        accepted[nacc++] = d;
    }
    if (!bonus) return ORC_ERR_INVALID_ARTIFACT;
    int st = orc_greedy_token(bonus, vocab, next_token);
    *verified = ver;
    *n_accepted = nacc;
    return st;
}

/* Temperature-scaled softmax in the sampler's arithmetic (scale by 1/T,
 * subtract the max, expf, sequential sum). */
static int softmax_t(const float *logits, size_t n, float invt, float *p) {
    float m = -INFINITY;
    for (size_t i = 0; i < n; i++) { p[i] = logits[i] * invt; m = fmaxf(m, p[i]); }
    float z = 0.0f;
    for (size_t i = 0; i < n; i++) { p[i] = expf(p[i] - m); z += p[i]; }
    if (!finite_f(z) || z <= 0.0f) return ORC_ERR_INVALID_ARTIFACT;
    for (size_t i = 0; i < n; i++) p[i] = p[i] / z;
    return ORC_OK;
}

static size_t cumulative_pick(const float *w, size_t n, float draw) {
    float total = 0.0f;
    for (size_t i = 0; i < n; i++) total += w[i];
    float thr = draw * total, cum = 0.0f;
    size_t last = 0;
    for (size_t i = 0; i < n; i++) {
        if (w[i] > 0.0f) last = i;
        cum += w[i];
        if (w[i] > 0.0f && thr <= cum) return i;
    }
    return last;
}

/* Speculative rejection sampling (Leviathan et al. 2023 / Chen et al. 2023):
 * draft i is accepted iff u_i * q(d_i) < p(d_i); on the first rejection the
 * replacement is drawn from norm(max(0, p - q)) with the next draw; if every
 * draft is accepted the bonus token is drawn from the bonus distribution.
 * Draws come from the crate's Pcg32 (Q/src/sampler.rs:149-174); the
 * cumulative search follows Q/src/sampler.rs:134-143. No crate counterpart. */
int orc_mtp_accept_sample(const float *draft, const float *target, const float *bonus,
                          const uint32_t *tokens, size_t drafts, size_t vocab, float temperature,
                          orc_pcg32 *rng, uint32_t *next_token, uint32_t *n_accepted) {
    return orc_mtp_accept_sample_restricted(draft, NULL, vocab, target, bonus, tokens, drafts, vocab,
                                            temperature, rng, next_token, n_accepted);
}

/* The same with restricted draft rows (DraftDistribution::Restricted,
 * Q/src/engine.rs:151-200): draft row i holds `draft_n` scores for the
 * strictly increasing token IDs `draft_ids` (Q/src/decoder.rs:597-608 rules);
 * q is their temperature softmax and 0 for every other token. draft_ids NULL
 * means a full draft row (draft_n == vocab). */
int orc_mtp_accept_sample_restricted(const float *draft, const uint32_t *draft_ids, size_t draft_n,
                                     const float *target, const float *bonus, const uint32_t *tokens,
                                     size_t drafts, size_t vocab, float temperature, orc_pcg32 *rng,
                                     uint32_t *next_token, uint32_t *n_accepted) {
    if (!(temperature > 0.0f) || !finite_f(temperature) || vocab == 0) return ORC_ERR_INVALID_ARTIFACT;
    if (draft_n == 0 || (!draft_ids && draft_n != vocab)) return ORC_ERR_SHAPE;
    if (draft_ids)
        for (size_t j = 0; j < draft_n; j++)
            if (draft_ids[j] >= vocab || (j && draft_ids[j - 1] >= draft_ids[j])) return ORC_ERR_SHAPE;
    float invt = 1.0f / temperature;
    float *p = (float *)malloc(vocab * sizeof(float));
    float *q = (float *)calloc(vocab, sizeof(float));
    float *qr = (float *)malloc(draft_n * sizeof(float));
    int st = ORC_OK;
    uint32_t acc = 0;
    for (size_t i = 0; i < drafts; i++) {
        if ((st = softmax_t(target + i * vocab, vocab, invt, p))) goto done;
        if ((st = softmax_t(draft + i * draft_n, draft_n, invt, qr))) goto done;
        for (size_t j = 0; j < draft_n; j++) q[draft_ids ? draft_ids[j] : j] = qr[j];
        uint32_t d = tokens[i];
        if (d >= vocab) { st = ORC_ERR_SHAPE; goto done; }
        float u = orc_pcg32_next_f32(rng);
        if (u * q[d] < p[d]) {
            acc++;
            for (size_t j = 0; j < draft_n; j++) q[draft_ids ? draft_ids[j] : j] = 0.0f;
            continue;
        }
        for (size_t t = 0; t < vocab; t++) { float r = p[t] - q[t]; p[t] = r > 0.0f ? r : 0.0f; }
        float u2 = orc_pcg32_next_f32(rng);
        *next_token = (uint32_t)cumulative_pick(p, vocab, u2);
        *n_accepted = acc;
        goto done;
    }
    if (!bonus) { st = ORC_ERR_INVALID_ARTIFACT; goto done; }
    if ((st = softmax_t(bonus, vocab, invt, p))) goto done;
    {
        float u = orc_pcg32_next_f32(rng);
        *next_token = (uint32_t)cumulative_pick(p, vocab, u);
        *n_accepted = acc;
    }
done:
    free(p);
    free(q);
    free(qr);
    return st;
}
