// Paged mixed Q2/Q4 KV cache on gfx950: token packing, page demotion and
// split-KV grouped-query attention for 1..5 query rows.
//
// Page format (Q/src/kv_cache.rs:280-300, :394-429): a page holds up to
// page_tokens tokens, token-major; each token is [K heads, V heads] as
// canonical Q4_B64 (34 B) or Q2_B64 (18 B) blocks of 64 values. A page is
// wholly Q2 or Q4. Logical page p is described by {precision (0 = Q2, else
// Q4), physical_slot, tokens, first_token}; its bytes live at
// pool + physical_slot * page_bytes in the Q2 or Q4 pool.
//
//  * ctox_kv_pack_q4_gfx950: quantize token rows of K and V into a Q4 page,
//    bit-exact with Q4Block64::quantize (Q/src/quant.rs:144-168): one wave per
//    64-value block, f32 max-abs, code = round(clamp(v / max) * 7.5 + 7.5)
//    with unfused multiply and add, fp16 scale rounded to nearest even.
//  * ctox_kv_demote_gfx950: rewrite a Q4 page as Q2. Q/src/kv_cache.rs:206-226
//    dequantizes and requantizes. A non-zero Q4 block always holds an extreme
//    code (its max-abs element maps to exactly +-1), so the requantized scale
//    is the same fp16 value and the nearest Q2 level of (c - 7.5) / 7.5 is
//    c <= 2 -> 0, <= 7 -> 1, <= 12 -> 2, else 3 (no level sits on a midpoint).
//    A block whose fp16 scale is zero dequantizes to zeros and requantizes to
//    an all-zero block.
//  * ctox_paged_gqa_partial_gfx950 / ctox_paged_gqa_combine_gfx950: the
//    attention of Q/src/reference.rs:420-499 over the dequantized pages
//    (Q/src/kv_cache.rs:579-605 flattens them for that oracle), split over the
//    token axis. One workgroup = one KV head x one token split; its four waves
//    take contiguous runs of 16-token tiles and run fp32 MFMA 16x16x4:
//      S^T = K Q^T : A = K (16 tokens x 4 dims; lane group g walks head-dim
//                    block g, so each lane dequantizes one 64-value block),
//                    B = Q^T (the group's G * rows query vectors, 16 per tile).
//      O^T += V^T P^T : the C layout of S^T hands lane group g tokens 4g..4g+3,
//                    which is exactly the k index P^T needs at step s = 0..3,
//                    so probabilities never leave registers.
//    Online softmax state (max, denominator) is per lane (one query per lane
//    per 16-query tile). Waves merge in LDS; splits merge in the combine
//    kernel. Causality: query row t sees tokens 0 ..= tokens - rows + t.
#include <hip/hip_runtime.h>

#include "kernel_args.h"

typedef float pa_v4f __attribute__((ext_vector_type(4)));

#define PA_HD 256  // head dim: four 64-value blocks, one per MFMA lane group

__device__ __forceinline__ float pa_half(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// ---------------------------------------------------------------------------
// pack
// ---------------------------------------------------------------------------
#pragma clang fp contract(off)
extern "C" __global__ __launch_bounds__(64) void ctox_kv_pack_q4_gfx950(KvPackArgs a) {
    const uint32_t lane = threadIdx.x, blk = blockIdx.x, tok = blockIdx.y;
    const uint32_t idx = blk * 64 + lane;
    const size_t row = (size_t)tok * a.component_values;
    const float v = idx < a.component_values ? a.keys[row + idx] : a.values[row + idx - a.component_values];
    float m = fabsf(v);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    uint32_t code = 0;
    if (m != 0.0f) {
        float n = v / m;  // correctly rounded division (HIP's default for f32)
        n = fminf(1.0f, fmaxf(-1.0f, n));
        const float sel = n * 7.5f + 7.5f;  // contraction is off in this file: two roundings
        code = (uint32_t)fminf(15.0f, fmaxf(0.0f, roundf(sel)));
    }
    const uint32_t hi = __shfl_down(code, 1);
    uint8_t *dst = a.q4_pages + (size_t)a.physical_slot * a.q4_page_bytes +
                   (size_t)(a.first_token_in_page + tok) * a.q4_token_bytes + (size_t)blk * 34;
    if ((lane & 1) == 0) dst[2 + lane / 2] = (uint8_t)(code | (hi << 4));
    if (lane == 0) {
        const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)m);  // round to nearest even
        dst[0] = (uint8_t)h;
        dst[1] = (uint8_t)(h >> 8);
    }
}
#pragma clang fp contract(fast)

// ---------------------------------------------------------------------------
// demote: one thread per output Q2 code byte (16 per block), block-major.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t pa_q4_to_q2(uint32_t c) { return c <= 2 ? 0u : c <= 7 ? 1u : c <= 12 ? 2u : 3u; }

extern "C" __global__ __launch_bounds__(256) void ctox_kv_demote_gfx950(KvDemoteArgs a) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.blocks * 16) return;
    const uint64_t blk = i >> 4;
    const uint32_t j = (uint32_t)(i & 15);
    const uint8_t *src = a.q4_page + blk * 34;
    uint8_t *dst = a.q2_page + blk * 18;
    const uint32_t sbits = (uint32_t)src[0] | ((uint32_t)src[1] << 8);
    const bool zero = (sbits & 0x7fffu) == 0;
    const uint32_t b0 = src[2 + 2 * j], b1 = src[3 + 2 * j];
    const uint32_t out = zero ? 0u
                              : pa_q4_to_q2(b0 & 15) | (pa_q4_to_q2(b0 >> 4) << 2) | (pa_q4_to_q2(b1 & 15) << 4) |
                                    (pa_q4_to_q2(b1 >> 4) << 6);
    dst[2 + j] = (uint8_t)out;
    if (j == 0) {
        dst[0] = zero ? 0 : src[0];
        dst[1] = zero ? 0 : src[1];
    }
}

// ---------------------------------------------------------------------------
// attention
// ---------------------------------------------------------------------------
struct PaToken {
    const uint8_t *run;  // first byte of the token (NULL if the token is absent)
    uint32_t q4;         // 1 = Q4 page, 0 = Q2 page
};

// Resolve logical token j through the page descriptors (Q/src/kv_cache.rs:558-575
// page views; tokens outside a page's [first_token, first_token + tokens) are absent).
__device__ __forceinline__ PaToken pa_token(const GqaArgs &a, uint32_t j) {
    PaToken t{nullptr, 0};
    if (j >= a.tokens) return t;
    const uint32_t p = j / a.page_tokens;
    if (p >= a.page_count) return t;
    const PagedKvDesc d = a.desc[p];
    if (j < d.first_token || j - d.first_token >= d.tokens) return t;
    const uint32_t tip = j - d.first_token;
    t.q4 = d.precision != 0;
    t.run = t.q4 ? a.q4 + (size_t)d.physical_slot * a.q4_page_bytes + (size_t)tip * a.q4_token_bytes
                 : a.q2 + (size_t)d.physical_slot * a.q2_page_bytes + (size_t)tip * a.q2_token_bytes;
    return t;
}

__device__ __forceinline__ uint32_t pa_ld32(const uint8_t *p) { return *(const uint32_t *)p; }
__device__ __forceinline__ uint32_t pa_ld16(const uint8_t *p) { return *(const uint16_t *)p; }

// K operand: 64 dequantized values of head-dim block g of one token's K head h.
// Values are scale * (2c - 15) / 15 (Q4) or scale * (2c - 3) / 3 (Q2), formed as
// one fused multiply-add per value.
__device__ __forceinline__ void pa_load_k(const PaToken &t, uint32_t h, uint32_t g, float kv[64]) {
    if (!t.run) {
#pragma unroll
        for (int e = 0; e < 64; e++) kv[e] = 0.0f;
        return;
    }
    if (t.q4) {
        const uint8_t *blk = t.run + (h * 4 + g) * 34;  // 2-byte aligned
        const float s = pa_half(pa_ld16(blk));
        const uintptr_t c = (uintptr_t)(blk + 2);
        const uint8_t *al = (const uint8_t *)(c & ~(uintptr_t)3);
        const uint32_t sh = (uint32_t)(c & 3);
        uint32_t w[9];
#pragma unroll
        for (int i = 0; i < 8; i++) w[i] = pa_ld32(al + 4 * i);
        w[8] = sh ? pa_ld32(al + 32) : 0u;  // only inside the block when shifted
        const float k2 = s * (2.0f / 15.0f);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t u = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
#pragma unroll
            for (int n = 0; n < 8; n++) kv[8 * i + n] = fmaf((float)((u >> (4 * n)) & 15u), k2, -s);
        }
    } else {
        const uint8_t *blk = t.run + (h * 4 + g) * 18;
        const float s = pa_half(pa_ld16(blk));
        const uintptr_t c = (uintptr_t)(blk + 2);
        const uint8_t *al = (const uint8_t *)(c & ~(uintptr_t)3);
        const uint32_t sh = (uint32_t)(c & 3);
        uint32_t w[5];
#pragma unroll
        for (int i = 0; i < 4; i++) w[i] = pa_ld32(al + 4 * i);
        w[4] = sh ? pa_ld32(al + 16) : 0u;
        const float k2 = s * (2.0f / 3.0f);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t u = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
#pragma unroll
            for (int n = 0; n < 16; n++) kv[16 * i + n] = fmaf((float)((u >> (2 * n)) & 3u), k2, -s);
        }
    }
}

// V operand: head-dim values 16 * li .. 16 * li + 15 of one token's V head h
// (block li / 4, quarter li % 4).
__device__ __forceinline__ void pa_load_v(const PaToken &t, uint32_t vrun_blocks, uint32_t h, uint32_t li,
                                          float vv[16]) {
    if (!t.run) {
#pragma unroll
        for (int e = 0; e < 16; e++) vv[e] = 0.0f;
        return;
    }
    const uint32_t b = vrun_blocks + h * 4 + li / 4, q = li & 3;
    if (t.q4) {
        const uint8_t *blk = t.run + b * 34;
        const float s = pa_half(pa_ld16(blk));
        const uintptr_t c = (uintptr_t)(blk + 2 + 8 * q);
        const uint8_t *al = (const uint8_t *)(c & ~(uintptr_t)3);
        const uint32_t sh = (uint32_t)(c & 3);
        const uint32_t w0 = pa_ld32(al), w1 = pa_ld32(al + 4), w2 = sh ? pa_ld32(al + 8) : 0u;
        const uint32_t u0 = __builtin_amdgcn_alignbyte(w1, w0, sh), u1 = __builtin_amdgcn_alignbyte(w2, w1, sh);
        const float k2 = s * (2.0f / 15.0f);
#pragma unroll
        for (int n = 0; n < 8; n++) {
            vv[n] = fmaf((float)((u0 >> (4 * n)) & 15u), k2, -s);
            vv[8 + n] = fmaf((float)((u1 >> (4 * n)) & 15u), k2, -s);
        }
    } else {
        const uint8_t *blk = t.run + b * 18;
        const float s = pa_half(pa_ld16(blk));
        const uintptr_t c = (uintptr_t)(blk + 2 + 4 * q);
        const uint8_t *al = (const uint8_t *)(c & ~(uintptr_t)3);
        const uint32_t sh = (uint32_t)(c & 3);
        const uint32_t w0 = pa_ld32(al), w1 = sh ? pa_ld32(al + 4) : 0u;
        const uint32_t u = __builtin_amdgcn_alignbyte(w1, w0, sh);
        const float k2 = s * (2.0f / 3.0f);
#pragma unroll
        for (int n = 0; n < 16; n++) vv[n] = fmaf((float)((u >> (2 * n)) & 3u), k2, -s);
    }
}

// Merge softmax state (m2, d2) into (m, d); f1, f2 rescale the two numerators.
__device__ __forceinline__ void pa_merge(float &m, float &d, float m2, float d2, float &f1, float &f2) {
    const float mm = fmaxf(m, m2);
    f1 = mm == -INFINITY ? 0.0f : expf(m - mm);
    f2 = mm == -INFINITY ? 0.0f : expf(m2 - mm);
    d = d * f1 + d2 * f2;
    m = mm;
}

// grid (splits, kv heads), 256 threads. R = 16-query tiles (queries = group * rows <= 16 R).
template <int R>
__device__ __forceinline__ void paged_gqa_partial(const GqaArgs &a) {
    __shared__ float xo[2][R * 16][PA_HD + 4];  // wave partials being merged
    __shared__ float xm[2][R * 16], xd[2][R * 16];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t li = lane & 15, lg = lane >> 4;
    const uint32_t h = blockIdx.y, split = blockIdx.x;
    const uint32_t vrun_blocks = a.component_values / 64;

    // Q^T fragments and per-query causal limits.
    float qf[R][64];
    int32_t lim[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t qi = 16 * r + li;
        lim[r] = -1;
        if (qi < a.queries) {
            const uint32_t t = qi / a.group, g = qi - t * a.group;
            const float4 *src = (const float4 *)(a.query + ((size_t)t * a.query_heads + h * a.group + g) * PA_HD + 64 * lg);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float4 v = src[i];
                qf[r][4 * i] = v.x;
                qf[r][4 * i + 1] = v.y;
                qf[r][4 * i + 2] = v.z;
                qf[r][4 * i + 3] = v.w;
            }
            lim[r] = (int32_t)(a.tokens - a.rows + t);
        } else {
#pragma unroll
            for (int i = 0; i < 64; i++) qf[r][i] = 0.0f;
        }
    }

    float m[R], den[R];
    pa_v4f o[R][16];
#pragma unroll
    for (int r = 0; r < R; r++) {
        m[r] = -INFINITY;
        den[r] = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++) o[r][j] = pa_v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }

    const uint32_t gw = split * 4 + wave;
    const uint32_t t0 = gw * a.tiles_per_wave;
    const uint32_t t1 = min(t0 + a.tiles_per_wave, a.tiles);
    for (uint32_t tile = t0; tile < t1; tile++) {
        const uint32_t tb = tile * 16;
        float kv[64];
        pa_load_k(pa_token(a, tb + li), h, lg, kv);
        pa_v4f s[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            s[r] = pa_v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int k = 0; k < 64; k++) s[r] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[k], qf[r][k], s[r], 0, 0, 0);
        }
        float vv[4][16];
        bool present[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const PaToken t = pa_token(a, tb + 4 * lg + c);
            present[c] = t.run != nullptr;
            pa_load_v(t, vrun_blocks, h, li, vv[c]);
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            float sc[4];
            float mt = -INFINITY;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int32_t j = (int32_t)(tb + 4 * lg + c);
                sc[c] = present[c] && j <= lim[r] ? s[r][c] * a.scale : -INFINITY;
                mt = fmaxf(mt, sc[c]);
            }
            mt = fmaxf(mt, __shfl_xor(mt, 16));
            mt = fmaxf(mt, __shfl_xor(mt, 32));
            const float mn = fmaxf(m[r], mt);
            float p[4], alpha = 1.0f;
            if (mn == -INFINITY) {
                p[0] = p[1] = p[2] = p[3] = 0.0f;
            } else {
                alpha = expf(m[r] - mn);
#pragma unroll
                for (int c = 0; c < 4; c++) p[c] = expf(sc[c] - mn);
            }
            den[r] = den[r] * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
            m[r] = mn;
#pragma unroll
            for (int j = 0; j < 16; j++) o[r][j] *= alpha;
#pragma unroll
            for (int c = 0; c < 4; c++)
#pragma unroll
                for (int j = 0; j < 16; j++)
                    o[r][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[c][j], p[c], o[r][j], 0, 0, 0);
        }
    }
    // Denominators: each lane group summed its own tokens.
#pragma unroll
    for (int r = 0; r < R; r++) {
        den[r] += __shfl_xor(den[r], 16);
        den[r] += __shfl_xor(den[r], 32);
    }

    // Merge the four waves: waves 2,3 publish, 0,1 absorb; then 1 publishes, 0 absorbs.
#pragma unroll
    for (int stage = 0; stage < 2; stage++) {
        const uint32_t lo = stage == 0 ? 2 : 1;  // publishing waves are [lo, 2 lo)
        if (wave >= lo && wave < 2 * lo) {
            const uint32_t slot = wave - lo;
#pragma unroll
            for (int r = 0; r < R; r++) {
                if (lg == 0) {
                    xm[slot][16 * r + li] = m[r];
                    xd[slot][16 * r + li] = den[r];
                }
#pragma unroll
                for (int j = 0; j < 16; j++)
#pragma unroll
                    for (int c = 0; c < 4; c++) xo[slot][16 * r + li][16 * (4 * lg + c) + j] = o[r][j][c];
            }
        }
        __syncthreads();
        if (wave < lo) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                float f1, f2;
                pa_merge(m[r], den[r], xm[wave][16 * r + li], xd[wave][16 * r + li], f1, f2);
#pragma unroll
                for (int j = 0; j < 16; j++)
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        o[r][j][c] = o[r][j][c] * f1 + xo[wave][16 * r + li][16 * (4 * lg + c) + j] * f2;
            }
        }
        __syncthreads();
    }
    if (wave != 0) return;
    // Partial layout: [kv head][split][query][PA_HD]; stats [kv head][split][query][2].
    const size_t base = ((size_t)h * a.splits + split) * a.queries;
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t qi = 16 * r + li;
        if (qi >= a.queries) continue;
        float *dst = a.part_out + (base + qi) * PA_HD;
#pragma unroll
        for (int j = 0; j < 16; j++)
#pragma unroll
            for (int c = 0; c < 4; c++) dst[16 * (4 * lg + c) + j] = o[r][j][c];
        if (lg == 0) {
            a.part_stats[2 * (base + qi)] = m[r];
            a.part_stats[2 * (base + qi) + 1] = den[r];
        }
    }
}

extern "C" __global__ __launch_bounds__(256) void ctox_paged_gqa_partial_r1_gfx950(GqaArgs a) {
    paged_gqa_partial<1>(a);
}
extern "C" __global__ __launch_bounds__(256) void ctox_paged_gqa_partial_r2_gfx950(GqaArgs a) {
    paged_gqa_partial<2>(a);
}

// grid (queries, kv heads), 256 threads = one per head dim.
// out[row][q head][dim] with q head = kv head * group + member.
extern "C" __global__ __launch_bounds__(256) void ctox_paged_gqa_combine_gfx950(GqaArgs a) {
    const uint32_t qi = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
    float mx = -INFINITY;
    for (uint32_t s = 0; s < a.splits; s++)
        mx = fmaxf(mx, a.part_stats[2 * (((size_t)h * a.splits + s) * a.queries + qi)]);
    float num = 0.0f, den = 0.0f;
    if (mx != -INFINITY) {
        for (uint32_t s = 0; s < a.splits; s++) {
            const size_t idx = ((size_t)h * a.splits + s) * a.queries + qi;
            const float f = expf(a.part_stats[2 * idx] - mx);
            den += a.part_stats[2 * idx + 1] * f;
            num += a.part_out[idx * PA_HD + d] * f;
        }
    }
    const uint32_t t = qi / a.group, g = qi - t * a.group;
    a.out[((size_t)t * a.query_heads + h * a.group + g) * PA_HD + d] = den > 0.0f ? num / den : 0.0f;
}
