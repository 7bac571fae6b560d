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

// One 16-token tile's page. When pages hold a multiple of 16 tokens the tile
// lies in one page, so the descriptor lookup is wave-uniform (scalar);
// otherwise every token is resolved on its own.
struct PaTile {
    const uint8_t *base;  // the page's first token (NULL: no such page)
    uint32_t first, count, q4, token_bytes;
};

__device__ __forceinline__ PaTile pa_tile_page(const GqaArgs &a, uint32_t tb) {
    PaTile T{nullptr, 0, 0, 0, 0};
    if (!a.tile_pages) return T;
    const uint32_t p = tb / a.page_tokens;
    if (p >= a.page_count) return T;
    const PagedKvDesc d = a.desc[p];
    T.first = d.first_token;
    T.count = d.tokens;
    T.q4 = d.precision != 0;
    T.token_bytes = T.q4 ? a.q4_token_bytes : a.q2_token_bytes;
    T.base = T.q4 ? a.q4 + (size_t)d.physical_slot * a.q4_page_bytes : a.q2 + (size_t)d.physical_slot * a.q2_page_bytes;
    return T;
}

__device__ __forceinline__ PaToken pa_tile_token(const GqaArgs &a, const PaTile &T, uint32_t j) {
    if (!a.tile_pages) return pa_token(a, j);
    PaToken t{nullptr, T.q4};
    if (T.base && j < a.tokens && j >= T.first && j - T.first < T.count)
        t.run = T.base + (size_t)(j - T.first) * T.token_bytes;
    return t;
}

__device__ __forceinline__ uint32_t pa_ld32(const uint8_t *p) { return *(const uint32_t *)p; }
__device__ __forceinline__ uint32_t pa_ld16(const uint8_t *p) { return *(const uint16_t *)p; }

// K operand of S^T = K Q^T on int8 MFMA 16x16x64: one MFMA per 64-dim block
// b and query limb; lane group g holds its token's dims 64 b + 16 g .. + 15 in
// the order [0, 2, 4, 6, 1, 3, 5, 7, 8, 10, 12, 14, 9, 11, 13, 15] that nibble
// splitting produces (the query limbs are stored in the same order). Codes
// enter as their raw values c (0..15 or 0..3); the level maps (2c - 15) / 15
// and (2c - 3) / 3 and the block scale are applied to the exact integer sums.
typedef int pa_i4 __attribute__((ext_vector_type(4)));

struct PaK {
    uint32_t w[12];  // block b -> w[3b .. 3b+2]: the dwords covering its 8 (Q4) or 4 (Q2) code bytes
    uint32_t meta;   // fp16 scale bits of block g | kind << 20 (kind: 0 absent, 1 Q2, 2 Q4)
};

__device__ __forceinline__ uint32_t pa_kind(uint32_t meta) { return meta >> 20; }
__device__ __forceinline__ uint32_t pa_sh(uint32_t meta) { return (meta >> 16) & 15u; }

// A token's K head run is 4-byte aligned (token, page and head sizes are
// multiples of 4 bytes). Codes of even blocks sit 2 bytes off a dword
// (Q4 34 B and Q2 18 B blocks both start even blocks aligned) and are fetched
// as the covering dwords, the spill-over staying inside the next block.
__device__ __forceinline__ void pa_issue_k(const PaToken &t, uint32_t h, uint32_t g, PaK &r) {
    const uint32_t kind = !t.run ? 0u : (t.q4 ? 2u : 1u);
    r.meta = kind << 20;
#pragma unroll
    for (int i = 0; i < 12; i++) r.w[i] = 0;
    if (kind == 2) {
        const uint8_t *run = t.run + h * 4 * 34;
        r.meta |= pa_ld16(run + g * 34);
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const uint8_t *blk = run + b * 34;
            if (b & 1) {  // codes 4-aligned
                r.w[3 * b] = pa_ld32(blk + 2 + 8 * g);
                r.w[3 * b + 1] = pa_ld32(blk + 6 + 8 * g);
            } else {      // codes at +2 from an aligned block start
                r.w[3 * b] = pa_ld32(blk + 8 * g);
                r.w[3 * b + 1] = pa_ld32(blk + 4 + 8 * g);
                r.w[3 * b + 2] = pa_ld32(blk + 8 + 8 * g);
            }
        }
    } else if (kind == 1) {
        const uint8_t *run = t.run + h * 4 * 18;
        r.meta |= pa_ld16(run + g * 18);
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const uint8_t *blk = run + b * 18;
            if (b & 1) {
                r.w[3 * b] = pa_ld32(blk + 2 + 4 * g);
            } else {
                r.w[3 * b] = pa_ld32(blk + 4 * g);
                r.w[3 * b + 1] = pa_ld32(blk + 4 + 4 * g);
            }
        }
    }
}

// Int8 operands (4 dwords) of block b for the lane's 16 dims.
__device__ __forceinline__ void pa_k_operands(const PaK &r, pa_i4 ak[4]) {
    const uint32_t kind = pa_kind(r.meta);
    if (kind == 2) {
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const uint32_t x0 = (b & 1) ? r.w[3 * b] : __builtin_amdgcn_alignbyte(r.w[3 * b + 1], r.w[3 * b], 2);
            const uint32_t x1 = (b & 1) ? r.w[3 * b + 1] : __builtin_amdgcn_alignbyte(r.w[3 * b + 2], r.w[3 * b + 1], 2);
            ak[b] = pa_i4{(int)(x0 & 0x0F0F0F0Fu), (int)((x0 >> 4) & 0x0F0F0F0Fu), (int)(x1 & 0x0F0F0F0Fu),
                          (int)((x1 >> 4) & 0x0F0F0F0Fu)};
        }
    } else if (kind == 1) {
#pragma unroll
        for (int b = 0; b < 4; b++) {
            // 16 crumbs, 4 per byte: dims 4i..4i+3 in byte i.
            const uint32_t x = (b & 1) ? r.w[3 * b] : __builtin_amdgcn_alignbyte(r.w[3 * b + 1], r.w[3 * b], 2);
            const uint32_t ev = x & 0x33333333u, od = (x >> 2) & 0x33333333u;  // crumbs 0,2 | 1,3 of each byte
            const uint32_t e0 = ev & 0x0F0F0F0Fu, e1 = (ev >> 4) & 0x0F0F0F0Fu;  // dims 4i, 4i + 2
            const uint32_t o0 = od & 0x0F0F0F0Fu, o1 = (od >> 4) & 0x0F0F0F0Fu;  // dims 4i + 1, 4i + 3
            // [0,2,4,6] [1,3,5,7] [8,10,12,14] [9,11,13,15]
            ak[b] = pa_i4{(int)__builtin_amdgcn_perm(e1, e0, 0x05010400u), (int)__builtin_amdgcn_perm(o1, o0, 0x05010400u),
                          (int)__builtin_amdgcn_perm(e1, e0, 0x07030602u), (int)__builtin_amdgcn_perm(o1, o0, 0x07030602u)};
        }
    } else {
#pragma unroll
        for (int b = 0; b < 4; b++) ak[b] = pa_i4{0, 0, 0, 0};
    }
}

// Raw bytes of one lane's V operand for one token: head-dim values
// 16 li .. 16 li + 15 of V head h (block li / 4, quarter li % 4).
struct PaV {
    uint32_t w0, w1, w2;
    uint32_t meta;  // as PaK::meta
};

__device__ __forceinline__ void pa_issue_v(const GqaArgs &a, const PaToken &t, uint32_t h, uint32_t li, PaV &r) {
    const uint32_t kind = !t.run ? 0u : (t.q4 ? 2u : 1u);
    r.meta = kind << 20;
    r.w0 = r.w1 = r.w2 = 0;
    const uint32_t b = a.component_values / 64 + h * 4 + li / 4, q = li & 3;
    if (kind == 2) {
        const uint8_t *blk = t.run + b * 34;
        const uintptr_t c = (uintptr_t)(blk + 2 + 8 * q);
        const uint8_t *al = (const uint8_t *)(c & ~(uintptr_t)3);
        const uint32_t sh = (uint32_t)(c & 3);
        r.meta |= pa_ld16(blk) | (sh << 16);
        r.w0 = pa_ld32(al);
        r.w1 = pa_ld32(al + 4);
        if (sh) r.w2 = pa_ld32(al + 8);
    } else if (kind == 1) {
        const uint8_t *blk = t.run + b * 18;
        const uintptr_t c = (uintptr_t)(blk + 2 + 4 * q);
        const uint8_t *al = (const uint8_t *)(c & ~(uintptr_t)3);
        const uint32_t sh = (uint32_t)(c & 3);
        r.meta |= pa_ld16(blk) | (sh << 16);
        r.w0 = pa_ld32(al);
        if (sh) r.w1 = pa_ld32(al + 4);
    }
}

__device__ __forceinline__ void pa_deq_v(const PaV &r, float vv[16]) {
    const float s = pa_half(r.meta & 0xffffu);
    const uint32_t kind = pa_kind(r.meta), sh = pa_sh(r.meta);
    if (kind == 2) {
        const uint32_t u0 = __builtin_amdgcn_alignbyte(r.w1, r.w0, sh), u1 = __builtin_amdgcn_alignbyte(r.w2, r.w1, sh);
        const float k2 = s * (2.0f / 15.0f);
#pragma unroll
        for (int n = 0; n < 8; n++) {
            vv[n] = fmaf((float)((u0 >> (4 * n)) & 15u), k2, -s);
            vv[8 + n] = fmaf((float)((u1 >> (4 * n)) & 15u), k2, -s);
        }
    } else if (kind == 1) {
        const uint32_t u = __builtin_amdgcn_alignbyte(r.w1, r.w0, sh);
        const float k2 = s * (2.0f / 3.0f);
#pragma unroll
        for (int n = 0; n < 16; n++) vv[n] = fmaf((float)((u >> (2 * n)) & 3u), k2, -s);
    } else {
#pragma unroll
        for (int n = 0; n < 16; n++) vv[n] = 0.0f;
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

#define PA_QS 260   // merge-area row of one query (floats)
#define PA_QB 272   // LDS row of one query limb (int8): 256 + 16 spreads the b128 reads over banks

template <int R>
struct PaState {
    float m[R], den[R];
    int32_t lim[R];
    float qscale[R][4];   // per 64-dim block: 2^-E of the query's fixed point
    int32_t xsum[R][4][3];  // per block and limb: sum of the limb over the block
    pa_v4f o[R][16];
};

// LDS of one workgroup: query limbs [3][R * 16][PA_QB] int8 while tiles run
// (the wave merge area afterwards), plus per-wave block scales of the
// current tile.
template <int R>
struct PaLds {
    static constexpr uint32_t merge_floats = 2 * R * 16 * PA_QS + 4 * R * 16;
    static constexpr uint32_t limb_floats = 3 * R * 16 * PA_QB / 4;
    static constexpr uint32_t main_floats = merge_floats > limb_floats ? merge_floats : limb_floats;
    float main[main_floats];
    float scl[4][16][4];  // [wave][token of tile][block]: scale / 15 (Q4) or / 3 (Q2)
    float qsc[R * 16][4];     // [query][block]: 2^-E of the query's fixed point
    int32_t xs[R * 16][4][3];  // [query][block][limb]: limb sums
};

// One 16-token tile: S^T = K Q^T, online softmax, O^T += V^T P^T.
template <int R>
__device__ __forceinline__ void pa_tile(const GqaArgs &a, PaLds<R> &L, uint32_t wave, uint32_t tb, uint32_t li,
                                        uint32_t lg, const PaK &rk, const PaV rv[4], PaState<R> &st) {
    {   // this lane's block scale (block lg of token li) for the score epilogue
        const uint32_t kind = pa_kind(rk.meta);
        const float sc = pa_half(rk.meta & 0xffffu);
        L.scl[wave][li][lg] = kind == 2 ? sc * (1.0f / 15.0f) : (kind == 1 ? sc * (1.0f / 3.0f) : 0.0f);
    }
    pa_i4 ak[4];
    pa_k_operands(rk, ak);
    const int8_t *qb = (const int8_t *)L.main;
    pa_i4 acc[R][4][3];
#pragma unroll
    for (int r = 0; r < R; r++) {
        // The query limbs are loop invariant; the opaque offset keeps the
        // compiler from hoisting all of them into registers across tiles.
        uint32_t off = (16 * r + li) * PA_QB + lg * 16;
        asm volatile("" : "+v"(off));
#pragma unroll
        for (int b = 0; b < 4; b++)
#pragma unroll
            for (int limb = 0; limb < 3; limb++) {
                const pa_i4 qv = *(const pa_i4 *)(qb + limb * R * 16 * PA_QB + off + 64 * b);
                acc[r][b][limb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ak[b], qv, pa_i4{0, 0, 0, 0}, 0, 0, 0);
            }
    }
    __builtin_amdgcn_wave_barrier();
    float4 f[4];  // block scales of tokens tb + 4 lg + c
#pragma unroll
    for (int c = 0; c < 4; c++) f[c] = *(const float4 *)&L.scl[wave][4 * lg + c][0];
    // Exact per-block integer sums T = sum X (2c - K) = 2 sum(X c) - K sum(X),
    // K = 15 (Q4) or 3 (Q2), per limb; then T = t0 + 256 t1 + 65536 t2.
    float s[R][4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int32_t kq = pa_kind(rv[c].meta) == 2 ? 15 : 3;
        const float fb[4] = {f[c].x, f[c].y, f[c].z, f[c].w};
#pragma unroll
        for (int r = 0; r < R; r++) {
            float dot = 0.0f;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const float t0 = (float)(2 * acc[r][b][0][c] - kq * st.xsum[r][b][0]);
                const float t1 = (float)(2 * acc[r][b][1][c] - kq * st.xsum[r][b][1]);
                const float t2 = (float)(2 * acc[r][b][2][c] - kq * st.xsum[r][b][2]);
                const float t = fmaf(t2, 65536.0f, fmaf(t1, 256.0f, t0));
                dot = fmaf(fb[b] * st.qscale[r][b], t, dot);
            }
            s[r][c] = dot;
        }
    }
    float p[R][4];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float sc[4];
        float mt = -INFINITY;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int32_t j = (int32_t)(tb + 4 * lg + c);
            sc[c] = pa_kind(rv[c].meta) != 0 && j <= st.lim[r] ? s[r][c] * a.scale : -INFINITY;
            mt = fmaxf(mt, sc[c]);
        }
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float mn = fmaxf(st.m[r], mt);
        float alpha = 1.0f;
        if (mn == -INFINITY) {
            p[r][0] = p[r][1] = p[r][2] = p[r][3] = 0.0f;
        } else {
            alpha = expf(st.m[r] - mn);
#pragma unroll
            for (int c = 0; c < 4; c++) p[r][c] = expf(sc[c] - mn);
        }
        st.den[r] = st.den[r] * alpha + ((p[r][0] + p[r][1]) + (p[r][2] + p[r][3]));
        st.m[r] = mn;
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {  // the running max moved for some query
#pragma unroll
            for (int j = 0; j < 16; j++) st.o[r][j] *= alpha;
        }
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
        float vv[16];
        pa_deq_v(rv[c], vv);
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int j = 0; j < 16; j++)
                st.o[r][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[j], p[r][c], st.o[r][j], 0, 0, 0);
    }
}

// grid (splits, kv heads), 256 threads; four waves take contiguous runs of
// tiles_per_wave tiles. R = 16-query tiles (queries = group * rows <= 16 R).
template <int R>
__device__ __forceinline__ void paged_gqa_partial(const GqaArgs &a) {
    __shared__ PaLds<R> L;
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t li = lane & 15, lg = lane >> 4;
    const uint32_t h = blockIdx.y, split = blockIdx.x;

    // Query fixed point per 64-dim block: X = rint(q 2^E) with |X| <= 2^21
    // (2^E from the block's max |q|), split into three balanced int8 limbs
    // X = l0 + 256 l1 + 65536 l2, dims reordered to the K operand's order
    // within each 16. One thread per (query, block); it also leaves 2^-E and
    // the limb sums for the score epilogue.
    for (uint32_t i = threadIdx.x; i < R * 16 * 16; i += 256) {
        // Four consecutive lanes share one (query, block), a quarter of it each.
        int8_t *qb = (int8_t *)L.main;
        const uint32_t qi = i / 16, b = (i / 4) % 4, part = i % 4;
        const float *q = nullptr;
        float mx = 0.0f;
        if (qi < a.queries) {
            const uint32_t t = qi / a.group, g = qi - t * a.group;
            q = a.query + ((size_t)t * a.query_heads + h * a.group + g) * PA_HD + 64 * b;
            for (int d = 0; d < 16; d++) mx = fmaxf(mx, fabsf(q[16 * part + d]));
        }
        mx = fmaxf(mx, __shfl_xor(mx, 1));
        mx = fmaxf(mx, __shfl_xor(mx, 2));
        int ex = 0;
        frexpf(mx, &ex);  // mx < 2^ex
        const float e = mx > 0.0f ? ldexpf(1.0f, 21 - ex) : 0.0f;
        int32_t sums[3] = {0, 0, 0};
#pragma unroll
        for (int dd = 0; dd < 16; dd++) {
            const int d = 16 * part + dd;
            const int32_t X = q ? (int32_t)rintf(q[d] * e) : 0;
            const int32_t l0 = ((X + 128) & 255) - 128;
            const int32_t X1 = (X - l0) >> 8;
            const int32_t l1 = ((X1 + 128) & 255) - 128;
            const int32_t l2 = (X1 - l1) >> 8;
            const uint32_t w = d % 8, pos = 64 * b + (d / 8) * 8 + (w % 2) * 4 + w / 2;
            qb[(0 * R * 16 + qi) * PA_QB + pos] = (int8_t)l0;
            qb[(1 * R * 16 + qi) * PA_QB + pos] = (int8_t)l1;
            qb[(2 * R * 16 + qi) * PA_QB + pos] = (int8_t)l2;
            sums[0] += l0;
            sums[1] += l1;
            sums[2] += l2;
        }
#pragma unroll
        for (int l = 0; l < 3; l++) {
            sums[l] += __shfl_xor(sums[l], 1);
            sums[l] += __shfl_xor(sums[l], 2);
        }
        if (part == 0) {
            L.qsc[qi][b] = mx > 0.0f ? ldexpf(1.0f, ex - 21) : 0.0f;
            L.xs[qi][b][0] = sums[0];
            L.xs[qi][b][1] = sums[1];
            L.xs[qi][b][2] = sums[2];
        }
    }
    PaState<R> st;
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t qi = 16 * r + li;
        st.lim[r] = qi < a.queries ? (int32_t)(a.tokens - a.rows + qi / a.group) : -1;
        st.m[r] = -INFINITY;
        st.den[r] = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++) st.o[r][j] = pa_v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < 4; b++) {
            st.qscale[r][b] = L.qsc[16 * r + li][b];
#pragma unroll
            for (int limb = 0; limb < 3; limb++) st.xsum[r][b][limb] = L.xs[16 * r + li][b][limb];
        }

    const uint32_t gw = split * 4 + wave;
    const uint32_t t0 = gw * a.tiles_per_wave;
    const uint32_t t1 = min(t0 + a.tiles_per_wave, a.tiles);
    if constexpr (R == 1) {
        // Two tiles per iteration: the second tile's loads are in flight while
        // the first computes (R = 2 has no registers to spare for it).
        for (uint32_t tile = t0; tile < t1; tile += 2) {
            const bool second = tile + 1 < t1;
            PaK ka, kb;
            PaV va[4], vb[4];
            const uint32_t tb = tile * 16;
            const uint32_t tb2 = second ? tb + 16 : a.tokens;  // absent tokens when there is no second tile
            const PaTile P1 = pa_tile_page(a, tb), P2 = pa_tile_page(a, tb2);
            pa_issue_k(pa_tile_token(a, P1, tb + li), h, lg, ka);
#pragma unroll
            for (int c = 0; c < 4; c++) pa_issue_v(a, pa_tile_token(a, P1, tb + 4 * lg + c), h, li, va[c]);
            pa_issue_k(pa_tile_token(a, P2, tb2 + li), h, lg, kb);
#pragma unroll
            for (int c = 0; c < 4; c++) pa_issue_v(a, pa_tile_token(a, P2, tb2 + 4 * lg + c), h, li, vb[c]);
            pa_tile<R>(a, L, wave, tb, li, lg, ka, va, st);
            if (second) pa_tile<R>(a, L, wave, tb + 16, li, lg, kb, vb, st);
        }
    } else {
        for (uint32_t tile = t0; tile < t1; tile++) {
            PaK ka;
            PaV va[4];
            const uint32_t tb = tile * 16;
            const PaTile P1 = pa_tile_page(a, tb);
            pa_issue_k(pa_tile_token(a, P1, tb + li), h, lg, ka);
#pragma unroll
            for (int c = 0; c < 4; c++) pa_issue_v(a, pa_tile_token(a, P1, tb + 4 * lg + c), h, li, va[c]);
            pa_tile<R>(a, L, wave, tb, li, lg, ka, va, st);
        }
    }
    // Denominators: each lane group summed its own tokens.
#pragma unroll
    for (int r = 0; r < R; r++) {
        st.den[r] += __shfl_xor(st.den[r], 16);
        st.den[r] += __shfl_xor(st.den[r], 32);
    }
    __syncthreads();  // queries are dead: the LDS becomes the merge area

    // Merge the four waves: waves 2,3 publish, 0,1 absorb; then 1 publishes, 0 absorbs.
    float *xo = L.main;                           // [2][R * 16][PA_QS]
    float *xm = L.main + 2 * R * 16 * PA_QS;      // [2][R * 16]
    float *xd = xm + 2 * R * 16;                  // [2][R * 16]
#pragma unroll
    for (int stage = 0; stage < 2; stage++) {
        const uint32_t lo = stage == 0 ? 2 : 1;  // publishing waves are [lo, 2 lo)
        if (wave >= lo && wave < 2 * lo) {
            const uint32_t slot = wave - lo;
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t row = slot * R * 16 + 16 * r + li;
                if (lg == 0) {
                    xm[row] = st.m[r];
                    xd[row] = st.den[r];
                }
#pragma unroll
                for (int j = 0; j < 16; j++)
#pragma unroll
                    for (int c = 0; c < 4; c++) xo[row * PA_QS + 16 * (4 * lg + c) + j] = st.o[r][j][c];
            }
        }
        __syncthreads();
        if (wave < lo) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t row = wave * R * 16 + 16 * r + li;
                float f1, f2;
                pa_merge(st.m[r], st.den[r], xm[row], xd[row], f1, f2);
#pragma unroll
                for (int j = 0; j < 16; j++)
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        st.o[r][j][c] = st.o[r][j][c] * f1 + xo[row * PA_QS + 16 * (4 * lg + c) + j] * f2;
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
            for (int c = 0; c < 4; c++) dst[16 * (4 * lg + c) + j] = st.o[r][j][c];
        if (lg == 0) {
            a.part_stats[2 * (base + qi)] = st.m[r];
            a.part_stats[2 * (base + qi) + 1] = st.den[r];
        }
    }
}

extern "C" __global__ __launch_bounds__(256, 2) void ctox_paged_gqa_partial_r1_gfx950(GqaArgs a) {
    paged_gqa_partial<1>(a);
}
extern "C" __global__ __launch_bounds__(256, 1) void ctox_paged_gqa_partial_r2_gfx950(GqaArgs a) {
    paged_gqa_partial<2>(a);
}

#define PA_MAX_SPLITS 1024

// grid (queries, kv heads), 256 threads. Split weights exp(m_s - M) are formed
// once in LDS; each wave then sums every fourth split over all 256 dims
// (a float4 per lane) and the four wave sums are added in a fixed order.
// out[row][q head][dim] with q head = kv head * group + member.
extern "C" __global__ __launch_bounds__(256) void ctox_paged_gqa_combine_gfx950(GqaArgs a) {
    __shared__ float wgt[PA_MAX_SPLITS];
    __shared__ float red[4];
    __shared__ float4 acc4[4][64];
    const uint32_t qi = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const uint32_t lane = tid & 63, wave = tid >> 6;
    const size_t base = (size_t)h * a.splits * a.queries + qi;  // + s * queries
    float mx = -INFINITY;
    for (uint32_t s = tid; s < a.splits; s += 256) mx = fmaxf(mx, a.part_stats[2 * (base + (size_t)s * a.queries)]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float den = 0.0f;
    for (uint32_t s = tid; s < a.splits; s += 256) {
        const size_t idx = base + (size_t)s * a.queries;
        const float ms = a.part_stats[2 * idx];
        const float f = ms == -INFINITY ? 0.0f : expf(ms - mx);
        wgt[s] = f;
        den += a.part_stats[2 * idx + 1] * f;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) den += __shfl_xor(den, o);
    if (lane == 0) red[wave] = den;
    __syncthreads();
    den = (red[0] + red[1]) + (red[2] + red[3]);
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 4
    for (uint32_t s = wave; s < a.splits; s += 4) {
        const float f = wgt[s];
        const float4 v = ((const float4 *)(a.part_out + (base + (size_t)s * a.queries) * PA_HD))[lane];
        acc.x += v.x * f;
        acc.y += v.y * f;
        acc.z += v.z * f;
        acc.w += v.w * f;
    }
    acc4[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    const float4 a0 = acc4[0][lane], a1 = acc4[1][lane], a2 = acc4[2][lane], a3 = acc4[3][lane];
    const float inv = den > 0.0f ? 1.0f / den : 0.0f;
    const uint32_t t = qi / a.group, g = qi - t * a.group;
    float4 *out = (float4 *)(a.out + ((size_t)t * a.query_heads + h * a.group + g) * PA_HD);
    out[lane] = make_float4(((a0.x + a1.x) + (a2.x + a3.x)) * inv, ((a0.y + a1.y) + (a2.y + a3.y)) * inv,
                            ((a0.z + a1.z) + (a2.z + a3.z)) * inv, ((a0.w + a1.w) + (a2.w + a3.w)) * inv);
}
