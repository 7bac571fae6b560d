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
#include "lds_barrier.h"

typedef float pa_v4f __attribute__((ext_vector_type(4)));

#define PA_HD 256  // head dim: four 64-value blocks, one per MFMA lane group
// The page-aligned kernel keeps its running maxima in base-2 units (scores
// times log2 e) so each probability is one v_exp_f32; its stats leave in
// natural units.
#define PA_LOG2E 1.44269504088896341f
#define PA_LN2 0.693147180559945309f

__device__ __forceinline__ float pa_half(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// ---------------------------------------------------------------------------
// pack
// ---------------------------------------------------------------------------
#pragma clang fp contract(off)
// One 64-value block held one value per lane: Q4 codes and fp16 scale at dst.
__device__ __forceinline__ void pa_pack_q4_block(float v, uint32_t lane, uint8_t *dst) {
    float m = fabsf(v);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    uint32_t code = 0;
    if (m != 0.0f) {
        float n = v / m;  // correctly rounded division (HIP's default for f32)
        n = fminf(1.0f, fmaxf(-1.0f, n));
        const float sel = n * 7.5f + 7.5f;  // contraction is off in this region: two roundings
        code = (uint32_t)fminf(15.0f, fmaxf(0.0f, roundf(sel)));
    }
    const uint32_t hi = __shfl_down(code, 1);
    if ((lane & 1) == 0) dst[2 + lane / 2] = (uint8_t)(code | (hi << 4));
    if (lane == 0) {
        const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)m);  // round to nearest even
        dst[0] = (uint8_t)h;
        dst[1] = (uint8_t)(h >> 8);
    }
}

extern "C" __global__ __launch_bounds__(64) void ctox_kv_pack_q4_gfx950(KvPackArgs a) {
    const uint32_t lane = threadIdx.x, blk = blockIdx.x, tok = blockIdx.y;
    const uint32_t idx = blk * 64 + lane;
    const size_t row = (size_t)tok * a.component_values;
    const float v = idx < a.component_values ? a.keys[row + idx] : a.values[row + idx - a.component_values];
    pa_pack_q4_block(v, lane, a.q4_pages + (size_t)a.physical_slot * a.q4_page_bytes +
                                  (size_t)(a.first_token_in_page + tok) * a.q4_token_bytes + (size_t)blk * 34);
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

#define PA_SROW 69  // stage row of one token (dwords): K run at 0, V run at 34, one pad
#define PA_QS 260   // merge-area row of one query (floats)
#define PA_QB 272   // LDS row of one query limb (int8): 256 + 16 spreads the b128 reads over banks

template <int R>
struct PaState {
    float m[R], den[R];
    int32_t lim[R];
    float qscale[R][4];   // per 64-dim block: 2^-E of the query's fixed point
    int32_t xsum[R][4][3];  // per block and limb: sum of the limb over the block
    int32_t xst[R][4];      // per block: sum of X (xsum combined)
    float corr[R][4];       // f16 path: sum over tokens of P * (block scale), per value block
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


// ---------------------------------------------------------------------------
// Page-aligned tiles (page_tokens % 16 == 0): P.V on f16 MFMA 16x16x16.
//
// O^T (dims x queries) += V^T P^T with k = the tile's 16 tokens. The score
// accumulator already leaves lane (li, lg) the probabilities of tokens
// 4 lg .. 4 lg + 3 for query li, which is exactly its B operand. Per value
// block b and chunk c the A operand row m is dim 64 b + 4 m + c, so lane
// (li, lg) needs one code byte (Q2) or two (Q4) per (token, block) and its
// C rows are dims 64 b + 16 lg + 4 i + c.
//
// A value is v = s (2 code - K) / K = (2 s / K) code - s (K = 3 Q2, 15 Q4).
// A holds the raw codes, exact in f16: the code field (placed at bit 2 c of
// each half, i.e. times 4^c) is ORed under the exponent field E and the
// implicit one is subtracted, giving code * 4^c * 2^(E - 25) exactly. B holds
// P * (2 s / K) * 2^(25 - E) as an f16 hi + lo pair (relative error ~2^-21),
// with E chosen per tile and block from the largest 2 s / K so that B stays
// in f16's normal range. The products are P (2 s / K) code 4^c whatever E
// is; the 4^c is removed at the end and the "- s" part is summed per
// (query, block) on the VALU (corr).
// ---------------------------------------------------------------------------
typedef _Float16 pa_h2 __attribute__((ext_vector_type(2)));
typedef _Float16 pa_h4 __attribute__((ext_vector_type(4)));

// One tile's K and V head runs (4 blocks each: 18 dwords Q2, 34 Q4) of the
// 16 tokens, moved through a per-wave LDS stage: lane (t = lane / 4, q =
// lane % 4) loads dwords q, q + 4, ... of token t's runs, so each quad of
// lanes reads 16 contiguous bytes. Absent tokens read a valid dummy address;
// presence is applied where the tile is computed, and no loaded value is
// used before then, so the wait before each tile's compute stays exact.

struct PaStage {
    uint32_t k[9], v[9];
};

__device__ __forceinline__ bool pa_present(const GqaArgs &a, const PaTile &T, uint32_t j) {
    return T.base != nullptr && j < a.tokens && j >= T.first && j - T.first < T.count;
}


__device__ __forceinline__ void pa_issue_stage(const GqaArgs &a, const PaTile &T, uint32_t tb, uint32_t h,
                                               uint32_t lane, PaStage &r) {
    // Buffer loads against the tile's page: one 32-bit lane offset, the
    // dword steps in the instructions' immediate offsets. Absent tokens use
    // an offset past the page, which returns zeros without memory traffic.
    // Loads past a run's end (up to 15 bytes) are never staged.
    const uint32_t t = lane >> 2, q = lane & 3, j = tb + t;
    const bool p = pa_present(a, T, j);
    const uint32_t bs = T.q4 ? 34u : 18u;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)T.base, (short)0, (int)(T.q4 ? a.q4_page_bytes : a.q2_page_bytes), 0x00020000);
    const uint32_t ko = p ? (j - T.first) * T.token_bytes + h * 4 * bs + 4 * q : 0x7fff0000u;
    const uint32_t vo = p ? ko + (a.component_values / 64) * bs : 0x7fff0000u;
    if (T.q4) {
#pragma unroll
        for (int m = 0; m < 9; m++) {
            r.k[m] = __builtin_amdgcn_raw_buffer_load_b32(rs, ko + 16 * m, 0, 0);
            r.v[m] = __builtin_amdgcn_raw_buffer_load_b32(rs, vo + 16 * m, 0, 0);
        }
    } else {
#pragma unroll
        for (int m = 0; m < 5; m++) {
            r.k[m] = __builtin_amdgcn_raw_buffer_load_b32(rs, ko + 16 * m, 0, 0);
            r.v[m] = __builtin_amdgcn_raw_buffer_load_b32(rs, vo + 16 * m, 0, 0);
        }
    }
}

// v_and_or_b32: (x & m) | o in one instruction (m a wave-uniform mask, o in a VGPR).
__device__ __forceinline__ uint32_t pa_and_or(uint32_t x, uint32_t m, uint32_t o) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(m), "v"(o));
    return r;
}

__device__ __forceinline__ void pa_stage_write(uint32_t *stage, uint32_t lane, bool q4, const PaStage &r) {
    const uint32_t t = lane >> 2, q = lane & 3, nd = q4 ? 34u : 18u;
    uint32_t *row = stage + t * PA_SROW;
#pragma unroll
    for (int m = 0; m < 9; m++) {
        const uint32_t d = q + 4 * m;
        if ((m < 5 || q4) && d < nd) {
            row[d] = r.k[m];
            row[34 + d] = r.v[m];
        }
    }
}

// Stage reads: dword-aligned byte offset o of a run; the fp16 at even offset o.
__device__ __forceinline__ uint32_t pa_s32(const uint32_t *run, uint32_t o) { return run[o >> 2]; }
__device__ __forceinline__ uint32_t pa_s16(const uint32_t *run, uint32_t o) {
    return (run[o >> 2] >> (8 * (o & 2))) & 0xffffu;
}

// K operand words of token li (dims 16 lg .. of each block) from the stage,
// in pa_issue_k's layout.
__device__ __forceinline__ void pa_k_from_stage(const uint32_t *kr, uint32_t lg, bool q4, bool present, PaK &r) {
#pragma unroll
    for (int i = 0; i < 12; i++) r.w[i] = 0;
    if (q4) {
        r.meta = (present ? 2u << 20 : 0u) | pa_s16(kr, lg * 34);
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const uint32_t o = b * 34 + 8 * lg;
            if (b & 1) {
                r.w[3 * b] = pa_s32(kr, o + 2);
                r.w[3 * b + 1] = pa_s32(kr, o + 6);
            } else {
                r.w[3 * b] = pa_s32(kr, o);
                r.w[3 * b + 1] = pa_s32(kr, o + 4);
                r.w[3 * b + 2] = pa_s32(kr, o + 8);
            }
        }
    } else {
        r.meta = (present ? 1u << 20 : 0u) | pa_s16(kr, lg * 18);
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const uint32_t o = b * 18 + 4 * lg;
            if (b & 1) {
                r.w[3 * b] = pa_s32(kr, o + 2);
            } else {
                r.w[3 * b] = pa_s32(kr, o);
                r.w[3 * b + 1] = pa_s32(kr, o + 4);
            }
        }
    }
}

// Lane i holds the page descriptor of tile t0 + i (all zeros, i.e. no
// tokens, past t1 or past the page table). Tiles lie in one page here.
__device__ __forceinline__ uint4 pa_load_descs(const GqaArgs &a, uint32_t t0, uint32_t t1, uint32_t lane) {
    const uint32_t t = t0 + lane;
    const uint32_t p = t < t1 ? t * 16 / a.page_tokens : a.page_count;
    const uint4 d = ((const uint4 *)a.desc)[p < a.page_count ? p : 0];
    return p < a.page_count ? d : make_uint4(0, 0, 0, 0);
}

// Tile k of the wave's range (k wave-uniform) from the descriptor registers.
__device__ __forceinline__ PaTile pa_tile_of(const GqaArgs &a, const uint4 &d, uint32_t k) {
    const uint32_t kk = k < 64 ? k : 0;
    const uint32_t prec = __builtin_amdgcn_readlane(d.x, kk), slot = __builtin_amdgcn_readlane(d.y, kk);
    const uint32_t cnt = __builtin_amdgcn_readlane(d.z, kk), first = __builtin_amdgcn_readlane(d.w, kk);
    PaTile T;
    T.first = first;
    T.count = k < 64 ? cnt : 0u;
    T.q4 = prec != 0;
    T.token_bytes = T.q4 ? a.q4_token_bytes : a.q2_token_bytes;
    T.base = T.q4 ? a.q4 + (size_t)slot * a.q4_page_bytes : a.q2 + (size_t)slot * a.q2_page_bytes;
    return T;
}

// Max over lanes l and l ^ 16 / l ^ 32 with permlane swaps (VALU, no LDS trip).
__device__ __forceinline__ float pa_max_x16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                    false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ __forceinline__ float pa_max_x32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                    false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
// Max over the four lanes of a 16-lane row that share lane % 4 (DPP row rotations by 4 and 8).
__device__ __forceinline__ float pa_max_rot48(float v) {
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false)));
    return v;
}

__device__ __forceinline__ pa_h2 pa_as_h2(uint32_t x) { return __builtin_bit_cast(pa_h2, x); }
__device__ __forceinline__ uint32_t pa_pk(float x, float y) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x, y));
}

// Q4: the tile's precision (-1: read from the tile; 0 / 1: a constant, so the
// block sizes, offsets, code masks and selectors fold).
// SH: the queries share one fixed point per block, folded into qsl (the
// K block scales); otherwise qsl is 1 and each query's 2^-E applies.
template <int R, int Q4, bool SH, class LDS>
__device__ __forceinline__ void pa_tile16(const GqaArgs &a, LDS &L, const int8_t *qb, uint32_t wave, uint32_t tb, uint32_t h,
                                          uint32_t li, uint32_t lg, const PaTile &T, const uint32_t *stage,
                                          float qsl, PaState<R> &st) {
    const uint32_t lane = 16 * lg + li;
    const bool q4 = Q4 >= 0 ? Q4 == 1 : T.q4 != 0;
    bool present[4];
#pragma unroll
    for (int c = 0; c < 4; c++) present[c] = pa_present(a, T, tb + 4 * lg + c);
    // Operands from the stage (rows: tokens; K run at dword 0, V run at 34).
    const uint32_t bs = q4 ? 34u : 18u;
    PaK rk;
    pa_k_from_stage(stage + li * PA_SROW, lg, q4, pa_present(a, T, tb + li), rk);
    uint32_t vw[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t *vr = stage + (4 * lg + i) * PA_SROW + 34;
#pragma unroll
        for (int b = 0; b < 4; b++) vw[b][i] = pa_s32(vr, (b * bs + 2 + (q4 ? 2 * li : li)) & ~3u);
    }
    // (absent tokens were staged as zeros: zero codes and scales)
    const uint32_t vsb = pa_s16(stage + (4 * lg + (li >> 2)) * PA_SROW + 34, (li & 3) * bs);
    {   // K block scale of (token li, block lg) times the queries' 2^-E of that block
        const uint32_t kind = pa_kind(rk.meta);
        const float sc = pa_half(rk.meta & 0xffffu) * qsl;
        L.scl[wave][li][lg] = kind == 2 ? sc * (1.0f / 15.0f) : (kind == 1 ? sc * (1.0f / 3.0f) : 0.0f);
    }
    int32_t Eb[4];  // the tile's exponent field per V block
    {   // V: 2 s / K of (token 4 lg + (li >> 2), block li & 3), staged unscaled;
        // the block maxima reduce on the VALU meanwhile.
        const float ws = pa_half(vsb) * (q4 ? 2.0f / 15.0f : 2.0f / 3.0f);
        L.vws[wave][4 * lg + (li >> 2)][li & 3] = ws;
        const float mx = pa_max_x32(pa_max_x16(pa_max_rot48(ws)));
        int ex = 0;
        frexpf(mx, &ex);  // mx < 2^ex: B = P * ws * 2^(25 - E) < 2^14 P, P < 2
        const int E = min(30, max(1, 11 + ex));
#pragma unroll
        for (int b = 0; b < 4; b++) Eb[b] = __builtin_amdgcn_readlane(E, b);  // lane b holds block b's
    }
    pa_i4 ak[4];
    {   // absent tokens staged as zeros: unpack with the tile-uniform precision
        PaK ku = rk;
        ku.meta = (rk.meta & 0xfffffu) | ((q4 ? 2u : 1u) << 20);
        pa_k_operands(ku, ak);
    }
    __builtin_amdgcn_wave_barrier();
    float4 f[4];   // K block scales of tokens tb + 4 lg + c
    float4 wv[4];  // V: 2 s / K * 2^(25 - E) of tokens tb + 4 lg + c, per block
    float fe[4];
#pragma unroll
    for (int b = 0; b < 4; b++) fe[b] = ldexpf(1.0f, 25 - Eb[b]);
#pragma unroll
    for (int c = 0; c < 4; c++) {
        f[c] = *(const float4 *)&L.scl[wave][4 * lg + c][0];
        const float4 w = *(const float4 *)&L.vws[wave][4 * lg + c][0];
        wv[c] = make_float4(w.x * fe[0], w.y * fe[1], w.z * fe[2], w.w * fe[3]);
    }
    // Scores, one block at a time: T = sum X (2c - K) = 2 sum(X c) - K sum X,
    // exact in 32-bit modular arithmetic (|T| < 2^31 although 2 sum(X c) may wrap).
    const uint32_t kq = q4 ? 15u : 3u;
    float s[R][4];
#pragma unroll
    for (int r = 0; r < R; r++) {
        uint32_t off = (16 * r + li) * PA_QB + lg * 16;
        asm volatile("" : "+v"(off));
#pragma unroll
        for (int c = 0; c < 4; c++) s[r][c] = 0.0f;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            pa_i4 acc[3];
#pragma unroll
            for (int limb = 0; limb < 3; limb++) {
                const pa_i4 qv = *(const pa_i4 *)(qb + limb * R * 16 * PA_QB + off + 64 * b);
                acc[limb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ak[b], qv, pa_i4{0, 0, 0, 0}, 0, 0, 0);
            }
            const uint32_t kx = kq * (uint32_t)st.xst[r][b];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint32_t U = (uint32_t)acc[0][c] + ((uint32_t)acc[1][c] << 8) + ((uint32_t)acc[2][c] << 16);
                const int32_t t = (int32_t)(2u * U - kx);
                const float fb = b == 0 ? f[c].x : b == 1 ? f[c].y : b == 2 ? f[c].z : f[c].w;
                s[r][c] = fmaf(SH ? fb : fb * st.qscale[r][b], (float)t, s[r][c]);
            }
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
            sc[c] = present[c] && j <= st.lim[r] ? s[r][c] * (a.scale * PA_LOG2E) : -INFINITY;
            mt = fmaxf(mt, sc[c]);
        }
        mt = pa_max_x32(pa_max_x16(mt));
        // The reference maximum moves only when the tile's exceeds it by
        // more than 1 (base 2): probabilities then stay below 2, which the V
        // operand's exponent headroom allows (B < 2^15), and most tiles skip
        // the accumulators' rescale. Leaving the empty state (m = -inf: the
        // accumulators are zero) needs no rescale either.
        const bool move = mt > st.m[r] + 1.0f;
        const float mn = move ? mt : st.m[r];
        float alpha = 1.0f;
        if (mn == -INFINITY) {
            p[r][0] = p[r][1] = p[r][2] = p[r][3] = 0.0f;
        } else {
            if (move && st.m[r] != -INFINITY) alpha = __builtin_amdgcn_exp2f(st.m[r] - mn);
#pragma unroll
            for (int c = 0; c < 4; c++) p[r][c] = __builtin_amdgcn_exp2f(sc[c] - mn);
        }
        st.den[r] = st.den[r] * alpha + ((p[r][0] + p[r][1]) + (p[r][2] + p[r][3]));
        st.m[r] = mn;
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
            for (int j = 0; j < 16; j++) st.o[r][j] *= alpha;
#pragma unroll
            for (int b = 0; b < 4; b++) st.corr[r][b] *= alpha;
        }
    }
#pragma unroll
    for (int b = 0; b < 4; b++) {
        // B operands (hi, lo) for block b, and the "- s" sums.
        pa_h4 bh[R], bl[R];
        const float kh = ldexpf(q4 ? 7.5f : 1.5f, Eb[b] - 25);  // K / 2 * 2^(E - 25): B back to P * s
#pragma unroll
        for (int r = 0; r < R; r++) {
            float pb[4];
            pb[0] = p[r][0] * wv[0][b];
            pb[1] = p[r][1] * wv[1][b];
            pb[2] = p[r][2] * wv[2][b];
            pb[3] = p[r][3] * wv[3][b];
            const uint32_t h01 = pa_pk(pb[0], pb[1]), h23 = pa_pk(pb[2], pb[3]);
            const pa_h2 H01 = pa_as_h2(h01), H23 = pa_as_h2(h23);
            const uint32_t l01 = pa_pk(pb[0] - (float)H01[0], pb[1] - (float)H01[1]);
            const uint32_t l23 = pa_pk(pb[2] - (float)H23[0], pb[3] - (float)H23[1]);
            bh[r] = __builtin_bit_cast(pa_h4, (uint64_t)h01 | ((uint64_t)h23 << 32));
            bl[r] = __builtin_bit_cast(pa_h4, (uint64_t)l01 | ((uint64_t)l23 << 32));
            st.corr[r][b] = fmaf((pb[0] + pb[1]) + (pb[2] + pb[3]), kh, st.corr[r][b]);
        }
        // A operands: codes of tokens (0, 1) and (2, 3) side by side in the two halves.
        const uint32_t o = (b * bs + 2 + (q4 ? 2 * li : li)) & 3u;
        const uint32_t sel = q4 ? (o | ((o + 1) << 8) | ((o + 4) << 16) | ((o + 5) << 24))
                                : (o | (0x0cu << 8) | ((o + 4) << 16) | (0x0cu << 24));
        const uint32_t y01 = __builtin_amdgcn_perm(vw[b][1], vw[b][0], sel);
        const uint32_t y23 = __builtin_amdgcn_perm(vw[b][3], vw[b][2], sel);
        const uint32_t E = (uint32_t)Eb[b];
        uint32_t magic = (E << 10) | (E << 26);
        asm volatile("" : "+v"(magic));  // a VGPR operand of v_and_or_b32
        const _Float16 one = (_Float16)ldexpf(1.0f, (int)E - 15);
        const pa_h2 bias = pa_h2{-one, -one};
        pa_h4 av[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            // Q4 nibble c sits at bit 4c: shifted to bit 2c like the Q2 crumb.
            const uint32_t x01 = q4 ? y01 >> (2 * c) : y01, x23 = q4 ? y23 >> (2 * c) : y23;
            const uint32_t m = (q4 ? 0x000F000Fu : 0x00030003u) << (2 * c);
            const pa_h2 a01 = pa_as_h2(pa_and_or(x01, m, magic)) + bias;
            const pa_h2 a23 = pa_as_h2(pa_and_or(x23, m, magic)) + bias;
            av[c] = pa_h4{a01[0], a01[1], a23[0], a23[1]};
        }
        // hi parts of the four chunks, then the lo parts: no MFMA waits on the one before.
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int c = 0; c < 4; c++)
                st.o[r][4 * b + c] = __builtin_amdgcn_mfma_f32_16x16x16f16(av[c], bh[r], st.o[r][4 * b + c], 0, 0, 0);
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int c = 0; c < 4; c++)
                st.o[r][4 * b + c] = __builtin_amdgcn_mfma_f32_16x16x16f16(av[c], bl[r], st.o[r][4 * b + c], 0, 0, 0);
    }
}

// The query values one thread of pa_prep_queries works on: iteration r is
// (query, block, quarter) i = threadIdx.x + 256 r, its 16 values (zeros past
// the queries). Loaded apart from the computation so that callers can issue
// other loads in between.
template <int R>
__device__ __forceinline__ void pa_prep_load(const GqaArgs &a, uint32_t h, float (&qv)[R][16]) {
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t i = threadIdx.x + 256 * r;
        const uint32_t qi = i / 16, b = (i / 4) % 4, part = i % 4;
        const bool valid = qi < a.queries;
        const uint32_t t = valid ? qi / a.group : 0, g = valid ? qi - t * a.group : 0;
        const float4 *qp = (const float4 *)(a.query + ((size_t)t * a.query_heads + h * a.group + g) * PA_HD + 64 * b +
                                            16 * part);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float4 v4 = qp[k];
            qv[r][4 * k] = valid ? v4.x : 0.0f;
            qv[r][4 * k + 1] = valid ? v4.y : 0.0f;
            qv[r][4 * k + 2] = valid ? v4.z : 0.0f;
            qv[r][4 * k + 3] = valid ? v4.w : 0.0f;
        }
    }
}

// Query fixed point per 64-dim block: X = rint(q 2^E) with |X| <= 2^21
// (2^E from the block's max |q|), split into three balanced int8 limbs
// X = l0 + 256 l1 + 65536 l2, dims reordered to the K operand's order
// within each 16. One thread per (query, block, quarter); it also leaves 2^-E
// and the limb sums for the score epilogue.
// SH: one fixed point per 64-dim block for all the workgroup's queries (2^E
// from the largest |q| of the block over every query; the query vectors are
// RMS-normed, so their block maxima are alike), so the score epilogue folds
// 2^-E into the keys' block scales. bmx: 16 LDS floats for that maximum.
template <int R, bool SH = false>
__device__ __forceinline__ void pa_prep_compute(const GqaArgs &a, const float (&q)[R][16], int8_t *qb,
                                                float (*qsc)[4], int32_t (*xs)[4][3], float *bmx = nullptr) {
    float mxs[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float mx = 0.0f;
#pragma unroll
        for (int d = 0; d < 16; d++) mx = fmaxf(mx, fabsf(q[r][d]));
        mx = fmaxf(mx, __shfl_xor(mx, 1));
        mx = fmaxf(mx, __shfl_xor(mx, 2));
        mxs[r] = mx;
    }
    if (SH) {
        // Lanes 4 b .. 4 b + 3 of each 16-lane row hold block b: the wave's
        // and then the workgroup's maximum per block.
        float m = mxs[0];
#pragma unroll
        for (int r = 1; r < R; r++) m = fmaxf(m, mxs[r]);
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
        const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        if (lane < 16 && (lane & 3) == 0) bmx[wave * 4 + lane / 4] = m;
        lds_barrier();
        const uint32_t b = (threadIdx.x / 4) % 4;
        m = fmaxf(fmaxf(bmx[b], bmx[4 + b]), fmaxf(bmx[8 + b], bmx[12 + b]));
#pragma unroll
        for (int r = 0; r < R; r++) mxs[r] = m;
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t i = threadIdx.x + 256 * r;
        // Four consecutive lanes share one (query, block), a quarter of it each.
        const uint32_t qi = i / 16, b = (i / 4) % 4, part = i % 4;
        const float *qv = q[r];
        const float mx = mxs[r];
        int ex = 0;
        frexpf(mx, &ex);  // mx < 2^ex
        const float e = mx > 0.0f ? ldexpf(1.0f, 21 - ex) : 0.0f;
        int32_t sums[3] = {0, 0, 0};
        // The quarter's dims land in 16 consecutive bytes of each limb row
        // (dims reordered within each 8 as 0,2,4,6,1,3,5,7): one 16-byte store per limb.
        uint32_t packed[3][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
        for (int dd = 0; dd < 16; dd++) {
            const int32_t X = (int32_t)rintf(qv[dd] * e);
            const int32_t l0 = ((X + 128) & 255) - 128;
            const int32_t X1 = (X - l0) >> 8;
            const int32_t l1 = ((X1 + 128) & 255) - 128;
            const int32_t l2 = (X1 - l1) >> 8;
            const uint32_t w = dd % 8, local = (dd / 8) * 8 + (w % 2) * 4 + w / 2;
            packed[0][local / 4] |= (uint32_t)(l0 & 255) << (8 * (local % 4));
            packed[1][local / 4] |= (uint32_t)(l1 & 255) << (8 * (local % 4));
            packed[2][local / 4] |= (uint32_t)(l2 & 255) << (8 * (local % 4));
            sums[0] += l0;
            sums[1] += l1;
            sums[2] += l2;
        }
#pragma unroll
        for (int l = 0; l < 3; l++)
            *(uint4 *)(qb + (l * R * 16 + qi) * PA_QB + 64 * b + 16 * part) =
                make_uint4(packed[l][0], packed[l][1], packed[l][2], packed[l][3]);
#pragma unroll
        for (int l = 0; l < 3; l++) {
            sums[l] += __shfl_xor(sums[l], 1);
            sums[l] += __shfl_xor(sums[l], 2);
        }
        if (part == 0) {
            qsc[qi][b] = mx > 0.0f ? ldexpf(1.0f, ex - 21) : 0.0f;
            xs[qi][b][0] = sums[0];
            xs[qi][b][1] = sums[1];
            xs[qi][b][2] = sums[2];
        }
    }
}

template <int R>
__device__ __forceinline__ void pa_prep_queries(const GqaArgs &a, uint32_t h, int8_t *qb, float (*qsc)[4],
                                                int32_t (*xs)[4][3]) {
    float q[R][16];
    pa_prep_load<R>(a, h, q);
    pa_prep_compute<R>(a, q, qb, qsc, xs);
}

// LDS of the page-aligned kernel: query limbs and the per-wave K/V stages
// while tiles run, overlaid afterwards by the merge area of waves 1..3.
template <int R>
struct PaLds16 {
    static constexpr uint32_t limb_bytes = 3 * R * 16 * PA_QB;
    static constexpr uint32_t merge_floats = 3 * R * 16 * PA_QS + 6 * R * 16;
    union {
        struct {
            int8_t limbs[limb_bytes];
            uint32_t stage[4][16 * PA_SROW];
        } run;
        float merge[merge_floats];
    } u;
    float scl[4][16][4];       // [wave][token of tile][block]: K scale / 15 (Q4) or / 3 (Q2)
    float vws[4][16][4];       // [wave][token][V block]: 2 V scale / K
    float qsc[R * 16][4];      // [query][block]: 2^-E of the (shared) fixed point
    int32_t xs[R * 16][4][3];  // [query][block][limb]: limb sums
    float bmx[16];             // [wave][block]: largest |q| (the prep's shared fixed point)
};

// grid (splits, kv heads), 256 threads; four waves take contiguous runs of
// tiles_per_wave (<= 64) page-aligned tiles. Lane (li, lg) ends with O^T of
// query 16 r + li at dims 64 b + 16 lg + 4 i + c in o[r][4 b + c][i].
template <int R>
__device__ __forceinline__ void paged_gqa_partial16(const GqaArgs &a) {
    __shared__ PaLds16<R> L;
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t li = lane & 15, lg = lane >> 4;
    const uint32_t h = blockIdx.y, split = blockIdx.x;
    const uint32_t gw = split * 4 + wave;
    const uint32_t t0 = gw * a.tiles_per_wave;
    const uint32_t t1 = min(t0 + a.tiles_per_wave, a.tiles);
    // The wave's page descriptors load together with the queries; the first
    // tile's loads go out (they need only the descriptors) before the query
    // limbs are computed.
    const uint4 dsc = pa_load_descs(a, t0, t1, lane);
    float qv[R][16];
    pa_prep_load<R>(a, h, qv);
    PaStage sg;
    PaTile PA = pa_tile_of(a, dsc, 0);
    pa_issue_stage(a, PA, t0 * 16, h, lane, sg);
    // Two query tiles share one fixed point per block (the 16 multiplies per
    // tile it saves outweigh the prep's extra barrier; one tile keeps its
    // per-query fixed point).
    constexpr bool SH = R > 1;
    pa_prep_compute<R, SH>(a, qv, L.u.run.limbs, L.qsc, L.xs, L.bmx);
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
    // The first tile's loads stay in flight across the (LDS-only) barrier.
    uint32_t *stage = L.u.run.stage[wave];
    lds_barrier();
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < 4; b++) {
            st.qscale[r][b] = L.qsc[16 * r + li][b];
            st.xst[r][b] = L.xs[16 * r + li][b][0] + 256 * L.xs[16 * r + li][b][1] + 65536 * L.xs[16 * r + li][b][2];
            st.corr[r][b] = 0.0f;
        }
    const float qsl = SH ? L.qsc[0][lg] : 1.0f;  // shared: 2^-E of block lg, the same for every query
    // Tile k computes from the stage while tile k + 1's loads are in flight.
    // A wave whose tiles all lie in Q2 pages (most of a long context) runs
    // the tile loop with the precision folded in.
    auto run = [&](auto q4c) {
        constexpr int Q4 = decltype(q4c)::value;
        for (uint32_t tile = t0; tile < t1; tile++) {
            pa_stage_write(stage, lane, Q4 >= 0 ? Q4 == 1 : PA.q4 != 0, sg);
            const PaTile PN = pa_tile_of(a, dsc, tile + 1 - t0);
            pa_issue_stage(a, PN, (tile + 1) * 16, h, lane, sg);
            pa_tile16<R, Q4, SH>(a, L, L.u.run.limbs, wave, tile * 16, h, li, lg, PA, stage, qsl, st);
            PA = PN;
        }
    };
    if (__builtin_amdgcn_ballot_w64(lane < t1 - t0 && dsc.x != 0) == 0)
        run(std::integral_constant<int, 0>{});
    else
        run(std::integral_constant<int, -1>{});
    // O = C 4^-c - sum P s (the latter summed over the four lane groups' tokens);
    // denominators likewise.
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int b = 0; b < 4; b++) {
            float cs = st.corr[r][b];
            cs += __shfl_xor(cs, 16);
            cs += __shfl_xor(cs, 32);
#pragma unroll
            for (int c = 0; c < 4; c++) st.o[r][4 * b + c] = st.o[r][4 * b + c] * (1.0f / (float)(1u << (2 * c))) - cs;
        }
        st.den[r] += __shfl_xor(st.den[r], 16);
        st.den[r] += __shfl_xor(st.den[r], 32);
    }
    __syncthreads();  // the stages and limbs are dead: the LDS becomes the merge area

    // One merge stage: waves 1..3 publish, wave 0 absorbs them in wave order.
    float *xo = L.u.merge;                      // [3][R * 16][PA_QS]
    float *xm = L.u.merge + 3 * R * 16 * PA_QS;  // [3][R * 16]
    float *xd = xm + 3 * R * 16;                 // [3][R * 16]
    if (wave != 0) {
        const uint32_t slot = wave - 1;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = slot * R * 16 + 16 * r + li;
            if (lg == 0) {
                xm[row] = st.m[r];
                xd[row] = st.den[r];
            }
#pragma unroll
            for (int b = 0; b < 4; b++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    *(float4 *)&xo[row * PA_QS + 64 * b + 16 * lg + 4 * i] =
                        make_float4(st.o[r][4 * b][i], st.o[r][4 * b + 1][i], st.o[r][4 * b + 2][i], st.o[r][4 * b + 3][i]);
        }
    }
    __syncthreads();
    if (wave != 0) return;
    // Partial layout: [kv head][split][query][PA_HD]; stats [kv head][split][query][2].
    const size_t base = ((size_t)h * a.splits + split) * a.queries;
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t qi = 16 * r + li;
        float mm = st.m[r];
#pragma unroll
        for (int w = 0; w < 3; w++) mm = fmaxf(mm, xm[w * R * 16 + 16 * r + li]);
        float f[4];
        f[0] = mm == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(st.m[r] - mm);
        float den = st.den[r] * f[0];
#pragma unroll
        for (int w = 0; w < 3; w++) {
            const uint32_t row = w * R * 16 + 16 * r + li;
            f[w + 1] = mm == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(xm[row] - mm);
            den += xd[row] * f[w + 1];
        }
        float *dst = a.part_out + (base + qi) * PA_HD;
#pragma unroll
        for (int b = 0; b < 4; b++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t d = 64 * b + 16 * lg + 4 * i;
                float4 v = make_float4(st.o[r][4 * b][i] * f[0], st.o[r][4 * b + 1][i] * f[0],
                                       st.o[r][4 * b + 2][i] * f[0], st.o[r][4 * b + 3][i] * f[0]);
#pragma unroll
                for (int w = 0; w < 3; w++) {
                    const float4 x = *(const float4 *)&xo[(w * R * 16 + 16 * r + li) * PA_QS + d];
                    v.x += x.x * f[w + 1];
                    v.y += x.y * f[w + 1];
                    v.z += x.z * f[w + 1];
                    v.w += x.w * f[w + 1];
                }
                if (qi < a.queries) *(float4 *)&dst[d] = v;
            }
        if (qi < a.queries && lg == 0) {
            a.part_stats[2 * (base + qi)] = mm * PA_LN2;  // the combine works in natural units
            a.part_stats[2 * (base + qi) + 1] = den;
        }
    }
}


template <int R>
__device__ __forceinline__ void paged_gqa_partial(const GqaArgs &a) {
    __shared__ PaLds<R> L;
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t li = lane & 15, lg = lane >> 4;
    const uint32_t h = blockIdx.y, split = blockIdx.x;
    const uint32_t gw = split * 4 + wave;
    const uint32_t t0 = gw * a.tiles_per_wave;
    const uint32_t t1 = min(t0 + a.tiles_per_wave, a.tiles);
    pa_prep_queries<R>(a, h, (int8_t *)L.main, L.qsc, L.xs);
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
            st.xst[r][b] = st.xsum[r][b][0] + 256 * st.xsum[r][b][1] + 65536 * st.xsum[r][b][2];
            st.corr[r][b] = 0.0f;
        }

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
// Page-aligned tiles (page_tokens % 16 == 0): P.V on f16 MFMA.
extern "C" __global__ __launch_bounds__(256, 2) void ctox_paged_gqa_partial16_r1_gfx950(GqaArgs a) {
    paged_gqa_partial16<1>(a);
}
extern "C" __global__ __launch_bounds__(256, 1) void ctox_paged_gqa_partial16_r2_gfx950(GqaArgs a) {
    paged_gqa_partial16<2>(a);
}

#define PA_MAX_SPLITS 1024

// grid (queries, kv heads, 4 dim quarters), 256 threads. Split weights
// exp(m_s - M) are formed once in LDS; thread (g = tid / 16, c = tid % 16)
// sums the float4 at dims 64 quarter + 4 c over splits g, g + 16, ..., and
// the 16 split groups are added in a fixed order.
// out[row][q head][dim] with q head = kv head * group + member.
extern "C" __global__ __launch_bounds__(256) void ctox_paged_gqa_combine_gfx950(GqaArgs a) {
    __shared__ float wgt[PA_MAX_SPLITS];
    __shared__ float red[4];
    __shared__ float4 acc4[16][16];
    const uint32_t qi = blockIdx.x, h = blockIdx.y, quarter = blockIdx.z, tid = threadIdx.x;
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
    const uint32_t g = tid >> 4, c = tid & 15;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 8
    for (uint32_t s = g; s < a.splits; s += 16) {
        const float f = wgt[s];
        const float4 v = ((const float4 *)(a.part_out + (base + (size_t)s * a.queries) * PA_HD + 64 * quarter))[c];
        acc.x += v.x * f;
        acc.y += v.y * f;
        acc.z += v.z * f;
        acc.w += v.w * f;
    }
    acc4[g][c] = acc;
    __syncthreads();
    const uint32_t t = qi / a.group, gm = qi - t * a.group, head = h * a.group + gm;
    __shared__ float stv[64];
    if (tid < 16) {
        float4 sum = acc4[0][tid];
#pragma unroll
        for (int k = 1; k < 16; k++) {
            const float4 v = acc4[k][tid];
            sum.x += v.x;
            sum.y += v.y;
            sum.z += v.z;
            sum.w += v.w;
        }
        const float inv = den > 0.0f ? 1.0f / den : 0.0f;
        const float4 o = make_float4(sum.x * inv, sum.y * inv, sum.z * inv, sum.w * inv);
        float4 *out = (float4 *)(a.out + ((size_t)t * a.query_heads + head) * PA_HD + 64 * quarter);
        out[tid] = o;
        *(float4 *)&stv[4 * tid] = o;
    }
    if (!a.st_xa) return;
    // The o projection's staged input for this 64-column block (wave 0).
    __syncthreads();
    if (tid >= 64) return;
    const uint32_t col = head * PA_HD + 64 * quarter + tid;
    const float gt = a.st_gate[(size_t)t * a.st_gate_stride + head * 2 * PA_HD + PA_HD + 64 * quarter + tid];
    float x = stv[tid] * (1.0f / (1.0f + expf(-gt)));
    if (a.st_s_in) x *= half_bits_to_float(a.st_s_in[col]);
    const uint32_t blk = col / 64;
    stage_block(x, a.st_xa + ((size_t)blk * a.rows + t) * 192, (float4 *)a.st_xc + (size_t)blk * a.rows + t, a.st_dtype,
                tid);
}

// ---------------------------------------------------------------------------
// Fused attention-layer prep: grid (qh + 2 kh, rows), one wave per (head, row).
//   q head: RMS norm with q_norm ((1 + w), Q/src/reference.rs:38-62, as
//           ctox_norm_rows_gfx950 sums it for a 256-wide row), partial RoPE
//           (Q/src/reference.rs:115-155, as ctox_rope_gfx950), written to q_out;
//   k head: the same with k_norm, then its four 64-value blocks packed into
//           the row's Q4 page slot (as ctox_kv_pack_q4_gfx950);
//   v head: packed as it is.
// Replaces the norm, norm, rope, copy, pack and descriptor-write launches of
// an attention layer's K/V append (Q/src/decoder.rs:687-800,
// Q/src/kv_cache.rs:200-206).
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(64) void ctox_attn_prep_gfx950(AttnPrepArgs a) {
    __shared__ float hs[PA_HD];
    const uint32_t job = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    // The cache's changed page descriptors, carried in the arguments.
    if (job == 0 && t == 0 && a.desc_dst && lane < a.desc_words) a.desc_dst[lane] = a.desc[lane];
    const bool is_q = job < a.qh, is_k = !is_q && job < a.qh + a.kh;
    const uint32_t kk = is_q ? job : is_k ? job - a.qh : job - a.qh - a.kh;
    const float *row = a.proj + (size_t)t * a.proj_stride;
    const float *x = is_q ? row + (size_t)kk * 2 * a.hd
                          : row + (size_t)2 * a.qh * a.hd + (is_k ? 0 : (size_t)a.kh * a.hd) + (size_t)kk * a.hd;
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) v[k] = x[lane + 64 * k];
    if (is_q || is_k) {
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) s += v[k] * v[k];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
        const float inv = 1.0f / sqrtf(s / (float)a.hd + a.eps);
        const float *w = is_q ? a.q_norm : a.k_norm;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float n = v[k] * inv;
            hs[lane + 64 * k] = n * (1.0f + w[lane + 64 * k]);
        }
        __syncthreads();
        const uint32_t half = a.rd / 2;
        for (uint32_t i = lane; i < half; i += 64) {
            const float invf = powf(a.theta, -((float)(2 * i)) / (float)a.rd);
            const float angle = (float)(a.position + t) * invf;  // u64 -> f32, as `position as f32`
            const float cs = cosf(angle), sn = sinf(angle);
            const float l = hs[i], r = hs[i + half];
            hs[i] = l * cs - r * sn;
            hs[i + half] = r * cs + l * sn;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = hs[lane + 64 * k];
        if (is_q) {
            float *q = a.q_out + ((size_t)t * a.qh + kk) * a.hd;
#pragma unroll
            for (int k = 0; k < 4; k++) q[lane + 64 * k] = v[k];
            return;
        }
    }
    // Blocks of this head inside the token: K blocks [0, 4 kh), V blocks after.
    uint8_t *tok = a.q4_pages + (size_t)a.slot[t] * a.q4_page_bytes + (size_t)a.pos[t] * a.q4_token_bytes;
    const uint32_t blk0 = (is_k ? 0u : 4u * a.kh) + 4 * kk;
#pragma unroll
    for (int k = 0; k < 4; k++) pa_pack_q4_block(v[k], lane, tok + (size_t)(blk0 + k) * 34);
}
