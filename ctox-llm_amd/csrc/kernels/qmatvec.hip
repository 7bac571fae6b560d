// Fused Q2_B64 / Q4_B64 dequantize-matvec for gfx950 (CDNA4), batch 1..8.
//
// Computes, for every token m < batch and row r (Q/src/backend/cpu.rs:242-310):
//   y[m][r] = act((sum_b scale[r,b] * sum_{i<64} w(c) * x'[m][64b+i] + bias[r]) * s_out[r])
// with x' = x * s_in (Q/src/backend/cpu.rs:228-240), w(c) = (2c-15)/15 for
// Q4 and (2c-3)/3 for Q2 (Q/src/quant.rs:107-111, 171-175; the same folding
// the crate's AVX2 path uses, Q/src/backend/cpu.rs:595-658).
//
// Design (MI355X-first, not a translation of the SM86 warp-per-row kernel):
//  * Weights stay in the crate's packed CTOXQ layout (34- / 18-byte blocks,
//    rows dense). Each wave stages 16 rows x 16 blocks of packed bytes into
//    LDS with 128-bit buffer loads (hardware bounds-checked), so HBM is read
//    with coalesced aligned 16-byte accesses although blocks are only 2-byte
//    aligned. Lane (row = lane/4, part = lane%4) owns units part, part+4, ...
//    of one row, so the staging addresses are per-lane constants plus
//    immediates.
//  * The contraction runs on the int8 matrix cores (v_mfma_i32_16x16x64_i8):
//    B = 16 rows x 64 codes (codes 0..15 / 0..3 unpacked with mask ops), A =
//    the activation as exact fixed point: per 64-column block X = x'/q with
//    q = 2^(e-22), split into three signed 8-bit limbs (A rows). Integer
//    products are exact; the only rounding is x' -> X (at most 2^-23 of the
//    block maximum) and the fp32 epilogue, so results agree with the fp32
//    scalar oracle to ~1e-6 relative.
//  * Batch 1 ("block-diagonal"): A row group t (rows 4t..4t+2) carries the
//    limbs of block t of a 4-block group, and only in k-group t; B k-group g
//    carries quarter q of block g. Four MFMAs (q = 0..3) accumulate the four
//    blocks' full 64-element sums, and C lane (g, j) ends up owning
//    (block g, row j): every lane does useful dequant work.
//  * Batch 2..8 ("token-stacked"): A rows 4t..4t+2 are token t's limbs of
//    the current block; C lane (g, j) owns (token g, row j).
//  * Per-block epilogue: f = 2q*C0 + 512q*C1 + 131072q*C2 + K*q with
//    K = -off*sum(X); acc += scale * f.
//  * K is split into chunks of 16 blocks across workgroups; the last
//    workgroup of a row group sums the partials in a fixed association
//    (deterministic) and applies bias, s_out and the activation.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "kernel_args.h"
#include "lds_barrier.h"

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)h));
}

__device__ __forceinline__ float load_scale(const void *p, uint32_t kind, uint32_t i) {
    if (kind == CTOX_KSCALE_F32) return ((const float *)p)[i];
    if (kind == CTOX_KSCALE_F16) return half_bits_to_float(((const uint16_t *)p)[i]);
    return 1.0f;
}

// Reductions over one 16-lane row with DPP (VALU speed, no LDS round
// trips): quad xor 1, quad xor 2, half-row mirror, row mirror; every lane
// of the row ends with the result.
template <typename T, typename F>
__device__ __forceinline__ T row16_reduce(T v, F op) {
    v = op(v, __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
    v = op(v, __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
    v = op(v, __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)));
    v = op(v, __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)));
    return v;
}
// The same over the whole wave: rows, then row pairs and halves with
// permlane swaps (every lane ends with the result). For max and integer
// sums the result does not depend on the order.
template <typename T, typename F>
__device__ __forceinline__ T wave64_reduce(T v, F op) {
    v = row16_reduce(v, op);
    const int b = __builtin_bit_cast(int, v);
    const auto s16 = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    v = op(__builtin_bit_cast(T, (int)s16[0]), __builtin_bit_cast(T, (int)s16[1]));
    const int c = __builtin_bit_cast(int, v);
    const auto s32 = __builtin_amdgcn_permlane32_swap(c, c, false, false);
    return op(__builtin_bit_cast(T, (int)s32[0]), __builtin_bit_cast(T, (int)s32[1]));
}
// Buffer resource over `bytes` bytes at p (none when p is NULL): reads past
// the end return 0, so operand loads need no branch around them.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t pv_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, p ? (int)bytes : 0, 0x00020000);
}
__device__ __forceinline__ float wave_max(float v) {
    return wave64_reduce(v, [](float x, float y) { return fmaxf(x, y); });
}

// Byte position v (0..15) inside a lane's 16-byte fragment that holds
// element w (0..15) of a 16-element quarter block. The B-fragment unpack
// order is Q4: [0,2,4,..,14, 1,3,..,15] (low nibbles then high nibbles);
// Q2: [0,4,8,12, 1,5,9,13, 2,6,10,14, 3,7,11,15] (crumb planes).
__device__ __forceinline__ int frag_pos(uint32_t dtype, int w) {
    return dtype ? ((w & 1) ? 8 + (w >> 1) : (w >> 1)) : ((w & 3) * 4 + (w >> 2));
}

// One wave (64 threads) per (block, token). Output layout:
//   xa: [block][token][limb 0..2][quarter 0..3][16 bytes]
//   xc: [block][token] float4 {2q, 512q, 131072q, K*q}, K = -off*sum(X)
// Stages one 64-value block from one value per lane (x already multiplied
// by s_in; element e of the block in lane e): its three limbs go to frag
// (192 bytes, the xa order above) and, from lane 0, its constants to *xc.
// Every lane of the wave takes part.
__device__ __forceinline__ void stage_block(float x, int8_t *frag, float4 *xc, uint32_t dtype, uint32_t e) {
    const bool bad = !__builtin_isfinite(x);
    const bool any_bad = __any(bad);
    const float m = wave_max(bad ? 0.0f : fabsf(x));
    int X = 0;
    float q = 0.0f;
    if (any_bad) {
        q = __builtin_nanf("");
    } else if (m > 0.0f) {
        int ex;
        frexpf(m, &ex);
        X = (int)rintf(ldexpf(x, ctox_staged_xfrac_bits(dtype) - ex));
        q = ldexpf(1.0f, ex - ctox_staged_xfrac_bits(dtype));
    }
    // Balanced signed limbs: X = X0 + 256*X1 + 65536*X2, X0, X1 in [-128,127].
    const int x0 = (int)(int8_t)(X & 0xff);
    const int r1 = (X - x0) >> 8;
    const int x1 = (int)(int8_t)(r1 & 0xff);
    const int x2 = (r1 - x1) >> 8;
    // sum(X) = sum(X0) + 256 sum(X1) + 65536 sum(X2); |X| <= 2^22, so the
    // 64-lane sum fits int32.
    const int sxw = wave64_reduce(X, [](int p, int q) { return p + q; });

    const uint32_t g = e >> 4, w = e & 15;
    const int v = frag_pos(dtype, (int)w);
    frag[(0 * 4 + g) * 16 + v] = (int8_t)x0;
    frag[(1 * 4 + g) * 16 + v] = (int8_t)x1;
    frag[(2 * 4 + g) * 16 + v] = (int8_t)x2;
    if (e == 0) {
        const long long sx = sxw;
        const long long off = dtype ? 15 : 3;
        float4 c;
        c.x = 2.0f * q;
        c.y = 512.0f * q;
        c.z = 131072.0f * q;
        c.w = (float)(-off * sx) * q;
        *xc = c;
    }
}

// Prepares one 64-value block of token t from one value per lane (x already
// multiplied by s_in); every lane of the wave takes part.
__device__ __forceinline__ void prep_block(const PrepArgs &a, float x, uint32_t b, uint32_t t, uint32_t e) {
    stage_block(x, a.xa + ((size_t)b * a.batch + t) * (3 * 64), (float4 *)a.xc + (size_t)b * a.batch + t, a.dtype, e);
}

extern "C" __global__ __launch_bounds__(64) void ctox_prep_activation_gfx950(PrepArgs a) {
    const uint32_t b = blockIdx.x, t = blockIdx.y, e = threadIdx.x;
    const uint32_t col = b * CTOX_BLOCK_LEN + e;
    float x = a.input[(size_t)t * a.columns + col];
    if (a.s_in_kind != CTOX_KSCALE_NONE) x = x * load_scale(a.s_in, a.s_in_kind, col);
    prep_block(a, x, b, t, e);
}

// Residual add + (1 + w) RMS norm of token row t (Q/src/reference.rs:38-62),
// then the activation staging of prep_block from the normalized row.
// grid (ceil(blocks / 4), batch), 256 threads: every workgroup reduces the
// whole row's sum of squares itself (the row is L2-resident, a few KB), or
// the producer's per-tile sums of it (sq_n), then each of its four waves
// stages one 64-value block. The residual sum goes to
// x_out, so no workgroup reads a value another one has already updated.
extern "C" __global__ __launch_bounds__(256) void ctox_norm_prep_gfx950(NormPrepArgs a) {
    __shared__ float red[4];
    const uint32_t t = blockIdx.y, tid = threadIdx.x, cols = a.p.columns;
    const float *x = a.x + (size_t)t * cols;
    const float *dl = a.delta ? a.delta + (size_t)t * cols : nullptr;
    // The lane's own column (wave w stages block 4 blockIdx.x + w): its
    // operands are read first, branch-free (an absent operand reads 0), so
    // they travel with the row reads below.
    const uint32_t wave = tid >> 6, e = tid & 63;
    const uint32_t b = blockIdx.x * 4 + wave;
    const bool live = b < cols / CTOX_BLOCK_LEN;
    const uint32_t col = (live ? b : 0u) * CTOX_BLOCK_LEN + e;
    const uint32_t np = a.delta ? a.delta_parts : 0u;
    const __amdgpu_buffer_rsrc_t xr = pv_rsrc(x, 4 * cols), wr = pv_rsrc(a.w, 4 * cols);
    const __amdgpu_buffer_rsrc_t dr = pv_rsrc(dl, np ? 4 * ((np - 1) * a.delta_stride + cols) : 0u);
    const bool s16 = a.p.s_in_kind == CTOX_KSCALE_F16, s32 = a.p.s_in_kind == CTOX_KSCALE_F32;
    const __amdgpu_buffer_rsrc_t sr16 = pv_rsrc(s16 ? a.p.s_in : nullptr, 2 * cols);
    const __amdgpu_buffer_rsrc_t sr32 = pv_rsrc(s32 ? a.p.s_in : nullptr, 4 * cols);
    const float xv0 = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(xr, col * 4, 0, 0));
    float dv[8];
#pragma unroll
    for (int p = 0; p < 8; p++)
        dv[p] = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(
            dr, ((uint32_t)p < np ? p * a.delta_stride + col : 0x3fffffffu) * 4, 0, 0));
    const float wv = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(wr, col * 4, 0, 0));
    const uint32_t sv16 = __builtin_amdgcn_raw_buffer_load_b16(sr16, col * 2, 0, 0);
    const uint32_t sv32 = __builtin_amdgcn_raw_buffer_load_b32(sr32, col * 4, 0, 0);
    float s = 0.0f;
    const uint32_t n4 = cols / 4;
    if (a.sq_n) {
        // The producer's per-tile sums of squares of this row (at most 512).
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const uint32_t i = tid + 256 * k;
            s += i < a.sq_n ? a.sq_in[(size_t)t * a.sq_n + i] : 0.0f;
        }
    } else {
        // Every load of a thread's row share (up to 8 float4 per array, all parts)
        // is issued before the first use; parts are added in part order.
#define NP_V4 8
#define NP_PARTS 8
        float4 v[NP_V4];
#pragma unroll
        for (int k = 0; k < NP_V4; k++) {
            const uint32_t i = tid + 256 * k;
            v[k] = i < n4 ? ((const float4 *)x)[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        if (dl) {
            float4 d[NP_V4];
#pragma unroll
            for (int k = 0; k < NP_V4; k++) {
                const uint32_t i = tid + 256 * k;
                d[k] = i < n4 ? ((const float4 *)dl)[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
            for (int p = 1; p < NP_PARTS; p++) {
                if ((uint32_t)p < a.delta_parts) {
#pragma unroll
                    for (int k = 0; k < NP_V4; k++) {
                        const uint32_t i = tid + 256 * k;
                        if (i < n4) {
                            const float4 d2 = ((const float4 *)(dl + (size_t)p * a.delta_stride))[i];
                            d[k].x += d2.x;
                            d[k].y += d2.y;
                            d[k].z += d2.z;
                            d[k].w += d2.w;
                        }
                    }
                }
            }
#pragma unroll
            for (int k = 0; k < NP_V4; k++) {
                v[k].x += d[k].x;
                v[k].y += d[k].y;
                v[k].z += d[k].z;
                v[k].w += d[k].w;
            }
        }
#pragma unroll
        for (int k = 0; k < NP_V4; k++) s += v[k].x * v[k].x + v[k].y * v[k].y + v[k].z * v[k].z + v[k].w * v[k].w;
    }
    s = wave64_reduce(s, [](float p, float q) { return p + q; });
    if ((tid & 63) == 0) red[tid >> 6] = s;
    lds_barrier();
    const float inv = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)cols + a.eps);
    if (!live) return;
    float xv = xv0;
    if (dl) {
        float d = dv[0];
#pragma unroll
        for (int p = 1; p < 8; p++)
            if ((uint32_t)p < np) d += dv[p];
        xv += d;
        a.x_out[(size_t)t * cols + col] = xv;
    }
    const float y = xv * inv * (1.0f + wv);
    if (a.out) a.out[(size_t)t * cols + col] = y;
    const float sc = s16 ? half_bits_to_float(sv16 & 0xffffu) : (s32 ? __int_as_float(sv32) : 1.0f);
    prep_block(a.p, a.p.s_in_kind != CTOX_KSCALE_NONE ? y * sc : y, b, t, e);
}

// Activation staging of a value computed on the fly (one wave per 64-value
// block and token, as the prep kernel): the producer of a projection's input
// fused into its staging.
//   mode 1  swiglu:   x = silu(a[t][c]) * a[t][off + c]       Q/src/reference.rs:96-112
//   mode 2  gated norm per head of head_dim values:
//           x = a[t][c] * rsqrt(mean_head(a^2) + eps) * w[c % head_dim] * silu(b[t][c])
//                                                            Q/src/reference.rs:66-93
//   mode 3  attention gate: x = a[t][c] * sigmoid(b[t][h * 2 hd + hd + d]),
//           h = c / head_dim, d = c % head_dim              Q/src/decoder.rs:727-737, :788
// a rows are a_stride floats apart, b rows b_stride; in mode 1 a may be
// a_parts partials a_pstride floats apart, added in part order.
__device__ __forceinline__ float px_silu(float v) { return v / (1.0f + expf(-v)); }

extern "C" __global__ __launch_bounds__(64) void ctox_prep_transform_gfx950(PrepXArgs a) {
    const uint32_t b = blockIdx.x, t = blockIdx.y, e = threadIdx.x, cols = a.p.columns;
    const uint32_t col = b * CTOX_BLOCK_LEN + e, m = a.mode, hd = a.head_dim;
    // Every operand goes out before the first use, branch-free (an operand
    // the mode does not use has an empty range and reads 0).
    const uint32_t np = m == 1 ? (a.a_parts > 1 ? a.a_parts : 1u) : 0u;
    const __amdgpu_buffer_rsrc_t ar =
        pv_rsrc(a.a + (size_t)t * a.a_stride, 4 * (m == 1 ? (np - 1) * a.a_pstride + a.off + cols : cols));
    const __amdgpu_buffer_rsrc_t br = pv_rsrc(m == 1 ? nullptr : a.b + (size_t)t * a.b_stride, 4 * (m == 3 ? 2 * cols : cols));
    const __amdgpu_buffer_rsrc_t wr = pv_rsrc(m == 2 ? a.w : nullptr, 4 * hd);
    const bool s16 = a.p.s_in_kind == CTOX_KSCALE_F16, s32 = a.p.s_in_kind == CTOX_KSCALE_F32;
    const __amdgpu_buffer_rsrc_t sr16 = pv_rsrc(s16 ? a.p.s_in : nullptr, 2 * cols);
    const __amdgpu_buffer_rsrc_t sr32 = pv_rsrc(s32 ? a.p.s_in : nullptr, 4 * cols);
    const uint32_t oob = 0x3fffffffu;  // a float index past every range (byte offset stays below 2^32)
    // mode 1: the parts of a[col] and a[off + col]; modes 2, 3: a[col]
    float pa[6], pu[6];
#pragma unroll
    for (int k = 0; k < 6; k++) {
        const bool in = (uint32_t)k < (m == 1 ? np : 1u);
        pa[k] = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(ar, (in ? k * a.a_pstride + col : oob) * 4, 0, 0));
        pu[k] = __int_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(ar, (in && m == 1 ? k * a.a_pstride + a.off + col : oob) * 4, 0, 0));
    }
    // mode 2: this head's values (head_dim <= 256 here), the gate z and the norm weight
    const uint32_t head0 = m == 2 ? col / hd * hd : 0u;
    float hv[4];
#pragma unroll
    for (int k = 0; k < 4; k++)
        hv[k] = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(
            ar, (m == 2 && e + 64 * k < hd ? head0 + e + 64 * k : oob) * 4, 0, 0));
    const uint32_t hh = m == 3 ? col / hd : 0u, dd = m == 3 ? col % hd : 0u;
    const float g = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(
        br, (m == 3 ? hh * 2 * hd + hd + dd : col) * 4, 0, 0));
    const float wv = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(wr, (m == 2 ? col % hd : 0u) * 4, 0, 0));
    const uint32_t sv16 = __builtin_amdgcn_raw_buffer_load_b16(sr16, col * 2, 0, 0);
    const uint32_t sv32 = __builtin_amdgcn_raw_buffer_load_b32(sr32, col * 4, 0, 0);
    float x;
    if (m == 1) {
        // A producer's chunk partials are added in part order.
        float ga = pa[0], ua = pu[0];
#pragma unroll
        for (int k = 1; k < 6; k++)
            if ((uint32_t)k < np) {
                ga += pa[k];
                ua += pu[k];
            }
        x = px_silu(ga) * ua;
    } else if (m == 2) {
        float ss = 0.0f;
        if (hd <= 256) {
#pragma unroll
            for (int k = 0; k < 4; k++) ss += hv[k] * hv[k];  // zeros past the head
        } else {
            const float *arow = a.a + (size_t)t * a.a_stride;
            for (uint32_t i = e; i < hd; i += 64) {  // this head's values, same order for every wave
                const float v = arow[head0 + i];
                ss += v * v;
            }
        }
        ss = wave64_reduce(ss, [](float p, float q) { return p + q; });
        const float inv = 1.0f / sqrtf(ss / (float)hd + a.eps);
        x = pa[0] * inv * wv * px_silu(g);
    } else {
        x = pa[0] * (1.0f / (1.0f + expf(-g)));
    }
    if (a.p.s_in_kind != CTOX_KSCALE_NONE) x = x * (s16 ? half_bits_to_float(sv16 & 0xffffu) : __int_as_float(sv32));
    prep_block(a.p, x, b, t, e);
}

template <int DT, int MODE>  // MODE 0: batch 1, 1: batch 2..4, 2: batch 5..8
struct MvCfg {
    static constexpr int BB = DT ? CTOX_Q4_BLOCK_BYTES : CTOX_Q2_BLOCK_BYTES;
    static constexpr int QB = DT ? 8 : 4;                    // code bytes per quarter block
    static constexpr int CD = DT ? 8 : 4;                    // code dwords per block
    static constexpr int CB = MODE == 0 ? 16 : 8;            // blocks per chunk
    static constexpr int MAXB = MODE == 0 ? 1 : (MODE == 1 ? 4 : 8);
    static constexpr int TG = MODE == 2 ? 2 : 1;
    static constexpr int UMAX = (15 + CB * BB + 15) / 16;    // 16-byte units per staged row
    static constexpr int STRIDE = UMAX * 16;                 // LDS bytes per staged row
    static constexpr int ROUNDS = (UMAX + 3) / 4;            // staging loads per lane
    static constexpr int XA_UNITS = CB * MAXB * 12;          // 16-byte units of fragments
    static constexpr int XA_ROUNDS = (XA_UNITS + 63) / 64;
    static constexpr int XC_N = CB * MAXB;
    static constexpr float DEN = DT ? 15.0f : 3.0f;
};

// Per-wave LDS: staged rows of the current chunk, its activation fragments
// and block constants.
template <int DT, int MODE>
struct MvWave {
    using C = MvCfg<DT, MODE>;
    uint8_t rows[16 * C::STRIDE + 64];  // +64: the last block's dword reads may run 12 bytes past
    int8_t xa[C::CB * C::MAXB * 192];
    float4 xc[C::XC_N];
};

template <int DT, int MODE>
struct MvShared {
    MvWave<DT, MODE> w[CTOX_MV_WAVES];
    int8_t zero[MODE == 0 ? 3 * 1024 + 64 : 16];  // zero A fragments (batch 1)
    float red[CTOX_MV_WAVES][MvCfg<DT, MODE>::MAXB][16];
};

__device__ __forceinline__ float epilogue(float v, uint32_t row, const MatvecArgs &a) {
    if (a.bias) v += a.bias[row];
    if (a.s_out_kind != CTOX_KSCALE_NONE) v *= load_scale(a.s_out, a.s_out_kind, row);
    if (a.activation == 1) v = v / (1.0f + expf(-v));
    return v;
}

// B fragment (16 codes as int8) of one quarter block from its code dword(s).
template <int DT>
__device__ __forceinline__ v4i unpack_quarter(uint32_t w0, uint32_t w1) {
    if (DT)
        return (v4i){(int)(w0 & 0x0f0f0f0fu), (int)(w1 & 0x0f0f0f0fu), (int)((w0 >> 4) & 0x0f0f0f0fu),
                     (int)((w1 >> 4) & 0x0f0f0f0fu)};
    return (v4i){(int)(w0 & 0x03030303u), (int)((w0 >> 2) & 0x03030303u), (int)((w0 >> 4) & 0x03030303u),
                 (int)((w0 >> 6) & 0x03030303u)};
}

// Register copy of one chunk in flight (weights, fragments, constants).
template <int DT, int MODE>
struct MvPrefetch {
    using C = MvCfg<DT, MODE>;
    v4i rows[C::ROUNDS];
    v4i xa[C::XA_ROUNDS];
    float4 xc;
};

// Issues the global loads of chunk [cb0, cb0 + nbc) for this wave.
template <int DT, int MODE>
__device__ __forceinline__ void mv_fetch(MvPrefetch<DT, MODE> &pf, const MatvecArgs &a,
                                         __amdgpu_buffer_rsrc_t rsrc, uint32_t P, uint32_t rowbytes,
                                         uint32_t rows_here, uint32_t cb0, uint32_t nbc, uint32_t lane) {
    using C = MvCfg<DT, MODE>;
    const uint32_t srow = lane >> 2, part = lane & 3;
    const uint32_t o = P + srow * rowbytes + cb0 * C::BB;
    const uint32_t nu = ((o & 15) + nbc * C::BB + 15) >> 4;
    const bool rowok = srow < rows_here;
    const uint32_t gbase = ((o >> 4) + part) * 16;
#pragma unroll
    for (int it = 0; it < C::ROUNDS; it++) {
        pf.rows[it] = (v4i){0, 0, 0, 0};
        if (rowok && part + 4 * it < nu)
            pf.rows[it] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, gbase + it * 64, 0, 0);
    }
    const uint32_t nxa = nbc * a.batch * 12;
    const v4i *src = (const v4i *)(a.xa + (size_t)cb0 * a.batch * 192);
#pragma unroll
    for (int it = 0; it < C::XA_ROUNDS; it++) {
        const uint32_t u = it * 64 + lane;
        pf.xa[it] = u < nxa ? src[u] : (v4i){0, 0, 0, 0};
    }
    pf.xc = lane < nbc * a.batch ? ((const float4 *)a.xc)[(size_t)cb0 * a.batch + lane]
                                 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

template <int DT, int MODE>
__device__ __forceinline__ void mv_store(const MvPrefetch<DT, MODE> &pf, MvWave<DT, MODE> &wl, uint32_t lane) {
    using C = MvCfg<DT, MODE>;
    const uint32_t srow = lane >> 2, part = lane & 3;
#pragma unroll
    for (int it = 0; it < C::ROUNDS; it++)
        if (part + 4 * it < (uint32_t)C::UMAX) *(v4i *)(wl.rows + srow * C::STRIDE + part * 16 + it * 64) = pf.rows[it];
#pragma unroll
    for (int it = 0; it < C::XA_ROUNDS; it++) {
        const uint32_t u = it * 64 + lane;
        if (u < (uint32_t)C::XA_UNITS) ((v4i *)wl.xa)[u] = pf.xa[it];
    }
    if (lane < (uint32_t)C::XC_N) wl.xc[lane] = pf.xc;
}

// Workgroup = 16 rows; wave w covers quant blocks [w*nb/4, (w+1)*nb/4) of
// those rows in chunks of CB blocks, prefetching chunk c+1 into registers
// while chunk c is computed from LDS. The four wave partials are added in
// LDS in fixed order, so results are deterministic.
template <int DT, int MODE>
__device__ __forceinline__ void qmatvec_body(const MatvecArgs &a) {
    using C = MvCfg<DT, MODE>;
    constexpr int TG = C::TG;
    __shared__ __align__(16) MvShared<DT, MODE> sh;

    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t nblocks = a.columns / CTOX_BLOCK_LEN;
    const uint32_t rowbytes = nblocks * C::BB;
    const uint32_t r0 = blockIdx.x * 16;
    const uint32_t rows_here = min(16u, a.rows - r0);
    const uint32_t wb0 = wave * nblocks / CTOX_MV_WAVES, wb1 = (wave + 1) * nblocks / CTOX_MV_WAVES;
    const uint32_t nchunks = (wb1 - wb0 + C::CB - 1) / C::CB;
    MvWave<DT, MODE> &wl = sh.w[wave];

    const uint64_t wg_off = (uint64_t)r0 * rowbytes;
    const uintptr_t base = (uintptr_t)a.weights + wg_off;
    const uintptr_t aligned = base & ~(uintptr_t)15;
    const uint32_t P = (uint32_t)(base - aligned);
    // The buffer range check rejects a whole 16-byte load that straddles
    // num_records, so the range is rounded up to the 16-byte granule that
    // holds the last weight byte. That granule lies inside the same page as
    // the last byte (pages are 16-byte aligned), so the extra bytes are
    // mapped; they are never used.
    const uint64_t remain = (a.weights_len - wg_off + P + 15) & ~15ULL;
    const int nrec = (int)(remain > 0x7ffffff0ULL ? 0x7ffffff0ULL : remain);
    __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)aligned, (short)0, nrec, 0x00020000);

    if (MODE == 0) {
        for (uint32_t i = threadIdx.x; i < sizeof(sh.zero) / 16; i += blockDim.x)
            ((v4i *)sh.zero)[i] = (v4i){0, 0, 0, 0};
        __syncthreads();
    }

    const uint32_t g = lane >> 4, j = lane & 15;
    const uint32_t *lds32 = (const uint32_t *)wl.rows;
    const uint16_t *lds16 = (const uint16_t *)wl.rows;
    float acc[TG];
#pragma unroll
    for (int tg = 0; tg < TG; tg++) acc[tg] = 0.0f;

    MvPrefetch<DT, MODE> pf;
    if (nchunks > 0) mv_fetch<DT, MODE>(pf, a, rsrc, P, rowbytes, rows_here, wb0, min((uint32_t)C::CB, wb1 - wb0), lane);
    for (uint32_t c = 0; c < nchunks; c++) {
        const uint32_t cb0 = wb0 + c * C::CB;
        const uint32_t nbc = min((uint32_t)C::CB, wb1 - cb0);
        mv_store<DT, MODE>(pf, wl, lane);
        // LDS operations of one wave complete in issue order; the fence only
        // keeps the compiler from moving the reads below above the writes.
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        if (c + 1 < nchunks)
            mv_fetch<DT, MODE>(pf, a, rsrc, P, rowbytes, rows_here, cb0 + C::CB,
                               min((uint32_t)C::CB, wb1 - cb0 - C::CB), lane);
        const uint32_t ph = (P + j * rowbytes + cb0 * C::BB) & 15;
        const uint32_t rowoff = j * C::STRIDE + ph;

        if (MODE == 0) {
            // Block-diagonal: lane (g, j) owns block 4G+g of row j.
            const uint32_t boff = rowoff + g * C::BB;
            const uint32_t d0 = (boff + 2) >> 2, sft = (boff + 2) & 3;
            const bool scale_hi = sft == 0;  // scale in the upper half of dword d0-1
            const uint32_t i = lane & 15, t = i >> 2, limb = i & 3;
            const bool aok = t == g && limb < 3;
            const int8_t *xab = (aok ? wl.xa : sh.zero) + g * 192 + min(limb, 2u) * 64;
            const uint32_t ngroups = (nbc + 3) >> 2;
            for (uint32_t G = 0; G < ngroups; G++) {
                constexpr int GD = C::BB;  // dwords per 4-block step (4*BB bytes)
                uint32_t d[C::CD + 2];
#pragma unroll
                for (int k = 0; k < C::CD + 2; k++) d[k] = lds32[d0 + G * GD + k - 1];
                uint32_t cd[C::CD];
#pragma unroll
                for (int k = 0; k < C::CD; k++) cd[k] = __builtin_amdgcn_alignbyte(d[k + 2], d[k + 1], sft);
                const uint32_t sbits = scale_hi ? (d[0] >> 16) : d[1];
                v4i cc = (v4i){0, 0, 0, 0};
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const v4i bf = DT ? unpack_quarter<DT>(cd[2 * q], cd[2 * q + 1]) : unpack_quarter<DT>(cd[q], 0);
                    const v4i af = *(const v4i *)(xab + G * 768 + q * 16);
                    cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf, cc, 0, 0, 0);
                }
                const float4 kq = wl.xc[G * 4 + g];
                const float scale = G * 4 + g < nbc ? half_bits_to_float(sbits) : 0.0f;
                float f = fmaf((float)cc[0], kq.x, kq.w);
                f = fmaf((float)cc[1], kq.y, f);
                f = fmaf((float)cc[2], kq.z, f);
                acc[0] = fmaf(f, scale, acc[0]);
            }
        } else {
            // Token-stacked: lane (g, j) reads quarter g of every block of row j.
            constexpr int NW = DT ? 3 : 2;
            for (uint32_t bl = 0; bl < nbc; bl++) {
                const uint32_t boff = rowoff + bl * C::BB;
                const uint32_t sbits = lds16[boff >> 1];
                const uint32_t ca = boff + 2 + C::QB * g;
                const uint32_t sftq = ca & 3;
                uint32_t cw[NW];
#pragma unroll
                for (int w = 0; w < NW; w++) cw[w] = lds32[(ca >> 2) + w];
                const uint32_t w0 = __builtin_amdgcn_alignbyte(cw[1], cw[0], sftq);
                const uint32_t w1 = DT ? __builtin_amdgcn_alignbyte(cw[NW - 1], cw[1], sftq) : 0u;
                const v4i bf = unpack_quarter<DT>(w0, w1);
                const float scale = half_bits_to_float(sbits);
#pragma unroll
                for (int tg = 0; tg < TG; tg++) {
                    const uint32_t tok = tg * 4 + (j >> 2), limb = j & 3;
                    const bool aok = limb < 3 && tok < a.batch;
                    const uint32_t tok_c = min(tok, a.batch - 1), limb_c = min(limb, 2u);
                    const v4i av = *(const v4i *)(wl.xa + ((bl * a.batch + tok_c) * 3 + limb_c) * 64 + g * 16);
                    const v4i af = aok ? av : (v4i){0, 0, 0, 0};
                    const v4i cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf, (v4i){0, 0, 0, 0}, 0, 0, 0);
                    const float4 kq = wl.xc[bl * a.batch + min((uint32_t)(tg * 4) + g, a.batch - 1)];
                    float f = fmaf((float)cc[0], kq.x, kq.w);
                    f = fmaf((float)cc[1], kq.y, f);
                    f = fmaf((float)cc[2], kq.z, f);
                    acc[tg] = fmaf(f, scale, acc[tg]);
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    }

    // Lane (g, j) owns row r0+j for token 0 (batch 1, after summing the four
    // block lanes) or token tg*4+g.
    if (MODE == 0) {
        acc[0] += __shfl_xor(acc[0], 16);
        acc[0] += __shfl_xor(acc[0], 32);
        if (g == 0) sh.red[wave][0][j] = acc[0];
    } else {
#pragma unroll
        for (int tg = 0; tg < TG; tg++) {
            const uint32_t tok = tg * 4 + g;
            if (tok < a.batch) sh.red[wave][tok][j] = acc[tg];
        }
    }
    __syncthreads();
    if (threadIdx.x < a.batch * 16) {
        const uint32_t tok = threadIdx.x >> 4, jj = threadIdx.x & 15, row = r0 + jj;
        const float s = ((sh.red[0][tok][jj] + sh.red[1][tok][jj]) + sh.red[2][tok][jj]) + sh.red[3][tok][jj];
        if (jj < rows_here) a.output[(size_t)tok * a.out_stride + row] = epilogue(s / C::DEN, row, a);
    }
}

extern "C" __global__ __launch_bounds__(256) void ctox_q4_matvec_b1_gfx950(MatvecArgs a) {
    qmatvec_body<1, 0>(a);
}
extern "C" __global__ __launch_bounds__(256) void ctox_q4_matvec_b4_gfx950(MatvecArgs a) {
    qmatvec_body<1, 1>(a);
}
extern "C" __global__ __launch_bounds__(256) void ctox_q4_matvec_b8_gfx950(MatvecArgs a) {
    qmatvec_body<1, 2>(a);
}
extern "C" __global__ __launch_bounds__(256) void ctox_q2_matvec_b1_gfx950(MatvecArgs a) {
    qmatvec_body<0, 0>(a);
}
extern "C" __global__ __launch_bounds__(256) void ctox_q2_matvec_b4_gfx950(MatvecArgs a) {
    qmatvec_body<0, 1>(a);
}
extern "C" __global__ __launch_bounds__(256) void ctox_q2_matvec_b8_gfx950(MatvecArgs a) {
    qmatvec_body<0, 2>(a);
}

// Backend::recovered_row: one thread per column (Q/src/backend/cpu.rs:312-370);
// output = ((scale * w(c)) * s_in) * s_out in the oracle's multiplication order.
extern "C" __global__ __launch_bounds__(256) void ctox_recovered_row_gfx950(RecoveredRowArgs a) {
    const uint32_t col = blockIdx.x * blockDim.x + threadIdx.x;
    if (col >= a.columns) return;
    const uint32_t b = col / CTOX_BLOCK_LEN, i = col % CTOX_BLOCK_LEN;
    float n;
    uint32_t sbits;
    if (a.dtype) {
        const uint8_t *blk = a.weights + b * CTOX_Q4_BLOCK_BYTES;
        sbits = blk[0] | (blk[1] << 8);
        const uint32_t code = (blk[2 + i / 2] >> ((i % 2) * 4)) & 0xf;
        n = ((float)code - 7.5f) / 7.5f;
    } else {
        const uint8_t *blk = a.weights + b * CTOX_Q2_BLOCK_BYTES;
        sbits = blk[0] | (blk[1] << 8);
        const uint32_t code = (blk[2 + i / 4] >> ((i % 4) * 2)) & 3;
        const float cb[4] = {-1.0f, -1.0f / 3.0f, 1.0f / 3.0f, 1.0f};
        n = cb[code];
    }
    a.output[col] = half_bits_to_float(sbits) * n * load_scale(a.s_in, a.s_in_kind, col) * a.s_out;
}

// Backend::recovered_row_matvec (Q/src/backend/cpu.rs:478-497): one wave,
// lane i owns column i of every block; per-block sums in fp32, then the
// block sums are added in block order by lane 0 like row_sum_q2/q4.
extern "C" __global__ __launch_bounds__(64) void ctox_row_dot_gfx950(RowDotArgs a) {
    const uint32_t lane = threadIdx.x;
    const uint32_t nblocks = a.len / CTOX_BLOCK_LEN;
    float total = 0.0f;
    for (uint32_t b = 0; b < nblocks; b++) {
        float term;
        uint32_t sbits;
        if (a.dtype) {
            const uint8_t *blk = a.weights + b * CTOX_Q4_BLOCK_BYTES;
            sbits = blk[0] | (blk[1] << 8);
            const uint32_t code = (blk[2 + lane / 2] >> ((lane % 2) * 4)) & 0xf;
            term = half_bits_to_float(sbits) * (((float)code - 7.5f) / 7.5f);
        } else {
            const uint8_t *blk = a.weights + b * CTOX_Q2_BLOCK_BYTES;
            sbits = blk[0] | (blk[1] << 8);
            const uint32_t code = (blk[2 + lane / 4] >> ((lane % 4) * 2)) & 3;
            const float cb[4] = {-1.0f, -1.0f / 3.0f, 1.0f / 3.0f, 1.0f};
            term = half_bits_to_float(sbits) * cb[code];
        }
        float p = term * a.x[b * CTOX_BLOCK_LEN + lane];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) p += __shfl_xor(p, o);
        total += p;
    }
    if (lane == 0) *a.result = total * a.s_out;
}
