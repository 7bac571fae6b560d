// Fused Q2_B64 / Q4_B64 dequantize-matvec for gfx950 (CDNA4), batch 1..8.
//
// Computes, for every token m < batch and row r (Q/src/backend/cpu.rs:242-310):
//   y[m][r] = act((sum_b scale[r,b] * sum_{i<64} w(c) * x'[m][64b+i] + bias[r]) * s_out[r])
// with x' = x * s_in (Q/src/backend/cpu.rs:228-240), w(c) = (2c-15)/15 for
// Q4 and (2c-3)/3 for Q2 (Q/src/quant.rs:107-111, 171-175; the same folding
// the crate's AVX2 path uses, Q/src/backend/cpu.rs:595-658).
//
// Design (MI355X-first, not a translation of the SM86 warp-per-row kernel):
//  * The weights stay in the crate's packed CTOXQ layout (34- / 18-byte
//    blocks, rows dense). Each wave stages 16 rows x 16 blocks of packed bytes
//    into LDS with 128-bit buffer loads (hardware bounds-checked), so HBM is
//    read with fully coalesced aligned 16-byte accesses even though blocks
//    are only 2-byte aligned.
//  * The contraction runs on the int8 matrix cores:
//    v_mfma_i32_16x16x64_i8 with B = 16 rows x 64 codes (one quant block,
//    codes 0..15 / 0..3 unpacked with two mask ops per dword) and A = the
//    activation as exact fixed point: per 64-column block X = x'/q with
//    q = 2^(e-22), split into three signed 8-bit limbs in A rows 4t+l.
//    The integer products are exact; the only rounding is x' -> X (at most
//    2^-23 of the block maximum) and the fp32 epilogue, so results agree with
//    the fp32 scalar oracle to ~1e-6 relative.
//  * C lane (g, j) holds limbs of token g for row j: the per-block dequant
//    epilogue f = 2*sum(c*X) - off*sum(X), acc += scale*q*f is lane-local.
//  * K is split into chunks of 16 blocks across workgroups when the row
//    count alone cannot fill 256 CUs; the last workgroup of a row group sums
//    the partials in fixed chunk order (deterministic) and applies bias,
//    s_out and the activation.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "kernel_args.h"

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)h));
}

__device__ __forceinline__ float load_scale(const void *p, uint32_t kind, uint32_t i) {
    if (kind == CTOX_KSCALE_F32) return ((const float *)p)[i];
    if (kind == CTOX_KSCALE_F16) return half_bits_to_float(((const uint16_t *)p)[i]);
    return 1.0f;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Byte position v (0..15) inside a lane's 16-byte fragment that holds
// element w (0..15) of a 16-element quarter block. The B-fragment unpack
// order is Q4: [0,2,4,..,14, 1,3,..,15] (low nibbles then high nibbles);
// Q2: [0,4,8,12, 1,5,9,13, 2,6,10,14, 3,7,11,15] (crumb planes).
__device__ __forceinline__ int frag_pos(uint32_t dtype, int w) {
    return dtype ? ((w & 1) ? 8 + (w >> 1) : (w >> 1)) : ((w & 3) * 4 + (w >> 2));
}

// One wave (64 threads) per (block, token).
extern "C" __global__ __launch_bounds__(64) void ctox_prep_activation_gfx950(PrepArgs a) {
    const uint32_t b = blockIdx.x, t = blockIdx.y, e = threadIdx.x;
    const uint32_t col = b * CTOX_BLOCK_LEN + e;
    float x = a.input[(size_t)t * a.columns + col];
    if (a.s_in_kind != CTOX_KSCALE_NONE) x = x * load_scale(a.s_in, a.s_in_kind, col);
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
        X = (int)rintf(ldexpf(x, CTOX_XFRAC_BITS - ex));
        q = ldexpf(1.0f, ex - CTOX_XFRAC_BITS);
    }
    // Balanced signed limbs: X = X0 + 256*X1 + 65536*X2, X0, X1 in [-128,127].
    const int x0 = (int)(int8_t)(X & 0xff);
    const int r1 = (X - x0) >> 8;
    const int x1 = (int)(int8_t)(r1 & 0xff);
    const int x2 = (r1 - x1) >> 8;
    const int s0 = wave_sum_i(x0), s1 = wave_sum_i(x1), s2 = wave_sum_i(x2);

    const uint32_t g = e >> 4, w = e & 15;
    const int v = frag_pos(a.dtype, (int)w);
    const uint32_t tg = t >> 2, slot = (t & 3) * 4;
    int8_t *frag = a.xa + (((size_t)b * a.tgroups + tg) * 64) * 16;
    frag[(g * 16 + slot + 0) * 16 + v] = (int8_t)x0;
    frag[(g * 16 + slot + 1) * 16 + v] = (int8_t)x1;
    frag[(g * 16 + slot + 2) * 16 + v] = (int8_t)x2;
    frag[(g * 16 + slot + 3) * 16 + v] = 0;
    if (e == 0) {
        const long long sx = (long long)s0 + 256LL * s1 + 65536LL * s2;
        const long long off = a.dtype ? 15 : 3;
        float *c = a.xc + ((size_t)b * a.batch + t) * 2;
        c[0] = q;
        c[1] = (float)(-off * sx);
    }
}

template <int DT>
struct QFmt {
    static constexpr int BB = DT ? CTOX_Q4_BLOCK_BYTES : CTOX_Q2_BLOCK_BYTES;
    static constexpr int QB = DT ? 8 : 4;                     // code bytes per quarter block
    static constexpr int UMAX = (15 + CTOX_KCHUNK * BB + 15) / 16;  // 16B units per staged row
    static constexpr int STRIDE = UMAX * 16;                  // LDS bytes per staged row
    static constexpr float DEN = DT ? 15.0f : 3.0f;
};

__device__ __forceinline__ float epilogue(float v, uint32_t row, const MatvecArgs &a) {
    if (a.bias) v += a.bias[row];
    if (a.s_out_kind != CTOX_KSCALE_NONE) v *= load_scale(a.s_out, a.s_out_kind, row);
    if (a.activation == 1) v = v / (1.0f + expf(-v));
    return v;
}

template <int DT, int TG>
__device__ __forceinline__ void qmatvec_body(const MatvecArgs &a) {
    using F = QFmt<DT>;
    // +64 bytes of slack: the 3-dword code read of the last block may touch
    // up to 12 bytes past a wave's last staged row.
    __shared__ __align__(16) uint8_t lds[CTOX_MV_WAVES * 16 * F::STRIDE + 64];
    __shared__ uint32_t s_last;

    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t nblocks = a.columns / CTOX_BLOCK_LEN;
    const uint32_t rowbytes = nblocks * F::BB;
    const uint32_t kc = blockIdx.x % a.ksplit, rg = blockIdx.x / a.ksplit;
    const uint32_t b0 = kc * CTOX_KCHUNK;
    const uint32_t nb = min((uint32_t)CTOX_KCHUNK, nblocks - b0);
    const uint32_t rbase = rg * CTOX_MV_ROWS + wave * 16;

    // ---- issue activation-fragment and per-block constant loads early ----
    const uint32_t g = lane >> 4, j = lane & 15;
    v4i afrag[CTOX_KCHUNK][TG];
    float2 xcv[CTOX_KCHUNK][TG];
#pragma unroll
    for (int bl = 0; bl < CTOX_KCHUNK; bl++) {
#pragma unroll
        for (int tg = 0; tg < TG; tg++) {
            afrag[bl][tg] = (v4i){0, 0, 0, 0};
            xcv[bl][tg] = make_float2(0.0f, 0.0f);
            if ((uint32_t)bl < nb) {
                const uint32_t slot_tok = tg * 4 + (j >> 2);
                if ((j & 3) < 3 && slot_tok < a.batch)
                    afrag[bl][tg] = ((const v4i *)a.xa)[((size_t)(b0 + bl) * a.tgroups + tg) * 64 + lane];
                const uint32_t tok = tg * 4 + g;
                if (tok < a.batch)
                    xcv[bl][tg] = ((const float2 *)a.xc)[(size_t)(b0 + bl) * a.batch + tok];
            }
        }
    }

    // ---- stage 16 rows x nb blocks of packed bytes into this wave's LDS ----
    const uint64_t wg_off = (uint64_t)rg * CTOX_MV_ROWS * rowbytes + (uint64_t)b0 * F::BB;
    const uintptr_t base = (uintptr_t)a.weights + wg_off;
    const uintptr_t aligned = base & ~(uintptr_t)15;
    const uint32_t P = (uint32_t)(base - aligned);
    const uint64_t remain = a.weights_len - wg_off + P;
    const int nrec = (int)(remain > 0x7fffffffULL ? 0x7fffffffULL : remain);
    __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void *)aligned, (short)0, nrec, 0x00020000);
    uint8_t *wlds = lds + wave * 16 * F::STRIDE;
    constexpr int ITEMS = 16 * F::UMAX;
    constexpr int ROUNDS = (ITEMS + 63) / 64;
    v4i stage[ROUNDS];
#pragma unroll
    for (int it = 0; it < ROUNDS; it++) {
        const uint32_t idx = it * 64 + lane;
        const uint32_t rj = idx / F::UMAX, u = idx % F::UMAX;
        const uint32_t o = P + (wave * 16 + rj) * rowbytes;
        const uint32_t nu = ((o & 15) + nb * F::BB + 15) >> 4;
        stage[it] = (v4i){0, 0, 0, 0};
        if (rj < 16 && u < nu && rbase + rj < a.rows)
            stage[it] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, ((o >> 4) + u) * 16, 0, 0);
    }
#pragma unroll
    for (int it = 0; it < ROUNDS; it++) {
        const uint32_t idx = it * 64 + lane;
        const uint32_t rj = idx / F::UMAX, u = idx % F::UMAX;
        if (rj < 16) *(v4i *)(wlds + rj * F::STRIDE + u * 16) = stage[it];
    }
    __syncthreads();

    // ---- one int8 MFMA per quant block, lane-local dequant epilogue ----
    const uint32_t ph = (P + (wave * 16 + j) * rowbytes) & 15;
    const uint8_t *rowl = wlds + j * F::STRIDE + ph;
    float acc[TG];
#pragma unroll
    for (int tg = 0; tg < TG; tg++) acc[tg] = 0.0f;
#pragma unroll
    for (int bl = 0; bl < CTOX_KCHUNK; bl++) {
        if ((uint32_t)bl >= nb) break;
        const uint8_t *blk = rowl + bl * F::BB;
        const float scale = half_bits_to_float(*(const uint16_t *)blk);
        const uintptr_t ca = (uintptr_t)(blk + 2 + F::QB * g);
        const uint32_t *cw = (const uint32_t *)(ca & ~(uintptr_t)3);
        const uint32_t sh = (uint32_t)(ca & 3);
        v4i bfrag;
        if (DT) {
            const uint32_t d0 = cw[0], d1 = cw[1], d2 = cw[2];
            const uint32_t w0 = __builtin_amdgcn_alignbyte(d1, d0, sh);
            const uint32_t w1 = __builtin_amdgcn_alignbyte(d2, d1, sh);
            bfrag = (v4i){(int)(w0 & 0x0f0f0f0fu), (int)(w1 & 0x0f0f0f0fu),
                          (int)((w0 >> 4) & 0x0f0f0f0fu), (int)((w1 >> 4) & 0x0f0f0f0fu)};
        } else {
            const uint32_t d0 = cw[0], d1 = cw[1];
            const uint32_t w = __builtin_amdgcn_alignbyte(d1, d0, sh);
            bfrag = (v4i){(int)(w & 0x03030303u), (int)((w >> 2) & 0x03030303u),
                          (int)((w >> 4) & 0x03030303u), (int)((w >> 6) & 0x03030303u)};
        }
#pragma unroll
        for (int tg = 0; tg < TG; tg++) {
            const v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(afrag[bl][tg], bfrag,
                                                                 (v4i){0, 0, 0, 0}, 0, 0, 0);
            const float2 xc = xcv[bl][tg];
            float f = fmaf((float)c[0], 2.0f, xc.y);
            f = fmaf((float)c[1], 512.0f, f);
            f = fmaf((float)c[2], 131072.0f, f);
            acc[tg] = fmaf(f, scale * xc.x, acc[tg]);
        }
    }

    const uint32_t row = rbase + j;
    if (a.ksplit == 1) {
#pragma unroll
        for (int tg = 0; tg < TG; tg++) {
            const uint32_t tok = tg * 4 + g;
            if (tok < a.batch && row < a.rows)
                a.output[(size_t)tok * a.out_stride + row] = epilogue(acc[tg] / F::DEN, row, a);
        }
        return;
    }

    // ---- split-K: publish partials, last workgroup of the row group combines ----
#pragma unroll
    for (int tg = 0; tg < TG; tg++) {
        const uint32_t tok = tg * 4 + g;
        if (tok < a.batch)
            a.partial[(((size_t)rg * a.ksplit + kc) * a.batch + tok) * CTOX_MV_ROWS + wave * 16 + j] =
                acc[tg];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t old = __hip_atomic_fetch_add(&a.counters[rg], 1u, __ATOMIC_ACQ_REL,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        s_last = (old == a.ksplit - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    for (uint32_t idx = threadIdx.x; idx < a.batch * CTOX_MV_ROWS; idx += blockDim.x) {
        const uint32_t tok = idx / CTOX_MV_ROWS, rr = idx % CTOX_MV_ROWS;
        const uint32_t orow = rg * CTOX_MV_ROWS + rr;
        float s = 0.0f;
        for (uint32_t c = 0; c < a.ksplit; c++)
            s += __builtin_nontemporal_load(
                &a.partial[(((size_t)rg * a.ksplit + c) * a.batch + tok) * CTOX_MV_ROWS + rr]);
        if (orow < a.rows) a.output[(size_t)tok * a.out_stride + orow] = epilogue(s / F::DEN, orow, a);
    }
    if (threadIdx.x == 0)
        __hip_atomic_store(&a.counters[rg], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

extern "C" __global__ __launch_bounds__(256) void ctox_q4_matvec_b4_gfx950(MatvecArgs a) {
    qmatvec_body<1, 1>(a);
}
extern "C" __global__ __launch_bounds__(256) void ctox_q4_matvec_b8_gfx950(MatvecArgs a) {
    qmatvec_body<1, 2>(a);
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
