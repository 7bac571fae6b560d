// Chunked (WY-form) gated-delta prefill, fp32, gfx950.
//
// The token recurrence of Q/src/reference.rs:230-297 / 377-415,
//   S_t = a_t (I - b_t k_t k_t^T) S_{t-1} + b_t k_t v_t^T,   o_t = S_t^T q_t
// (k, q L2-normalised, q also scaled by 1/sqrt(key_dim), a_t = exp(log_decay_t),
// b_t = beta_t), is evaluated chunk by chunk. Within a chunk of C tokens, with
// G_t = sum_{s<=t} log_decay_s (relative to the chunk start) and
// g_t = exp(G_t):
//   S_t = g_t S_0 + sum_{r<=t} exp(G_t - G_r) k_r d_r^T
//   d_s = b_s (v_s - g_s S_0^T k_s - sum_{r<s} exp(G_s - G_r) (k_s.k_r) d_r)
// i.e. (I + diag(b) M) D = diag(b) V - diag(b g) K S_0 with M the strictly
// lower, decay-weighted K K^T, so D = T (diag(b) V - diag(b g) K S_0),
// T = (I + diag(b) M)^{-1} (unit lower triangular). Then
//   O   = diag(g) Q S_0 + A D,       A[t][r] = exp(G_t - G_r) (q_t.k_r), r <= t
//   S_C = g_C S_0 + sum_r exp(G_C - G_r) k_r d_r^T.
// Every decay factor is exp of a non-positive difference (<= 1), so nothing
// overflows however strong the decay.
//
// Pass 1 (ctox_gdn_chunk_prep_gfx950, one workgroup per (head, chunk), all
// chunks in parallel): norms, G, M and A from the lower 16 x 16 tiles of
// K K^T and Q K^T on v_mfma_f32_16x16x4_f32, T by
// blocks: the four 16 x 16 diagonal blocks by forward substitution (a wave
// each), the blocks below them on MFMA one block row at a time.
// Pass 2 (ctox_gdn_chunk_scan_gfx950, one workgroup per (head, 16 value
// columns), chunks in order): the 128 x 16 state slice stays in LDS across
// chunks; the five small products per chunk run on v_mfma_f32_16x16x4_f32.
// Value columns are independent in the recurrence, so slices need no
// exchange. Padded tokens of a partial last chunk have k = q = v = 0,
// beta = 0 and log_decay = 0: identity steps.

#include <hip/hip_runtime.h>

#include "kernel_args.h"
#include "lds_barrier.h"

#define GC 64        // max chunk length
#define GKD 128      // max key_dim of the chunked path
#define GVS 16       // value columns per pass-2 workgroup
#define TPAD 65      // LDS row stride of T / A / M

typedef float gv4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ gv4f mfma4(float a, float b, gv4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

#define SPAD 132  // LDS row stride (floats) of pass-2 K / Q tiles and of S^T
#define TSPAD 68  // LDS row stride of pass-2 T / A / Y^T / (b v)^T

// 16 x 16 tile of A[16 x K] * B[K x 16] with both operands stored k-contiguous
// (A row-major [m][k], B as B^T [n][k]): lane (m = l % 16, kq = l / 16)
// covers k = kq * (K / 4) + u for MFMA u, so each lane reads a contiguous
// run of K / 4 floats of both operands.
template <int K, int LDA, int LDB>
__device__ __forceinline__ gv4f tile_kk(const float *a, const float *bt, gv4f acc, uint32_t lane) {
    const uint32_t m = lane & 15, kq = lane >> 4;
    const float *ap = a + m * LDA + kq * (K / 4);
    const float *bp = bt + m * LDB + kq * (K / 4);
    // Four independent accumulation chains, summed at the end.
    gv4f c1 = {0.0f, 0.0f, 0.0f, 0.0f}, c2 = c1, c3 = c1;
#pragma unroll
    for (int u = 0; u < K / 4; u += 4) {
        const float4 av = *(const float4 *)(ap + u), bv = *(const float4 *)(bp + u);
        acc = mfma4(av.x, bv.x, acc);
        c1 = mfma4(av.y, bv.y, c1);
        c2 = mfma4(av.z, bv.z, c2);
        c3 = mfma4(av.w, bv.w, c3);
    }
    return (acc + c1) + (c2 + c3);
}

// Scratch per (head, chunk): T[64][64], A[64][64], then per token g = exp(G),
// exp(G_C - G), kinv and kinv's counterpart for q times 1/sqrt(key_dim) g.
__host__ __device__ constexpr uint32_t ctox_gdn_chunk_floats() { return 2 * GC * GC + 4 * GC; }

extern "C" __global__ __launch_bounds__(256) void ctox_gdn_chunk_prep_gfx950(GdnArgs a) {
    __shared__ __align__(16) float kh[GC * SPAD];
    __shared__ __align__(16) float qh[GC * SPAD];  // q^ rows, then M (after the dot-product tiles)
    __shared__ float G[GC], bt[GC], kinv_s[GC], qinv_s[GC];
    float *mm = qh;
    const uint32_t tid = threadIdx.x;
    const uint32_t nch = (a.tokens + a.chunk - 1) / a.chunk;
    const uint32_t h = blockIdx.x / nch, c = blockIdx.x % nch;
    const uint32_t t0 = c * a.chunk;
    const uint32_t n = min(a.chunk, a.tokens - t0);
    const uint32_t dk = a.key_dim;
    const float qscale = 1.0f / sqrtf((float)dk);

    // Raw k, q rows into LDS (zeros beyond n rows and key_dim columns), four
    // threads per row accumulating the squares. The tiles below use the raw
    // rows and scale their products by the inverse norms.
    {
        const uint32_t s = tid >> 2, p = tid & 3;
        float sk = 0.0f, sq = 0.0f;
        if (s < n) {
            const size_t qk = (size_t)(t0 + s) * a.qk_stride + (size_t)(h / a.rep) * dk;
            const float *kr = a.k + qk;
            const float *qr = a.q + qk;
            for (uint32_t i = p; i < dk; i += 4) {
                const float kv = kr[i], qv = qr[i];
                kh[s * SPAD + i] = kv;
                qh[s * SPAD + i] = qv;
                sk += kv * kv;
                sq += qv * qv;
            }
        }
        for (uint32_t i = (s < n ? dk : 0) + p; i < GKD; i += 4) {
            kh[s * SPAD + i] = 0.0f;
            qh[s * SPAD + i] = 0.0f;
        }
        sk += __shfl_xor(sk, 1);
        sk += __shfl_xor(sk, 2);
        sq += __shfl_xor(sq, 1);
        sq += __shfl_xor(sq, 2);
        if (p == 0) {
            kinv_s[s] = s < n ? 1.0f / sqrtf(sk + 1e-6f) : 0.0f;
            qinv_s[s] = s < n ? 1.0f / sqrtf(sq + 1e-6f) : 0.0f;
        }
    }
    if (tid < GC) {
        const size_t th = (size_t)(t0 + tid) * a.heads + h;
        const float ld = tid < n ? a.log_decay[th] : 0.0f;
        bt[tid] = tid < n ? a.beta[th] : 0.0f;
        // inclusive prefix sum of log decay over the chunk (one wave)
        float g = ld;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float up = __shfl_up(g, o);
            if (tid >= (uint32_t)o) g += up;
        }
        G[tid] = g;
    }
    __syncthreads();
    // The lower 16 x 16 tiles of K K^T and Q K^T on MFMA: 10 tiles each,
    // (sb, rb) with rb <= sb, five per wave; the upper tiles of A are zero.
    {
        const uint32_t lane = tid & 63, w = tid >> 6, m16 = lane & 15, kq = lane >> 4;
        gv4f acc[5];
#pragma unroll
        for (int u = 0; u < 5; u++) {
            const uint32_t t = w + 4 * u, l = t % 10;
            const uint32_t sb = l >= 6 ? 3 : (l >= 3 ? 2 : (l >= 1 ? 1 : 0));
            const uint32_t rb = l - sb * (sb + 1) / 2;
            acc[u] = tile_kk<GKD, SPAD, SPAD>((t < 10 ? kh : qh) + 16 * sb * SPAD, kh + 16 * rb * SPAD,
                                              (gv4f){0, 0, 0, 0}, lane);
        }
        float *Aout = a.norms + ((size_t)h * nch + c) * ctox_gdn_chunk_floats() + GC * GC;
        __syncthreads();  // every tile has read q^: its rows become M
#pragma unroll
        for (int u = 0; u < 5; u++) {
            const uint32_t t = w + 4 * u, l = t % 10;
            const uint32_t sb = l >= 6 ? 3 : (l >= 3 ? 2 : (l >= 1 ? 1 : 0));
            const uint32_t rb = l - sb * (sb + 1) / 2;
#pragma unroll
            for (int x = 0; x < 4; x++) {
                const uint32_t s = 16 * sb + 4 * kq + x, r = 16 * rb + m16;
                const float dec = expf(G[s] - G[r]) * kinv_s[r] * (t < 10 ? kinv_s[s] : qinv_s[s] * qscale);
                if (t < 10) mm[s * TPAD + r] = r < s ? dec * acc[u][x] : 0.0f;
                else Aout[s * GC + r] = r <= s ? dec * acc[u][x] : 0.0f;
            }
        }
        for (uint32_t e = tid; e < GC * GC / 4; e += 256) {
            const uint32_t s = e / 16, r = (e % 16) * 4;
            if (r / 16 > s / 16) *(float4 *)(Aout + s * GC + r) = make_float4(0, 0, 0, 0);
        }
    }
    __syncthreads();
    float *base = a.norms + ((size_t)h * nch + c) * ctox_gdn_chunk_floats();
    // T = (I + L)^{-1}, L = diag(b) M strictly lower, blockwise over 16 x 16
    // blocks into LDS (tt, over the k rows, free after the tiles):
    //   T_ii = (I + L_ii)^{-1}                   forward substitution, wave i;
    //   T_ij = -T_ii sum_{k=j}^{i-1} L_ik T_kj   block row i after row i - 1,
    //                                            task j on wave j, on MFMA.
    float *tt = kh;
    {
        const uint32_t lane = tid & 63, w = tid >> 6, m16 = lane & 15, kq = lane >> 4;
        if (lane < 16) {
            const uint32_t cc = 16 * w + lane;
            float col[16];
#pragma unroll
            for (int s = 0; s < 16; s++) {
                const uint32_t row = 16 * w + s;
                float acc = 0.0f;
#pragma unroll
                for (int r = 0; r < s; r++) acc = fmaf(mm[row * TPAD + 16 * w + r], col[r], acc);
                col[s] = ((uint32_t)s == lane ? 1.0f : 0.0f) - bt[row] * acc;
                tt[row * TPAD + cc] = col[s];
            }
        }
#pragma unroll
        for (uint32_t bi = 1; bi < 4; bi++) {
            __syncthreads();  // block row bi - 1 (and the diagonal) written
            if (w < bi) {
                const uint32_t bj = w;
                // X = sum_k L_ik T_kj: A = L rows of block bi, B = T rows of block k.
                gv4f x = {0.0f, 0.0f, 0.0f, 0.0f};
                for (uint32_t bk = bj; bk < bi; bk++) {
                    const float b = bt[16 * bi + m16];
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const uint32_t kk = 16 * bk + 4 * u + kq;
                        x = mfma4(b * mm[(16 * bi + m16) * TPAD + kk], tt[kk * TPAD + 16 * bj + m16], x);
                    }
                }
                // T_ij = -T_ii X. Lane (kq, n) holds X rows 4 kq + u of column
                // n, so MFMA u takes k = 4 kq + u: A reads T_ii[m][4 kq + u].
                gv4f y = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int u = 0; u < 4; u++)
                    y = mfma4(tt[(16 * bi + m16) * TPAD + 16 * bi + 4 * kq + u], x[u], y);
#pragma unroll
                for (int u = 0; u < 4; u++) tt[(16 * bi + 4 * kq + u) * TPAD + 16 * bj + m16] = -y[u];
            }
        }
        __syncthreads();
        for (uint32_t e = tid; e < GC * GC / 4; e += 256) {
            const uint32_t s = e / 16, r = (e % 16) * 4;
            const bool up = r / 16 > s / 16;
            *(float4 *)(base + s * GC + r) = up ? make_float4(0, 0, 0, 0)
                                                : make_float4(tt[s * TPAD + r], tt[s * TPAD + r + 1],
                                                              tt[s * TPAD + r + 2], tt[s * TPAD + r + 3]);
        }
    }
    if (tid < GC) {
        const float g = expf(G[tid]);
        base[2 * GC * GC + tid] = g;
        base[2 * GC * GC + GC + tid] = expf(G[GC - 1] - G[tid]);
        base[2 * GC * GC + 2 * GC + tid] = kinv_s[tid];
        base[2 * GC * GC + 3 * GC + tid] = qinv_s[tid] * qscale * g;
    }
}

// A buffer resource over [p, p + bytes) whose fields the compiler keeps in
// scalar registers: p and bytes are wave-uniform but computed through vector
// registers, and a resource in vector registers costs a waterfall loop per load.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const void *p, uint32_t bytes) {
    const uint64_t v = (uint64_t)p;
    const uint64_t u = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32)) << 32) |
                       (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
    return __builtin_amdgcn_make_buffer_rsrc((void *)u, (short)0, (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

// Registers holding the next chunk while the current one computes.
struct GdnPrefetch {
    float4 k[8], q[8];   // 64 x 128 each: float4 index tid + 256 m
    float4 t[4], am[4];  // T, A: 64 x 64 each
    float4 v;            // 64 x 16 value slice: row tid / 4, part tid % 4
    float4 aux;          // g / g_C/g / kinv / q scale (threads 0..63), float4 tid % 16 of array tid / 16
    float beta;          // threads 0..63
};

// VEC: key_dim and value_dim multiples of 4 and 16, token strides multiples
// of 4 floats, q, k, v 16-byte aligned and a chunk's rows spanning under
// 2 GB; the host launches the VEC instantiation exactly then. Its loads are
// 16-byte buffer reads with no branches (the generic path's predicated reads
// make the compiler wait for every outstanding load at each branch join,
// which serialises the next chunk's prefetch).
template <bool VEC>
__device__ __forceinline__ void chunk_scan(const GdnArgs &a) {
    // k^ rows [s][i]; (g q^) rows [s][i]; T [s][r]; A [t][r]; S^T [n][i] (x2);
    // Y^T / D^T [n][s]; (b v)^T [n][s]; D [r][n] for the state update; K~^T [i][r].
    __shared__ __align__(16) float kh[GC * SPAD];
    __shared__ __align__(16) float qh[GC * SPAD];
    __shared__ __align__(16) float tm[GC * TSPAD];
    __shared__ __align__(16) float am[GC * TSPAD];
    __shared__ __align__(16) float st[2][GVS * SPAD];
    __shared__ __align__(16) float yt[GVS * TSPAD];
    __shared__ __align__(16) float vt[GVS * TSPAD];
    __shared__ float eg[GC], ec[GC], kinv[GC], qsc[GC], bt[GC];
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint32_t m16 = lane & 15, kq = lane >> 4;
    const uint32_t slices = (a.value_dim + GVS - 1) / GVS;
    // Workgroup b runs on XCD b % 8. All slices of one head are placed on the
    // same XCD so that they share the chunk's k, q, T and A in that XCD's L2:
    // XCD x takes heads x, x + 8, ..., its q-th workgroup being slice q % slices
    // of head x + 8 (q / slices). The grid is 8 * ceil(heads / 8) * slices.
    const uint32_t xcd = blockIdx.x & 7, qx = blockIdx.x >> 3;
    const uint32_t h = xcd + 8 * (qx / slices), j0 = (qx % slices) * GVS;
    if (h >= a.heads) return;
    const uint32_t nch = (a.tokens + a.chunk - 1) / a.chunk;
    const uint32_t dk = a.key_dim, dv = a.value_dim;
    const size_t rowv = (size_t)a.heads * dv;
    float *S = a.state + (size_t)h * dk * dv;
    for (uint32_t e = tid; e < GKD * GVS; e += 256) {
        const uint32_t i = e / GVS, n = e % GVS;
        st[0][n * SPAD + i] = (i < dk && j0 + n < dv) ? S[(size_t)i * dv + j0 + n] : 0.0f;
    }

    // parts: 1 = k (with q on the generic path), 2 = q, 4 = T, A, v, aux, beta.
    auto fetch = [&](GdnPrefetch &p, uint32_t c, const int parts) {
        const uint32_t t0 = c * a.chunk, n = min(a.chunk, a.tokens - t0);
        const float *base = a.norms + ((size_t)h * nch + c) * ctox_gdn_chunk_floats();
        // Branch-free loads: one buffer over the chunk's rows of this key head
        // (of this value slice); a lane past the chunk or past key_dim reads at
        // the buffer's end, which the range check returns as zero.
        const uint32_t kq_end = VEC ? ((n - 1) * a.qk_stride + dk) * 4 : 0;
        const size_t kq0 = (size_t)t0 * a.qk_stride + (size_t)(h / a.rep) * dk;
        const __amdgpu_buffer_rsrc_t rk = uniform_rsrc(a.k + kq0, kq_end);
        const __amdgpu_buffer_rsrc_t rq = uniform_rsrc(a.q + kq0, kq_end);
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const uint32_t f = tid + 256 * m, s = f >> 5, i = (f & 31) * 4;
            const bool ok = s < n && i < dk;
            if (VEC) {
                const uint32_t off = ok ? (s * a.qk_stride + i) * 4 : kq_end;
                if (parts & 1) p.k[m] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
                if (parts & 2) p.q[m] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rq, off, 0, 0));
            } else if (parts & 1) {
                const size_t off = (size_t)(t0 + (ok ? s : 0)) * a.qk_stride + (size_t)(h / a.rep) * dk + (ok ? i : 0);
                float kk4[4], qq4[4];
#pragma unroll
                for (int x = 0; x < 4; x++) {
                    const bool ox = s < n && i + x < dk;
                    kk4[x] = ox ? a.k[off + x] : 0.0f;
                    qq4[x] = ox ? a.q[off + x] : 0.0f;
                }
                p.k[m] = make_float4(kk4[0], kk4[1], kk4[2], kk4[3]);
                p.q[m] = make_float4(qq4[0], qq4[1], qq4[2], qq4[3]);
            }
        }
        if (!(parts & 4)) return;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            p.t[m] = ((const float4 *)base)[tid + 256 * m];
            p.am[m] = ((const float4 *)(base + GC * GC))[tid + 256 * m];
        }
        {
            const uint32_t s = tid >> 2, part = tid & 3;
            const bool ok = s < n;
            if (VEC) {
                const uint32_t v_end = ((n - 1) * a.v_stride + GVS) * 4;
                const __amdgpu_buffer_rsrc_t rv = uniform_rsrc(a.v + (size_t)t0 * a.v_stride + (size_t)h * dv + j0, v_end);
                p.v = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rv, ok ? (s * a.v_stride + 4 * part) * 4 : v_end, 0, 0));
            } else {
                const size_t off = (size_t)(t0 + (ok ? s : 0)) * a.v_stride + (size_t)h * dv + j0 + 4 * part;
                float v4[4];
#pragma unroll
                for (int x = 0; x < 4; x++) v4[x] = (ok && j0 + 4 * part + x < dv) ? a.v[off + x] : 0.0f;
                p.v = make_float4(v4[0], v4[1], v4[2], v4[3]);
            }
        }
        p.aux = tid < 64 ? ((const float4 *)(base + 2 * GC * GC))[tid] : make_float4(0, 0, 0, 0);
        {
            const uint32_t b_end = ((n - 1) * a.heads + 1) * 4;
            const __amdgpu_buffer_rsrc_t rb = uniform_rsrc(a.beta + (size_t)t0 * a.heads + h, b_end);
            p.beta = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, tid < n ? tid * a.heads * 4 : b_end, 0, 0));
        }
    };

    GdnPrefetch pf;
    fetch(pf, 0, 7);
    uint32_t cur = 0;
    for (uint32_t c = 0; c < nch; c++) {
        const uint32_t t0 = c * a.chunk, n = min(a.chunk, a.tokens - t0);
        lds_barrier();  // the previous chunk is done with every buffer
        if (tid < GC) {
            float *aux = tid < 16 ? eg : (tid < 32 ? ec : (tid < 48 ? kinv : qsc));
            ((float4 *)aux)[tid & 15] = pf.aux;
            bt[tid] = pf.beta;
        }
        lds_barrier();
        // Stage: k^ = k kinv; (g q^) = q qinv qscale exp(G) (one factor from
        // the prep); T; A; (b v)^T.
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const uint32_t f = tid + 256 * m, s = f >> 5, i = (f & 31) * 4;
            const float ks = kinv[s], qs = qsc[s];
            *(float4 *)(kh + s * SPAD + i) = make_float4(pf.k[m].x * ks, pf.k[m].y * ks, pf.k[m].z * ks, pf.k[m].w * ks);
            *(float4 *)(qh + s * SPAD + i) = make_float4(pf.q[m].x * qs, pf.q[m].y * qs, pf.q[m].z * qs, pf.q[m].w * qs);
        }
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const uint32_t f = tid + 256 * m, s = f >> 4, r = (f & 15) * 4;
            *(float4 *)(tm + s * TSPAD + r) = pf.t[m];
            *(float4 *)(am + s * TSPAD + r) = pf.am[m];
        }
        {
            const uint32_t s = tid >> 2, part = tid & 3;
            const float b = bt[s];
            vt[(4 * part + 0) * TSPAD + s] = pf.v.x * b;
            vt[(4 * part + 1) * TSPAD + s] = pf.v.y * b;
            vt[(4 * part + 2) * TSPAD + s] = pf.v.z * b;
            vt[(4 * part + 3) * TSPAD + s] = pf.v.w * b;
        }
        lds_barrier();
        // The next chunk's loads are issued in three groups between this
        // chunk's products, so that their address traffic overlaps MFMA work;
        // the loop's barriers order LDS only, so nothing waits for them before
        // the next chunk's staging.
        const bool more = c + 1 < nch;
        if (more) fetch(pf, c + 1, 4);
        const float *Sc = st[cur];
        // Y^T[n][s] = (b v)^T - b_s g_s (K S)[s][n]   (wave w: rows s = 16w..16w+15)
        {
            gv4f acc = tile_kk<GKD, SPAD, SPAD>(kh + 16 * w * SPAD, Sc, (gv4f){0, 0, 0, 0}, lane);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t s = 16 * w + 4 * kq + r;
                yt[m16 * TSPAD + s] = vt[m16 * TSPAD + s] - bt[s] * eg[s] * acc[r];
            }
        }
        if (more) fetch(pf, c + 1, 1);
        lds_barrier();
        // D = T Y  (T rows [s][r] and Y^T [n][r] are both r-contiguous)
        gv4f dacc = tile_kk<GC, TSPAD, TSPAD>(tm + 16 * w * TSPAD, yt, (gv4f){0, 0, 0, 0}, lane);
        lds_barrier();
        // D^T [n][s] into yt, and (D^T scaled by g_C / g_s) into vt, whose
        // (b v)^T the Y step has consumed: the state update's left operand.
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t s = 16 * w + 4 * kq + r;
            yt[m16 * TSPAD + s] = dacc[r];
            vt[m16 * TSPAD + s] = dacc[r] * ec[s];
        }
        lds_barrier();
        if (more) fetch(pf, c + 1, 2);
        // O = (g Q) S + A D
        {
            gv4f acc = tile_kk<GKD, SPAD, SPAD>(qh + 16 * w * SPAD, Sc, (gv4f){0, 0, 0, 0}, lane);
            acc = tile_kk<GC, TSPAD, TSPAD>(am + 16 * w * TSPAD, yt, acc, lane);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t s = 16 * w + 4 * kq + r, j = j0 + m16;
                if (s < n && j < dv) a.out[(size_t)(t0 + s) * rowv + (size_t)h * dv + j] = acc[r];
            }
        }
        // S'^T[n][i] = g_C S^T[n][i] + sum_r D^T[n][r] exp(G_C - G_r) k^[r][i]
        //   as a 16 x 16 tile per (n, i-block): A = the scaled D^T [n][r]
        //   (r-contiguous), B = k^[r][i] read column-wise.
        {
            const float decC = eg[GC - 1];
            float *Sn = st[cur ^ 1];
#pragma unroll
            for (int half = 0; half < 2; half++) {
                const uint32_t i0 = 32 * w + 16 * half;
                gv4f acc;
#pragma unroll
                for (int r = 0; r < 4; r++) acc[r] = decC * Sc[(4 * kq + r) * SPAD + i0 + m16];
                const float *ap = vt + m16 * TSPAD + kq * (GC / 4);
                gv4f c1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int u = 0; u < GC / 4; u += 2) {
                    const uint32_t rr = kq * (GC / 4) + u;
                    acc = mfma4(ap[u], kh[rr * SPAD + i0 + m16], acc);
                    c1 = mfma4(ap[u + 1], kh[(rr + 1) * SPAD + i0 + m16], c1);
                }
                acc += c1;
                // acc rows = n (4 kq + r), columns = i0 + m16
#pragma unroll
                for (int r = 0; r < 4; r++) Sn[(4 * kq + r) * SPAD + i0 + m16] = acc[r];
            }
        }
        cur ^= 1;
    }
    __syncthreads();
    for (uint32_t e = tid; e < GKD * GVS; e += 256) {
        const uint32_t i = e / GVS, n = e % GVS;
        if (i < dk && j0 + n < dv) S[(size_t)i * dv + j0 + n] = st[cur][n * SPAD + i];
    }
}

extern "C" __global__ __launch_bounds__(256) void ctox_gdn_chunk_scan_gfx950(GdnArgs a) { chunk_scan<false>(a); }
extern "C" __global__ __launch_bounds__(256) void ctox_gdn_chunk_scan_vec_gfx950(GdnArgs a) { chunk_scan<true>(a); }
