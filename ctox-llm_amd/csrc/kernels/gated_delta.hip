// Gated-delta (GatedDeltaNet) recurrence with an fp32 state, gfx950.
//
// Per token and value head h (Q/src/reference.rs:230-297):
//   q^ = q / sqrt(|q|^2 + 1e-6), k^ likewise
//   S' = exp(log_decay) * S
//   mem_j = sum_i S'[i,j] k^_i ; delta_j = (v_j - mem_j) * beta
//   S''[i,j] = S'[i,j] + k^_i delta_j
//   o_j = sum_i S''[i,j] q^_i / sqrt(key_dim)
// State layout [head][key i][value j], row-major, updated in place.
//
// Work split: value columns are independent given q^ and k^, so a workgroup
// owns one head and a 16-column slice of its state (8 workgroups per head for
// value_dim 128: 256 workgroups at 32 heads fill the chip). Thread (ig, jj)
// keeps rows i = ig + 16r of column jj in registers, so one token reads and
// writes each state element exactly once; the token-serial scan keeps the
// slice register-resident across all tokens. Column reductions over i go
// through LDS. The workgroup barriers order LDS only (lds_barrier): a
// __syncthreads would also wait for every global store issued before it
// (the gate and output stores), which costs a memory round trip per barrier.
#include <hip/hip_runtime.h>

#include "kernel_args.h"
#include "lds_barrier.h"

#define GDN_COLS 16
#define GDN_GROUPS 16
#define GDN_MAX_ROWS 16  // key_dim <= 256

// Sum over the four 16-lane rows of a wave (lane swaps, no LDS trip).
__device__ __forceinline__ float gdn_sum_rows(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v), false,
                                              false);
    v = __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
    r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v), false, false);
    return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}

// Token-serial scan over a.tokens tokens (tokens = 1 is the decode step).
// grid = heads * ceil(value_dim / 16), block = 256. One reduction over the
// key rows per token: with the decayed state S' the thread sums over its rows
// k . S', q . S' (per column), |k|^2, |q|^2 and k . q; the four 16-lane row
// groups of a wave add by lane swaps and the four waves through LDS (double
// buffered by token parity, so one barrier per token). Then per column
// mem_j = (k . S'_j) k_inv, delta_j = (v_j - mem_j) beta, and the output
// follows without a second reduction: q . S''_j = q . S'_j + (k . q) k_inv delta_j,
// o_j = that * q_inv / sqrt(key_dim).
extern "C" __global__ __launch_bounds__(256) void ctox_gdn_scan_gfx950(GdnArgs a) {
    __shared__ __align__(16) float red[2][5][GDN_COLS][4];  // [token parity][sum][column][wave]

    const uint32_t slices = (a.value_dim + GDN_COLS - 1) / GDN_COLS;
    const uint32_t h = blockIdx.x / slices, slice = blockIdx.x % slices;
    const uint32_t jj = threadIdx.x % GDN_COLS, ig = threadIdx.x / GDN_COLS, wave = threadIdx.x >> 6;
    const uint32_t j = slice * GDN_COLS + jj;
    const bool colok = j < a.value_dim;
    const uint32_t nrows = (a.key_dim + GDN_GROUPS - 1) / GDN_GROUPS;
    const float qscale = 1.0f / sqrtf((float)a.key_dim);

    float *S = a.state + (size_t)h * a.key_dim * a.value_dim;
    float s[GDN_MAX_ROWS];
#pragma unroll
    for (int r = 0; r < GDN_MAX_ROWS; r++) {
        const uint32_t i = ig + GDN_GROUPS * r;
        s[r] = ((uint32_t)r < nrows && i < a.key_dim && colok) ? S[(size_t)i * a.value_dim + j] : 0.0f;
    }

    for (uint32_t t = 0; t < a.tokens; t++) {
        const size_t th = (size_t)t * a.heads + h;
        const size_t qk = (size_t)t * a.qk_stride + (size_t)(h / a.rep) * a.key_dim;
        const float *q = a.q + qk;
        const float *k = a.k + qk;
        const float decay = expf(a.log_decay[th]);
        const float beta = a.beta[th];
        const float vj = colok ? a.v[(size_t)t * a.v_stride + (size_t)h * a.value_dim + j] : 0.0f;

        float kk[GDN_MAX_ROWS];
        float v5[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};  // k . S', q . S', |k|^2, |q|^2, k . q
#pragma unroll
        for (int r = 0; r < GDN_MAX_ROWS; r++) {
            const uint32_t i = ig + GDN_GROUPS * r;
            const bool ok = (uint32_t)r < nrows && i < a.key_dim;
            kk[r] = ok ? k[i] : 0.0f;
            const float qq = ok ? q[i] : 0.0f;
            s[r] = s[r] * decay;
            v5[0] += s[r] * kk[r];
            v5[1] += s[r] * qq;
            v5[2] += kk[r] * kk[r];
            v5[3] += qq * qq;
            v5[4] += kk[r] * qq;
        }
#pragma unroll
        for (int c = 0; c < 5; c++) v5[c] = gdn_sum_rows(v5[c]);
        float(*rb)[GDN_COLS][4] = red[t & 1];
        if ((threadIdx.x & 63) < GDN_COLS)
#pragma unroll
            for (int c = 0; c < 5; c++) rb[c][jj][wave] = v5[c];
        lds_barrier();
#pragma unroll
        for (int c = 0; c < 5; c++) {
            const float4 w = *(const float4 *)rb[c][jj];
            v5[c] = (w.x + w.y) + (w.z + w.w);
        }
        const float kinv = 1.0f / sqrtf(v5[2] + 1e-6f), qinv = 1.0f / sqrtf(v5[3] + 1e-6f);
        const float delta = (vj - v5[0] * kinv) * beta;
#pragma unroll
        for (int r = 0; r < GDN_MAX_ROWS; r++) s[r] += kk[r] * kinv * delta;
        if (ig == 0 && colok) a.out[th * a.value_dim + j] = (v5[1] + v5[4] * kinv * delta) * qinv * qscale;
        // The next token writes the other parity's buffer; the one after it
        // this one again, past the next token's barrier, which every thread
        // reaches only after reading this token's sums.
    }

#pragma unroll
    for (int r = 0; r < GDN_MAX_ROWS; r++) {
        const uint32_t i = ig + GDN_GROUPS * r;
        if ((uint32_t)r < nrows && i < a.key_dim && colok) S[(size_t)i * a.value_dim + j] = s[r];
    }
}

// Fused token mixer core (GdnFusedArgs): one workgroup per (head, 16-column
// slice), 256 threads, tokens in order. Per token, threads 0 .. 2 dk - 1 run
// the causal conv + SiLU (Q/src/reference.rs:159-187) of the head's q and k
// channels (key head h / rep, Q/src/decoder.rs:868-880) and threads 0..15 the
// slice's v channels, each keeping its channel's window in registers; the
// gates (Q/src/decoder.rs:29-35, 881-902) are computed by one thread (or read
// when given); then the recurrence step of ctox_gdn_scan_gfx950 on those
// values from LDS. The conv windows are read from conv_in and the final ones
// written to conv_out: a key head's q/k windows by its first value head's
// slice-0 workgroup, v windows by the workgroup that owns the columns. The
// conv arithmetic is that of ctox_conv_update_gfx950, the gates that of
// ctox_gdn_gates_gfx950 (same operation order).
#define GDN_MAX_KERNEL 8
#define GDN_PREFETCH 8  // token rows whose inputs are loaded up front
// A buffer for branch-free loads: a lane without an element reads at `end`
// (the buffer's byte size), which the range check turns into a zero without
// a memory access. The address stays inside the allocation's pages (an
// offset far past the buffer made every such read pay a translation miss).
struct GdnBuf {
    __amdgpu_buffer_rsrc_t r;
    uint32_t end;
};
__device__ __forceinline__ GdnBuf gdn_buf(const float *p, size_t floats) {
    const uint32_t bytes = p ? (uint32_t)min(floats * 4, (size_t)0x7ffffff0) : 0u;
    return GdnBuf{__builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, (int)bytes, 0x00020000), bytes};
}
__device__ __forceinline__ float gdn_ld(const GdnBuf &b, bool ok, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(b.r, ok ? off : b.end, 0, 0));
}
// The k (<= 8) floats at byte offset off (ok) as two 16-byte reads. Entries
// past k hold the next channel's values: the conv step never reads them.
__device__ __forceinline__ void gdn_load8(const GdnBuf &b, bool ok, uint32_t off, uint32_t k, float v[GDN_MAX_KERNEL]) {
    const v4i lo = __builtin_amdgcn_raw_buffer_load_b128(b.r, ok ? off : b.end, 0, 0);
    const v4i hi = __builtin_amdgcn_raw_buffer_load_b128(b.r, ok && k > 4 ? off + 16 : b.end, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[i] = __int_as_float(lo[i]);
        v[4 + i] = __int_as_float(hi[i]);
    }
}
// Values reduced over the key rows once per block of rows (phase 2a/2b of
// gdn_fused): A_u = S0[:, j] . k_u and B_u = S0[:, j] . q_u per row u and
// column, then per row u the Gram sums k_w . k_u (w <= u, with |k_u|^2 last),
// k_w . q_u (w <= u) and |q_u|^2: row u's 2u + 3 sums start at pair u^2 + 2u,
// so the rows of a block of nb rows use the first nb^2 + 2nb pairs.
#define GDN_NA (GDN_PREFETCH * GDN_COLS)
#define GDN_V_B GDN_NA
#define GDN_V_P (2 * GDN_NA)
#define GDN_NPAIRS (GDN_PREFETCH * GDN_PREFETCH + 2 * GDN_PREFETCH)
#define GDN_NV (GDN_V_P + GDN_NPAIRS)
#define GDN_KK(w, u) (GDN_V_P + (u) * (u) + 2 * (u) + (w))
#define GDN_KQ(w, u) (GDN_V_P + (u) * (u) + 3 * (u) + 1 + (w))
#define GDN_QQ(u) (GDN_V_P + (u) * (u) + 4 * (u) + 2)

// ONE: a single row (the batch-1 decode step; its one snapshot is the final
// state). Its key-row reductions (k . S, q . S, |k|^2, k . q, |q|^2 per
// column) finish with lane swaps inside each wave and one LDS pass over the
// four waves: two workgroup barriers in all instead of the row block's three
// and its Gram pass (same arithmetic otherwise; the sums associate
// differently).
// KC: the conv kernel size as a constant (0: a.kernel at run time); with it
// the window shifts, taps and window stores are straight-line code (a row's
// conv is otherwise mostly the selects of a runtime-length window).
template <bool BLOCKED, bool ONE = false, int KC = 0>
__device__ __forceinline__ void gdn_fused(const GdnFusedArgs &a) {
    constexpr int PF = ONE ? 1 : GDN_PREFETCH;  // rows whose inputs are loaded up front
    // Rows are processed in blocks of up to GDN_PREFETCH. Phase 1 of a block
    // runs every row's conv + SiLU and gates (they do not depend on the
    // state) into LDS. Phase 2 needs one reduction over the key rows for the
    // whole block: with S0 the state at the block's start, a row's k . S and
    // q . S follow from S0 . k_u, S0 . q_u and the Gram sums of the block's
    // k and q (the state after row u is P_u S0 + sum_{u' <= u} c_{u'u} k^_u' d_u'^T,
    // P and c products of the decays), so each column then runs its rows'
    // recurrence on scalars and updates its state elements row by row.
    // Rows padded by one float: lanes reading or writing different rows at
    // one column hit different banks.
    __shared__ float red[GDN_NV][GDN_GROUPS + 1];
    __shared__ float tot[GDN_NV];
    __shared__ float qks[2][GDN_PREFETCH][257];  // conv outputs: [0] q, [1] k (padded rows)
    __shared__ float vs[GDN_PREFETCH][GDN_COLS], gsc[GDN_PREFETCH][2];
    __shared__ __align__(16) float red1[5][GDN_COLS][4];  // ONE: [sum][column][wave]

    const uint32_t slices = (a.value_dim + GDN_COLS - 1) / GDN_COLS;
    const uint32_t h = blockIdx.x / slices, slice = blockIdx.x % slices;
    const uint32_t tid = threadIdx.x, jj = tid % GDN_COLS, ig = tid / GDN_COLS;
    const uint32_t j = slice * GDN_COLS + jj;
    const bool colok = j < a.value_dim;
    const uint32_t dk = a.key_dim, rep = a.heads / a.key_heads, kh = h / rep;
    const uint32_t kw = a.key_heads * dk, K = KC ? (uint32_t)KC : a.kernel;
    const uint32_t nrows = (dk + GDN_GROUPS - 1) / GDN_GROUPS;
    const float qscale = 1.0f / sqrtf((float)dk);

    // Conv channels of this thread: one q/k channel (tid < 2 dk) and, for
    // tid < 16, the slice's v channel.
    const bool qk_thr = tid < 2 * dk;
    const uint32_t qk_ch = tid < dk ? kh * dk + tid : kw + kh * dk + (tid - dk);
    const uint32_t vj = slice * GDN_COLS + tid;
    const bool v_thr = tid < GDN_COLS && vj < a.value_dim;
    const uint32_t v_ch = 2 * kw + h * a.value_dim + vj;
    // Every input read of the workgroup is a buffer load issued before the
    // first wait, with no branch around it: a thread without a channel reads
    // past the buffer's range (zeros, no memory traffic). Loads issued inside
    // divergent branches made the compiler wait for earlier loads before
    // reusing their registers, which serialized the round trips.
    const uint32_t C = 2 * kw + a.heads * a.value_dim;  // conv channels
    const GdnBuf wr = gdn_buf(a.conv_w, (size_t)C * K), cr = gdn_buf(a.conv_in, (size_t)C * K);
    const uint32_t qko = qk_ch * K * 4, vo = v_ch * K * 4;
    float wq[GDN_MAX_KERNEL], sq_[GDN_MAX_KERNEL], wv[GDN_MAX_KERNEL], sv_[GDN_MAX_KERNEL];
    gdn_load8(wr, qk_thr, qko, K, wq);
    gdn_load8(cr, qk_thr, qko, K, sq_);
    gdn_load8(wr, v_thr, vo, K, wv);
    gdn_load8(cr, v_thr, vo, K, sv_);

    float s[GDN_MAX_ROWS];
    // Blocked layout: this thread's 8 rows at one 32-byte run.
    const size_t blk = (((size_t)h * slices + slice) * 256 + tid) * 8;
    const size_t head_floats = BLOCKED ? (size_t)slices * 2048 : (size_t)dk * a.value_dim;
    {
        const GdnBuf sr = gdn_buf(a.state + (size_t)h * head_floats, head_floats);
        if (BLOCKED) {
            const uint32_t bo = (uint32_t)(blk - (size_t)h * head_floats) * 4;
            const v4i lo = __builtin_amdgcn_raw_buffer_load_b128(sr.r, bo, 0, 0);
            const v4i hi = __builtin_amdgcn_raw_buffer_load_b128(sr.r, bo + 16, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                s[r] = __int_as_float(lo[r]);
                s[4 + r] = __int_as_float(hi[r]);
            }
#pragma unroll
            for (int r = 8; r < GDN_MAX_ROWS; r++) s[r] = 0.0f;
        } else {
#pragma unroll
            for (int r = 0; r < GDN_MAX_ROWS; r++) {
                const uint32_t i = ig + GDN_GROUPS * r;
                s[r] = gdn_ld(sr, (uint32_t)r < nrows && i < dk && colok, (i * a.value_dim + j) * 4);
            }
        }
    }
    auto store_state = [&](float *base) {
        if (BLOCKED) {
            float4 *S4 = (float4 *)(base + blk);
            S4[0] = make_float4(s[0], s[1], s[2], s[3]);
            S4[1] = make_float4(s[4], s[5], s[6], s[7]);
            return;
        }
        float *So = base + (size_t)h * head_floats;
#pragma unroll
        for (int r = 0; r < GDN_MAX_ROWS; r++) {
            const uint32_t i = ig + GDN_GROUPS * r;
            if ((uint32_t)r < nrows && i < dk && colok) So[(size_t)i * a.value_dim + j] = s[r];
        }
    };

    // The gate inputs of block row u are read by thread 256 - GDN_PREFETCH + u.
    const GdnBuf pr = gdn_buf(a.proj, (size_t)a.tokens * a.proj_stride);
    const GdnBuf dr = gdn_buf(a.gates_given ? a.log_decay : nullptr, (size_t)a.tokens * a.heads);
    const GdnBuf br = gdn_buf(a.gates_given ? a.beta : nullptr, (size_t)a.tokens * a.heads);
    const uint32_t gu = tid - (256 - PF);  // block row of this thread's gates (< PF)
    const bool g_thr = tid >= 256 - PF;
    // One conv step (shift the window left, append x) and its SiLU output.
    auto conv_step = [&](float (&win)[GDN_MAX_KERNEL], const float (&w)[GDN_MAX_KERNEL], float x) {
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i + 1 < GDN_MAX_KERNEL; i++)
            if ((uint32_t)i + 1 < K) {
                const float v = win[i + 1];
                win[i] = v;
                sum += v * w[i];
            }
        float wl = 0.0f;
#pragma unroll
        for (int i = 0; i < GDN_MAX_KERNEL; i++)
            if ((uint32_t)i == K - 1) {
                win[i] = x;
                wl = w[i];
            }
        sum += x * wl;
        return sum / (1.0f + expf(-sum));
    };
    // Inputs of one block of rows: the conv channels' values and, for thread
    // 256 - GDN_PREFETCH + u, row u's gate inputs. The first block's are read
    // here, ahead of any use of the conv windows and state loaded above, so
    // every input read of the launch is in flight before the first wait;
    // later blocks' during the previous block's recurrence.
    float xq[PF], xv[PF], ga = 0.0f, gb = 0.0f;
    auto load_block = [&](uint32_t t0) {
        const uint32_t nb = min((uint32_t)PF, a.tokens - t0);
#pragma unroll
        for (int u = 0; u < PF; u++) {
            const uint32_t row = (t0 + min((uint32_t)u, nb - 1)) * a.proj_stride;
            xq[u] = gdn_ld(pr, qk_thr, (row + qk_ch) * 4);
            xv[u] = gdn_ld(pr, v_thr, (row + v_ch) * 4);
        }
        const bool g_row = g_thr && gu < nb;
        const uint32_t gt = t0 + (g_row ? gu : 0), gth = gt * a.heads + h, grow = gt * a.proj_stride;
        if (a.gates_given) {
            ga = gdn_ld(dr, g_row, gth * 4);
            gb = gdn_ld(br, g_row, gth * 4);
        } else {
            ga = gdn_ld(pr, g_row, (grow + a.a_off + h) * 4);
            gb = gdn_ld(pr, g_row, (grow + a.b_off + h) * 4);
        }
    };
    load_block(0);
    const GdnBuf gbuf_dt = gdn_buf(a.dt_bias, a.heads), gbuf_al = gdn_buf(a.a_log, a.heads);
    const float dtb = gdn_ld(gbuf_dt, g_thr && !a.gates_given, h * 4);
    const float alog = gdn_ld(gbuf_al, g_thr && !a.gates_given, h * 4);
    __builtin_amdgcn_sched_barrier(0);
    for (uint32_t t0 = 0; t0 < a.tokens; t0 += PF) {
        const uint32_t nb = min((uint32_t)PF, a.tokens - t0);
        const bool g_row = g_thr && gu < nb;
        const uint32_t gth = (t0 + (g_row ? gu : 0)) * a.heads + h;
        // Phase 1: conv + SiLU of every block row in order (the windows after
        // row t go to the row's conv snapshot), and the gates of row gu.
#pragma unroll
        for (int u = 0; u < PF; u++) {
            if ((uint32_t)u >= nb) break;
            if (qk_thr) {
                const float y = conv_step(sq_, wq, xq[u]);
                qks[tid < dk ? 0 : 1][u][tid < dk ? tid : tid - dk] = y;
            } else if (dk < 128) {
                // Rows dk..127 of both planes read as zeros in phase 2.
                const uint32_t z = tid - 2 * dk, zw = 128 - dk;
                qks[z / zw][u][dk + z % zw] = 0.0f;
            }
            if (v_thr) vs[u][tid] = conv_step(sv_, wv, xv[u]);
            if (a.snap_stride) {
                float *co = a.conv_out + (size_t)(t0 + u) * a.conv_snap_stride;
                if (qk_thr && h % rep == 0 && slice == 0)
#pragma unroll
                    for (int i = 0; i < GDN_MAX_KERNEL; i++)
                        if ((uint32_t)i < K) co[(size_t)qk_ch * K + i] = sq_[i];
                if (v_thr)
#pragma unroll
                    for (int i = 0; i < GDN_MAX_KERNEL; i++)
                        if ((uint32_t)i < K) co[(size_t)v_ch * K + i] = sv_[i];
            }
        }
        if (g_row) {
            float be, ld;
            if (a.gates_given) {
                be = gb;
                ld = ga;
            } else {
                be = 1.0f / (1.0f + expf(-gb));
                const float x = ga + dtb;
                const float sp = x > 20.0f ? x : log1pf(expf(x));
                ld = -expf(alog) * sp;
                if (slice == 0) {
                    a.beta[gth] = be;
                    a.log_decay[gth] = ld;
                }
            }
            gsc[gu][0] = expf(ld);
            gsc[gu][1] = be;
        }
        if (t0 + PF < a.tokens) load_block(t0 + PF);
        lds_barrier();
        if constexpr (ONE) {
            float v5[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};  // k . S, q . S, |k|^2, k . q, |q|^2
            float k1[8];  // this thread's k values, kept for the state update
#pragma unroll
            for (int r = 0; r < 8; r++) {
                const uint32_t i = ig + GDN_GROUPS * r;
                const float kv = qks[1][0][i], qv = qks[0][0][i];
                k1[r] = kv;
                v5[0] += s[r] * kv;
                v5[1] += s[r] * qv;
                v5[2] += kv * kv;
                v5[3] += kv * qv;
                v5[4] += qv * qv;
            }
#pragma unroll
            for (int k = 0; k < 5; k++) v5[k] = gdn_sum_rows(v5[k]);
            if ((tid & 63) < GDN_COLS)
#pragma unroll
                for (int k = 0; k < 5; k++) red1[k][jj][tid >> 6] = v5[k];
            lds_barrier();
#pragma unroll
            for (int k = 0; k < 5; k++) {
                const float4 w = *(const float4 *)red1[k][jj];
                v5[k] = (w.x + w.y) + (w.z + w.w);
            }
            const float decay = gsc[0][0], beta = gsc[0][1];
            const float vjv = colok ? vs[0][jj] : 0.0f;
            const float kinv = 1.0f / sqrtf(v5[2] + 1e-6f);
            const float qinv = 1.0f / sqrtf(v5[4] + 1e-6f);
            const float mem = decay * v5[0];
            const float delta = (vjv - mem * kinv) * beta;
            const float o = decay * v5[1] + (v5[3] * kinv) * delta;
            if (ig == 0 && colok) a.out[(size_t)h * a.value_dim + j] = o * qinv * qscale;
#pragma unroll
            for (int r = 0; r < 8; r++) {
                s[r] = s[r] * decay;
                s[r] += k1[r] * kinv * delta;
            }
            if (a.snap_stride) store_state(a.state_out);  // the snapshot of row 0 (conv windows: phase 1)
            continue;
        }
        // Phase 2a: this thread's partial sums over its key rows i = ig + 16 r
        // (key_dim <= 128: 8 rows; phase 1 zeroed the rows past key_dim).
        // No branch around the LDS reads, so they go out back to back.
        // This thread's k values of every block row stay in registers for
        // the state updates of phase 2c.
        float kr[GDN_PREFETCH][8];
#pragma unroll
        for (int u = 0; u < GDN_PREFETCH; u++) {
            if ((uint32_t)u >= nb) break;
            float pa = 0.0f, pb = 0.0f;
#pragma unroll
            for (int r = 0; r < 8; r++) {
                const uint32_t i = ig + GDN_GROUPS * r;
                kr[u][r] = qks[1][u][i];
                pa += s[r] * kr[u][r];
                pb += s[r] * qks[0][u][i];
            }
            red[u * GDN_COLS + jj][ig] = pa;
            red[GDN_V_B + u * GDN_COLS + jj][ig] = pb;
        }
        // Gram pairs of the block's rows: column thread jj takes pairs jj,
        // jj + 16, ...
        const uint32_t npairs = nb * nb + 2 * nb;
        for (uint32_t p0 = 0; p0 < npairs; p0 += GDN_COLS) {
            const uint32_t p = min(p0 + jj, npairs - 1);
            const uint32_t u = (uint32_t)sqrtf((float)(p + 1)) - 1u;  // (u + 1)^2 <= p + 1
            const uint32_t q = p - (u * u + 2 * u);
            // q <= u: k_q . k_u; q <= 2u + 1: k_(q-u-1) . q_u; else q_u . q_u
            const uint32_t w = q <= u ? q : (q <= 2 * u + 1 ? q - u - 1 : u);
            const uint32_t s0 = q <= 2 * u + 1 ? 1u : 0u, s1 = q <= u ? 1u : 0u;  // qks planes
            float g = 0.0f;
#pragma unroll
            for (int r = 0; r < 8; r++) {
                const uint32_t i = ig + GDN_GROUPS * r;
                g += qks[s0][w][i] * qks[s1][u][i];
            }
            if (p0 + jj < npairs) red[GDN_V_P + p][ig] = g;
        }
        lds_barrier();
        // Phase 2b: totals over the 16 key-row groups, in group order.
        for (uint32_t v = tid; v < GDN_NV; v += 256) {
            const bool need = v < GDN_V_B ? v < nb * GDN_COLS : (v < GDN_V_P ? v - GDN_V_B < nb * GDN_COLS : v - GDN_V_P < nb * nb + 2 * nb);
            if (!need) continue;
            float sum = 0.0f;
#pragma unroll
            for (int gi = 0; gi < GDN_GROUPS; gi++) sum += red[v][gi];
            tot[v] = sum;
        }
        lds_barrier();
        // Phase 2c: each column's rows on scalars, then its state elements.
        float P = 1.0f, coef[GDN_PREFETCH], dlt[GDN_PREFETCH], kin[GDN_PREFETCH];
#pragma unroll
        for (int u = 0; u < GDN_PREFETCH; u++) {
            if ((uint32_t)u >= nb) break;
            const uint32_t t = t0 + u;
            const float decay = gsc[u][0], beta = gsc[u][1];
            const float vjv = colok ? vs[u][jj] : 0.0f;
            const float kinv = 1.0f / sqrtf(tot[GDN_KK(u, u)] + 1e-6f);
            const float qinv = 1.0f / sqrtf(tot[GDN_QQ(u)] + 1e-6f);
            P *= decay;
#pragma unroll
            for (int w = 0; w < u; w++) coef[w] *= decay;
            // k_u . (decayed state after row u - 1)
            float mem = P * tot[u * GDN_COLS + jj];
#pragma unroll
            for (int w = 0; w < u; w++) mem += coef[w] * (tot[GDN_KK(w, u)] * kin[w]) * dlt[w];
            const float delta = (vjv - mem * kinv) * beta;
            coef[u] = 1.0f;
            dlt[u] = delta;
            kin[u] = kinv;
            // q_u . (state after row u)
            float o = P * tot[GDN_V_B + u * GDN_COLS + jj];
#pragma unroll
            for (int w = 0; w <= u; w++) o += coef[w] * (tot[GDN_KQ(w, u)] * kin[w]) * dlt[w];
            if (ig == 0 && colok) a.out[((size_t)t * a.heads + h) * a.value_dim + j] = o * qinv * qscale;
#pragma unroll
            for (int r = 0; r < 8; r++) {
                s[r] = s[r] * decay;
                s[r] += kr[u][r] * kinv * delta;
            }
            // Row snapshot: the state after row t.
            if (a.snap_stride) store_state(a.state_out + (size_t)t * a.snap_stride);
        }
        // The next block's phase 1 rewrites the row buffers read above.
        if (t0 + GDN_PREFETCH < a.tokens) lds_barrier();
    }
    if (a.snap_stride) return;

    store_state(a.state_out);
    // Final conv windows, each written once.
    if (qk_thr && h % rep == 0 && slice == 0)
#pragma unroll
        for (int i = 0; i < GDN_MAX_KERNEL; i++)
            if ((uint32_t)i < K) a.conv_out[(size_t)qk_ch * K + i] = sq_[i];
    if (v_thr)
#pragma unroll
        for (int i = 0; i < GDN_MAX_KERNEL; i++)
            if ((uint32_t)i < K) a.conv_out[(size_t)v_ch * K + i] = sv_[i];
}

// The crate's state layout, and the engine's blocked one (state_blocked);
// fused1: one row (the batch-1 decode step); _k4: conv kernel size 4 (the
// model's), the others take any size up to GDN_MAX_KERNEL.
#define CTOX_GDN_FUSED(name, blocked, one, kc) \
    extern "C" __global__ __launch_bounds__(256) void name(GdnFusedArgs a) { gdn_fused<blocked, one, kc>(a); }
CTOX_GDN_FUSED(ctox_gdn_fused_gfx950, false, false, 0)
CTOX_GDN_FUSED(ctox_gdn_fused_blk_gfx950, true, false, 0)
CTOX_GDN_FUSED(ctox_gdn_fused1_gfx950, false, true, 0)
CTOX_GDN_FUSED(ctox_gdn_fused1_blk_gfx950, true, true, 0)
CTOX_GDN_FUSED(ctox_gdn_fused_k4_gfx950, false, false, 4)
CTOX_GDN_FUSED(ctox_gdn_fused_blk_k4_gfx950, true, false, 4)
CTOX_GDN_FUSED(ctox_gdn_fused1_k4_gfx950, false, true, 4)
CTOX_GDN_FUSED(ctox_gdn_fused1_blk_k4_gfx950, true, true, 4)
