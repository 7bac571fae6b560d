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

// Token-serial scan over a.tokens tokens (tokens = 1 is the decode step).
// grid = heads * ceil(value_dim / 16), block = 256. The inverse norms of q and
// k are reduced in the same pass as k.S (no separate norms launch):
// mem_j = (sum_i S'[i,j] k_i) * k_inv and o_j = (sum_i S''[i,j] q_i) * q_inv / sqrt(key_dim).
extern "C" __global__ __launch_bounds__(256) void ctox_gdn_scan_gfx950(GdnArgs a) {
    __shared__ float red_mem[GDN_GROUPS][GDN_COLS];
    __shared__ float red_out[GDN_GROUPS][GDN_COLS];
    __shared__ float red_nrm[2][GDN_GROUPS];

    const uint32_t slices = (a.value_dim + GDN_COLS - 1) / GDN_COLS;
    const uint32_t h = blockIdx.x / slices, slice = blockIdx.x % slices;
    const uint32_t jj = threadIdx.x % GDN_COLS, ig = threadIdx.x / GDN_COLS;
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

        float kk[GDN_MAX_ROWS], qq[GDN_MAX_ROWS];
        float mem = 0.0f, sk = 0.0f, sq = 0.0f;
#pragma unroll
        for (int r = 0; r < GDN_MAX_ROWS; r++) {
            const uint32_t i = ig + GDN_GROUPS * r;
            const bool ok = (uint32_t)r < nrows && i < a.key_dim;
            kk[r] = ok ? k[i] : 0.0f;
            qq[r] = ok ? q[i] : 0.0f;
            sk += kk[r] * kk[r];
            sq += qq[r] * qq[r];
            s[r] = s[r] * decay;
            mem += s[r] * kk[r];
        }
        red_mem[ig][jj] = mem;
        if (jj == 0) {
            red_nrm[0][ig] = sk;
            red_nrm[1][ig] = sq;
        }
        lds_barrier();
        float memj = 0.0f, ssk = 0.0f, ssq = 0.0f;
#pragma unroll
        for (int gi = 0; gi < GDN_GROUPS; gi++) {
            memj += red_mem[gi][jj];
            ssk += red_nrm[0][gi];
            ssq += red_nrm[1][gi];
        }
        const float kinv = 1.0f / sqrtf(ssk + 1e-6f), qinv = 1.0f / sqrtf(ssq + 1e-6f);
        const float delta = (vj - memj * kinv) * beta;
        float o = 0.0f;
#pragma unroll
        for (int r = 0; r < GDN_MAX_ROWS; r++) {
            s[r] += kk[r] * kinv * delta;
            o += s[r] * qq[r];
        }
        red_out[ig][jj] = o;
        lds_barrier();
        if (ig == 0 && colok) {
            float oj = 0.0f;
#pragma unroll
            for (int gi = 0; gi < GDN_GROUPS; gi++) oj += red_out[gi][jj];
            a.out[th * a.value_dim + j] = oj * qinv * qscale;
        }
        // red_* are rewritten next token only after every thread has passed
        // the second barrier of this token and read red_mem / red_nrm; the
        // reads of red_out happen before the next token's first barrier.
        lds_barrier();
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
template <bool BLOCKED>
__device__ __forceinline__ void gdn_fused(const GdnFusedArgs &a) {
    __shared__ float red_mem[GDN_GROUPS][GDN_COLS];
    __shared__ float red_out[GDN_GROUPS][GDN_COLS];
    __shared__ float red_nrm[2][GDN_GROUPS];
    __shared__ float qs[256], ks[256], vs[GDN_COLS], gsc[2];

    const uint32_t slices = (a.value_dim + GDN_COLS - 1) / GDN_COLS;
    const uint32_t h = blockIdx.x / slices, slice = blockIdx.x % slices;
    const uint32_t tid = threadIdx.x, jj = tid % GDN_COLS, ig = tid / GDN_COLS;
    const uint32_t j = slice * GDN_COLS + jj;
    const bool colok = j < a.value_dim;
    const uint32_t dk = a.key_dim, rep = a.heads / a.key_heads, kh = h / rep;
    const uint32_t kw = a.key_heads * dk, K = a.kernel;
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

    // This thread's inputs of a token (its conv channels, and the gate
    // inputs for thread 255) are loaded ahead of the stores of earlier
    // tokens: a load issued after a store waits for it (loads and stores
    // retire in one in-order counter).
    const GdnBuf pr = gdn_buf(a.proj, (size_t)a.tokens * a.proj_stride);
    const GdnBuf dr = gdn_buf(a.gates_given ? a.log_decay : nullptr, (size_t)a.tokens * a.heads);
    const GdnBuf br = gdn_buf(a.gates_given ? a.beta : nullptr, (size_t)a.tokens * a.heads);
    auto load_in = [&](uint32_t t, float &xq, float &xv, float &ga, float &gb) {
        const uint32_t row = t * a.proj_stride, th = t * a.heads + h;
        xq = gdn_ld(pr, qk_thr, (row + qk_ch) * 4);
        xv = gdn_ld(pr, v_thr, (row + v_ch) * 4);
        const bool g = tid == 255;
        if (a.gates_given) {
            ga = gdn_ld(dr, g, th * 4);
            gb = gdn_ld(br, g, th * 4);
        } else {
            ga = gdn_ld(pr, g, (row + a.a_off + h) * 4);
            gb = gdn_ld(pr, g, (row + a.b_off + h) * 4);
        }
    };
    const float dtb = tid == 255 && !a.gates_given ? a.dt_bias[h] : 0.0f;
    const float alog = tid == 255 && !a.gates_given ? a.a_log[h] : 0.0f;
    // One token's step on inputs already in registers.
    auto step = [&](uint32_t t, float cxq, float cxv, float cga, float cgb) {
        // Conv step: shift the window left by one, append the input.
        if (qk_thr) {
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i + 1 < GDN_MAX_KERNEL; i++)
                if ((uint32_t)i + 1 < K) {
                    const float v = sq_[i + 1];
                    sq_[i] = v;
                    sum += v * wq[i];
                }
            const float x = cxq;
#pragma unroll
            for (int i = 0; i < GDN_MAX_KERNEL; i++)
                if ((uint32_t)i == K - 1) sq_[i] = x;
            float wl = 0.0f;
#pragma unroll
            for (int i = 0; i < GDN_MAX_KERNEL; i++)
                if ((uint32_t)i == K - 1) wl = wq[i];
            sum += x * wl;
            const float y = sum / (1.0f + expf(-sum));
            if (tid < dk) qs[tid] = y;
            else ks[tid - dk] = y;
        }
        if (v_thr) {
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i + 1 < GDN_MAX_KERNEL; i++)
                if ((uint32_t)i + 1 < K) {
                    const float v = sv_[i + 1];
                    sv_[i] = v;
                    sum += v * wv[i];
                }
            const float x = cxv;
            float wl = 0.0f;
#pragma unroll
            for (int i = 0; i < GDN_MAX_KERNEL; i++)
                if ((uint32_t)i == K - 1) {
                    sv_[i] = x;
                    wl = wv[i];
                }
            sum += x * wl;
            vs[tid] = sum / (1.0f + expf(-sum));
        }
        if (tid == 255) {
            const size_t th = (size_t)t * a.heads + h;
            float be, ld;
            if (a.gates_given) {
                be = cgb;
                ld = cga;
            } else {
                be = 1.0f / (1.0f + expf(-cgb));
                const float x = cga + dtb;
                const float sp = x > 20.0f ? x : log1pf(expf(x));
                ld = -expf(alog) * sp;
                if (slice == 0) {
                    a.beta[th] = be;
                    a.log_decay[th] = ld;
                }
            }
            gsc[0] = expf(ld);
            gsc[1] = be;
        }
        lds_barrier();
        const float decay = gsc[0], beta = gsc[1];
        const float vjv = colok ? vs[jj] : 0.0f;
        float kk[GDN_MAX_ROWS], qq[GDN_MAX_ROWS];
        float mem = 0.0f, sk = 0.0f, sqq = 0.0f;
#pragma unroll
        for (int r = 0; r < GDN_MAX_ROWS; r++) {
            const uint32_t i = ig + GDN_GROUPS * r;
            const bool ok = (uint32_t)r < nrows && i < dk;
            kk[r] = ok ? ks[i] : 0.0f;
            qq[r] = ok ? qs[i] : 0.0f;
            sk += kk[r] * kk[r];
            sqq += qq[r] * qq[r];
            s[r] = s[r] * decay;
            mem += s[r] * kk[r];
        }
        red_mem[ig][jj] = mem;
        if (jj == 0) {
            red_nrm[0][ig] = sk;
            red_nrm[1][ig] = sqq;
        }
        lds_barrier();
        float memj = 0.0f, ssk = 0.0f, ssq = 0.0f;
#pragma unroll
        for (int gi = 0; gi < GDN_GROUPS; gi++) {
            memj += red_mem[gi][jj];
            ssk += red_nrm[0][gi];
            ssq += red_nrm[1][gi];
        }
        const float kinv = 1.0f / sqrtf(ssk + 1e-6f), qinv = 1.0f / sqrtf(ssq + 1e-6f);
        const float delta = (vjv - memj * kinv) * beta;
        float o = 0.0f;
#pragma unroll
        for (int r = 0; r < GDN_MAX_ROWS; r++) {
            s[r] += kk[r] * kinv * delta;
            o += s[r] * qq[r];
        }
        red_out[ig][jj] = o;
        lds_barrier();
        if (ig == 0 && colok) {
            float oj = 0.0f;
#pragma unroll
            for (int gi = 0; gi < GDN_GROUPS; gi++) oj += red_out[gi][jj];
            a.out[((size_t)t * a.heads + h) * a.value_dim + j] = oj * qinv * qscale;
        }
        if (a.snap_stride) {
            // Row snapshot: the state and conv windows after token t.
            store_state(a.state_out + (size_t)t * a.snap_stride);
            float *co = a.conv_out + (size_t)t * a.conv_snap_stride;
            if (qk_thr && h % rep == 0 && slice == 0)
#pragma unroll
                for (int i = 0; i < GDN_MAX_KERNEL; i++)
                    if ((uint32_t)i < K) co[(size_t)qk_ch * K + i] = sq_[i];
            if (v_thr)
#pragma unroll
                for (int i = 0; i < GDN_MAX_KERNEL; i++)
                    if ((uint32_t)i < K) co[(size_t)v_ch * K + i] = sv_[i];
        }
        // qs/ks/vs/gsc and red_* are rewritten next token only after every
        // thread has passed this barrier.
        lds_barrier();
    };
    if (a.tokens <= GDN_PREFETCH) {
        // Every token's inputs are loaded before the first token's stores,
        // so no wait inside the loop ever covers an earlier store (the
        // verify rows' snapshots stream out while later tokens compute).
        float pq[GDN_PREFETCH], pv[GDN_PREFETCH], pa[GDN_PREFETCH], pb[GDN_PREFETCH];
#pragma unroll
        for (int u = 0; u < GDN_PREFETCH; u++) load_in(min((uint32_t)u, a.tokens - 1), pq[u], pv[u], pa[u], pb[u]);
        for (uint32_t t = 0; t < a.tokens; t++) {
            step(t, pq[0], pv[0], pa[0], pb[0]);
#pragma unroll
            for (int u = 0; u + 1 < GDN_PREFETCH; u++) {
                pq[u] = pq[u + 1];
                pv[u] = pv[u + 1];
                pa[u] = pa[u + 1];
                pb[u] = pb[u + 1];
            }
        }
    } else {
        float nxq, nxv, nga, ngb;
        load_in(0, nxq, nxv, nga, ngb);
        for (uint32_t t = 0; t < a.tokens; t++) {
            const float cxq = nxq, cxv = nxv, cga = nga, cgb = ngb;
            if (t + 1 < a.tokens) load_in(t + 1, nxq, nxv, nga, ngb);
            step(t, cxq, cxv, cga, cgb);
        }
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

// The crate's state layout, and the engine's blocked one (state_blocked).
extern "C" __global__ __launch_bounds__(256) void ctox_gdn_fused_gfx950(GdnFusedArgs a) { gdn_fused<false>(a); }
extern "C" __global__ __launch_bounds__(256) void ctox_gdn_fused_blk_gfx950(GdnFusedArgs a) { gdn_fused<true>(a); }
