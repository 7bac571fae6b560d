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
// through LDS.
#include <hip/hip_runtime.h>

#include "kernel_args.h"

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
        __syncthreads();
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
        __syncthreads();
        if (ig == 0 && colok) {
            float oj = 0.0f;
#pragma unroll
            for (int gi = 0; gi < GDN_GROUPS; gi++) oj += red_out[gi][jj];
            a.out[th * a.value_dim + j] = oj * qinv * qscale;
        }
        // red_* are rewritten next token only after every thread has passed
        // the second barrier of this token and read red_mem / red_nrm; the
        // reads of red_out happen before the next token's first barrier.
        __syncthreads();
    }

#pragma unroll
    for (int r = 0; r < GDN_MAX_ROWS; r++) {
        const uint32_t i = ig + GDN_GROUPS * r;
        if ((uint32_t)r < nrows && i < a.key_dim && colok) S[(size_t)i * a.value_dim + j] = s[r];
    }
}
