// Batch-1 Q2_B64 / Q4_B64 fused matvec for rows of whole 16-byte units
// (columns % 512 == 0, 16-byte aligned weights): the "slice" kernels.
//
// Same result as Q/src/backend/cpu.rs:242-310 and the same arithmetic as the
// block-diagonal path in qmatvec.hip (exact int8 limbs of the fixed-point
// activation against the unpacked codes on v_mfma_i32_16x16x64_i8). What
// differs is how HBM is streamed:
//  * A workgroup owns one 16-row tile and walks its K range in slices of SB
//    blocks (28 for Q4, 56 for Q2): SB * BB plus the 16-byte phase fits in
//    the 64 16-byte units of one wave-wide load, so every weight load is a
//    fully coalesced 1 KiB run of one row. Wave w loads rows 2w, 2w+1 of the
//    slice; the eight waves together stage the 16 x 1 KiB slice in LDS
//    (row stride 1040 bytes: at most 2-way bank conflicts on the per-block
//    dword reads) together with the slice's activation fragments.
//  * The slice's 4-block MFMA groups are split over the eight waves, so the
//    dependent LDS -> unpack -> MFMA -> epilogue chain of a slice is short
//    and many waves hide each other's latency.
//  * Loads run ahead of compute: with NS > 0 (compile-time slice count)
//    every slice of the tile is requested before the first is consumed
//    (straight-line code, exact vmcnt waits); with NS == 0 the next slice is
//    requested while the current one is computed. Workgroup barriers fence
//    LDS only, so they never drain the outstanding global loads.
//  * Every wave keeps its per-row partial in a register across slices; the
//    eight partials are added in LDS in a fixed order (deterministic), then
//    /15 (Q4) or /3 (Q2), bias, s_out and SiLU.
#include "lds_barrier.h"

template <int DT>
struct SlCfg {
    static constexpr uint32_t BB = DT ? CTOX_Q4_BLOCK_BYTES : CTOX_Q2_BLOCK_BYTES;
    static constexpr uint32_t CD = DT ? 8 : 4;        // code dwords per block
    static constexpr uint32_t SB = ctox_slice_blocks(DT);
    static constexpr uint32_t NG = SB / 4;            // MFMA groups per slice
    static constexpr uint32_t NW = CTOX_SLICE_WAVES, NT = NW * 64;
    static constexpr uint32_t RPW = 16 / NW;          // rows per wave per slice
    static constexpr uint32_t GPW = (NG + NW - 1) / NW;
    static constexpr uint32_t AU = (SB * 12 + NT - 1) / NT;  // fragment v4i per thread
    static constexpr uint32_t STR = 1040;             // LDS bytes per staged row
    static constexpr float DEN = DT ? 15.0f : 3.0f;
};

template <int DT>
struct SlLoad {
    v4i wv[SlCfg<DT>::RPW];
    v4i av[SlCfg<DT>::AU];
    v4i cv;
};

template <int DT, int NS>
__device__ __forceinline__ void qmatvec_slices(const MatvecArgs &a) {
    using C = SlCfg<DT>;
    // 16 bytes in front of the stage: the first block's scale read starts one
    // dword before the stage when the slice phase is 0.
    __shared__ __align__(16) uint8_t stage_raw[16 + 16 * C::STR + 64];
    __shared__ __align__(16) int8_t xal[C::AU * C::NT * 16];
    __shared__ __align__(16) float4 xcl[64];
    __shared__ __align__(16) int8_t zero[64];
    __shared__ float red[C::NW][16];
    uint8_t *stage = stage_raw + 16;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nb = a.columns / CTOX_BLOCK_LEN, R = nb * C::BB;
    const uint32_t ns = (nb + C::SB - 1) / C::SB;
    const uint32_t row0 = blockIdx.x * 16, last = a.rows - 1 - row0;
    const uint8_t *wbase = a.weights + (size_t)row0 * R;
    const uint64_t remain = (uint64_t)(a.rows - row0) * R;
    // Loads past the last row's end (last slice, last row) return zeros.
    __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)wbase, (short)0, (int)(remain > 0x7ffffff0ULL ? 0x7ffffff0ULL : remain), 0x00020000);
    __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void *)a.xa, (short)0, (int)(nb * 192), 0x00020000);
    __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc((void *)a.xc, (short)0, (int)(nb * 16), 0x00020000);
    if (tid < 4) ((v4i *)zero)[tid] = (v4i){0, 0, 0, 0};

    auto issue = [&](SlLoad<DT> &sl, uint32_t s) {
        const uint32_t sb0 = s * C::SB, a0 = (sb0 * C::BB) & ~15u;
#pragma unroll
        for (int r = 0; r < (int)C::RPW; r++)
            sl.wv[r] = __builtin_amdgcn_raw_buffer_load_b128(wr, a0 + lane * 16, min(C::RPW * w + r, last) * R, 0);
#pragma unroll
        for (int i = 0; i < (int)C::AU; i++)
            sl.av[i] = __builtin_amdgcn_raw_buffer_load_b128(xr, sb0 * 192 + (i * C::NT + tid) * 16, 0, 0);
        sl.cv = __builtin_amdgcn_raw_buffer_load_b128(cr, (sb0 + lane) * 16, 0, 0);
    };

    const uint32_t g = lane >> 4, j = lane & 15;
    const uint32_t t = j >> 2, limb = j & 3;
    const bool aok = t == g && limb < 3;  // A row group t carries block t, k-group t only
    const uint32_t *lds32 = (const uint32_t *)stage;
    float acc = 0.0f;

    // Stage slice s from registers, then run this wave's share of its groups.
    auto consume = [&](const SlLoad<DT> &sl, uint32_t s) {
        const uint32_t sb0 = s * C::SB;
        const uint32_t nbs = s < ns ? min(C::SB, nb - sb0) : 0u;
        const uint32_t ph = (sb0 * C::BB) & 15u;
        lds_barrier();  // the previous slice is fully consumed
#pragma unroll
        for (int r = 0; r < (int)C::RPW; r++) *(v4i *)(stage + (C::RPW * w + r) * C::STR + lane * 16) = sl.wv[r];
#pragma unroll
        for (int i = 0; i < (int)C::AU; i++) *(v4i *)(xal + (i * C::NT + tid) * 16) = sl.av[i];
        if (w == 0)
            xcl[lane] = make_float4(__int_as_float(sl.cv[0]), __int_as_float(sl.cv[1]), __int_as_float(sl.cv[2]),
                                    __int_as_float(sl.cv[3]));
        lds_barrier();
#pragma unroll
        for (uint32_t k = 0; k < C::GPW; k++) {
            const uint32_t G = w + C::NW * k;
            if (G < C::NG) {
                const uint32_t boff = j * C::STR + ph + (4 * G + g) * C::BB;
                const uint32_t d0 = (boff + 2) >> 2, sft = (boff + 2) & 3;
                uint32_t d[C::CD + 2];
#pragma unroll
                for (int q = 0; q < (int)C::CD + 2; q++) d[q] = lds32[d0 + q - 1];
                const int8_t *ap = aok ? xal + (4 * G + g) * 192 + limb * 64 : zero;
                v4i af[4];
#pragma unroll
                for (int q = 0; q < 4; q++) af[q] = *(const v4i *)(ap + (aok ? q * 16 : 0));
                const float4 kq = xcl[4 * G + g];
                uint32_t cd[C::CD];
#pragma unroll
                for (int q = 0; q < (int)C::CD; q++) cd[q] = __builtin_amdgcn_alignbyte(d[q + 2], d[q + 1], sft);
                // Scale bits: upper half of d[0] (sft 0) or lower half of d[1]
                // (sft 2); blocks past the slice are masked to 0.0.
                const uint32_t sbits = __builtin_amdgcn_perm(d[1], d[0], sft == 0 ? 0x0c0c0302u : 0x0c0c0504u);
                const uint32_t vmask = (4 * G + g < nbs) ? 0xffffffffu : 0u;
                const float scale = __uint_as_float(__float_as_uint(half_bits_to_float(sbits)) & vmask);
                v4i cc = (v4i){0, 0, 0, 0};
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const v4i bf = DT ? unpack_quarter<DT>(cd[2 * q], cd[2 * q + 1]) : unpack_quarter<DT>(cd[q], 0);
                    cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[q], bf, cc, 0, 0, 0);
                }
                float f = fmaf((float)cc[0], kq.x, kq.w);
                f = fmaf((float)cc[1], kq.y, f);
                f = fmaf((float)cc[2], kq.z, f);
                acc = fmaf(f, scale, acc);
            }
        }
    };

    if (NS > 0) {
        // Split K (gridDim.y > 1): workgroup y takes slices NS y .. NS y + NS - 1;
        // slices past the row are masked (their blocks count as zero).
        const uint32_t s0 = blockIdx.y * NS;
        SlLoad<DT> sl[NS > 0 ? NS : 1];
#pragma unroll
        for (int s = 0; s < NS; s++) {
            issue(sl[s], min(s0 + (uint32_t)s, ns - 1));
            __builtin_amdgcn_sched_barrier(0);  // keep slices in request order
        }
#pragma unroll
        for (int s = 0; s < NS; s++) consume(sl[s], s0 + s);
    } else {
        SlLoad<DT> cur;
        issue(cur, 0);
        for (uint32_t s = 0; s < ns; s++) {
            const SlLoad<DT> now = cur;
            if (s + 1 < ns) issue(cur, s + 1);
            consume(now, s);
        }
    }

    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    if (g == 0) red[w][j] = acc;
    __syncthreads();
    if (tid < 16 && row0 + tid < a.rows) {
        float sum = 0.0f;
#pragma unroll
        for (int q = 0; q < (int)C::NW; q++) sum += red[q][tid];
        a.output[(size_t)blockIdx.y * a.part_stride + row0 + tid] = epilogue(sum / C::DEN, row0 + tid, a);
    }
}

#define CTOX_SLICE_KERNEL(name, dt, ns)                                                  \
    extern "C" __global__ __launch_bounds__(CTOX_SLICE_WAVES * 64) void name(MatvecArgs a) { \
        qmatvec_slices<dt, ns>(a);                                                       \
    }
CTOX_SLICE_KERNEL(ctox_q4_matvec_sl_gfx950, 1, 0)
CTOX_SLICE_KERNEL(ctox_q4_matvec_sl1_gfx950, 1, 1)
CTOX_SLICE_KERNEL(ctox_q4_matvec_sl2_gfx950, 1, 2)
CTOX_SLICE_KERNEL(ctox_q4_matvec_sl3_gfx950, 1, 3)
CTOX_SLICE_KERNEL(ctox_q2_matvec_sl_gfx950, 0, 0)
CTOX_SLICE_KERNEL(ctox_q2_matvec_sl1_gfx950, 0, 1)
CTOX_SLICE_KERNEL(ctox_q2_matvec_sl2_gfx950, 0, 2)
CTOX_SLICE_KERNEL(ctox_q2_matvec_sl3_gfx950, 0, 3)

// ---------------------------------------------------------------------------
// Small-M (2..8 rows of activation) slice kernels: the same 16-row tiles,
// 8 waves and coalesced row-slice staging as above, with the token-stacked
// MFMA of qmatvec.hip: A rows 4t + limb carry token t's limbs of one block,
// B lane (g, j) carries quarter g of that block of row j, and C lane (g, j)
// holds token 4 * tg + g of row j. A slice is 28 (Q4) or 26 (Q2) blocks:
// one row of it fits 61 (Q4) or 31 (Q2) 16-byte units, so a Q2 load moves
// two rows (32 lanes each); lanes past the slice read out of range (zeros,
// no memory traffic). The slice's M-token fragments (SB * M * 192 bytes)
// are staged once per workgroup; the waves split the slice's blocks.
template <int DT>
struct TkCfg {
    static constexpr uint32_t BB = DT ? CTOX_Q4_BLOCK_BYTES : CTOX_Q2_BLOCK_BYTES;
    static constexpr uint32_t QB = DT ? 8 : 4;        // code bytes per quarter block
    static constexpr uint32_t SB = DT ? 28 : 26;
    static constexpr uint32_t UPR = DT ? 64 : 32;     // lanes per row in a load
    static constexpr uint32_t RPL = 64 / UPR;         // rows per load instruction
    static constexpr uint32_t NW = CTOX_SLICE_WAVES, NT = NW * 64;
    static constexpr uint32_t LPW = 16 / (NW * RPL);  // loads per wave per slice
    static constexpr uint32_t BPW = (SB + NW - 1) / NW;
    static constexpr uint32_t STR = 1040;
    static constexpr float DEN = DT ? 15.0f : 3.0f;
};
static_assert(ctox_slice_blocks_tok(0) == TkCfg<0>::SB && ctox_slice_blocks_tok(1) == TkCfg<1>::SB, "slice size");

template <int DT, int TG>
__device__ __forceinline__ void qmatvec_slices_tok(const MatvecArgs &a) {
    using C = TkCfg<DT>;
    constexpr uint32_t MAXB = 4 * TG;
    constexpr uint32_t AU = (C::SB * MAXB * 12 + C::NT - 1) / C::NT;  // fragment v4i per thread
    __shared__ __align__(16) uint8_t stage_raw[16 + 16 * C::STR + 64];
    __shared__ __align__(16) int8_t xal[AU * C::NT * 16];
    __shared__ __align__(16) float4 xcl[C::SB * MAXB];
    __shared__ float red[C::NW][MAXB][16];
    uint8_t *stage = stage_raw + 16;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t batch = a.batch;
    const uint32_t nb = a.columns / CTOX_BLOCK_LEN, R = nb * C::BB;
    const uint32_t ns = (nb + C::SB - 1) / C::SB;
    const uint32_t row0 = blockIdx.x * 16, last = a.rows - 1 - row0;
    const uint8_t *wbase = a.weights + (size_t)row0 * R;
    const uint64_t remain = (uint64_t)(a.rows - row0) * R;
    __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)wbase, (short)0, (int)(remain > 0x7ffffff0ULL ? 0x7ffffff0ULL : remain), 0x00020000);
    __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void *)a.xa, (short)0, (int)(nb * batch * 192), 0x00020000);
    __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc((void *)a.xc, (short)0, (int)(nb * batch * 16), 0x00020000);
    const uint32_t lrow = lane / C::UPR, lunit = lane % C::UPR;

    struct Ld {
        v4i wv[C::LPW];
        v4i av[AU];
        v4i cv;
    };
    auto issue = [&](Ld &sl, uint32_t s) {
        const uint32_t sb0 = s * C::SB, nbs = min(C::SB, nb - sb0);
        const uint32_t a0 = (sb0 * C::BB) & ~15u, ph = (sb0 * C::BB) & 15u;
        const uint32_t units = (ph + nbs * C::BB + 15) >> 4;
        const uint32_t voff = lunit < units ? a0 + lunit * 16 : 0x7ffffff0u;  // out of range: zeros, no traffic
#pragma unroll
        for (int r = 0; r < (int)C::LPW; r++) {
            const uint32_t row = (w * C::LPW + r) * C::RPL + lrow;
            sl.wv[r] = __builtin_amdgcn_raw_buffer_load_b128(wr, voff, min(row, last) * R, 0);
        }
#pragma unroll
        for (int i = 0; i < (int)AU; i++)
            sl.av[i] = __builtin_amdgcn_raw_buffer_load_b128(xr, sb0 * batch * 192 + (i * C::NT + tid) * 16, 0, 0);
        sl.cv = __builtin_amdgcn_raw_buffer_load_b128(cr, sb0 * batch * 16 + tid * 16, 0, 0);
    };

    const uint32_t g = lane >> 4, j = lane & 15;
    const uint32_t *lds32 = (const uint32_t *)stage;
    float acc[TG];
#pragma unroll
    for (int tg = 0; tg < TG; tg++) acc[tg] = 0.0f;

    auto consume = [&](const Ld &sl, uint32_t s) {
        const uint32_t sb0 = s * C::SB, nbs = min(C::SB, nb - sb0);
        const uint32_t ph = (sb0 * C::BB) & 15u;
        lds_barrier();
#pragma unroll
        for (int r = 0; r < (int)C::LPW; r++) {
            const uint32_t row = (w * C::LPW + r) * C::RPL + lrow;
            *(v4i *)(stage + row * C::STR + lunit * 16) = sl.wv[r];
        }
#pragma unroll
        for (int i = 0; i < (int)AU; i++) *(v4i *)(xal + (i * C::NT + tid) * 16) = sl.av[i];
        if (tid < C::SB * MAXB && tid < nbs * batch)
            xcl[tid] = make_float4(__int_as_float(sl.cv[0]), __int_as_float(sl.cv[1]), __int_as_float(sl.cv[2]),
                                   __int_as_float(sl.cv[3]));
        lds_barrier();
#pragma unroll
        for (uint32_t k = 0; k < C::BPW; k++) {
            const uint32_t bl = w + C::NW * k;
            if (bl < nbs) {
                const uint32_t boff = j * C::STR + ph + bl * C::BB;
                const uint32_t sd = lds32[boff >> 2];
                const uint32_t sbits = (boff & 2) ? (sd >> 16) : (sd & 0xffffu);
                const float scale = half_bits_to_float(sbits);
                const uint32_t ca = boff + 2 + C::QB * g, sftq = ca & 3;
                const uint32_t c0 = lds32[ca >> 2], c1 = lds32[(ca >> 2) + 1];
                const uint32_t w0 = __builtin_amdgcn_alignbyte(c1, c0, sftq);
                uint32_t w1 = 0;
                if (DT) w1 = __builtin_amdgcn_alignbyte(lds32[(ca >> 2) + 2], c1, sftq);
                const v4i bf = unpack_quarter<DT>(w0, w1);
#pragma unroll
                for (int tg = 0; tg < TG; tg++) {
                    const uint32_t tok = tg * 4 + (j >> 2), limb = j & 3;
                    const bool aok = limb < 3 && tok < batch;
                    const uint32_t tok_c = min(tok, batch - 1), limb_c = min(limb, 2u);
                    const v4i av = *(const v4i *)(xal + ((bl * batch + tok_c) * 3 + limb_c) * 64 + g * 16);
                    const v4i af = aok ? av : (v4i){0, 0, 0, 0};
                    const v4i cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf, (v4i){0, 0, 0, 0}, 0, 0, 0);
                    const float4 kq = xcl[bl * batch + min((uint32_t)(tg * 4) + g, batch - 1)];
                    float f = fmaf((float)cc[0], kq.x, kq.w);
                    f = fmaf((float)cc[1], kq.y, f);
                    f = fmaf((float)cc[2], kq.z, f);
                    acc[tg] = fmaf(f, scale, acc[tg]);
                }
            }
        }
    };

    Ld cur;
    issue(cur, 0);
    for (uint32_t s = 0; s < ns; s++) {
        const Ld now = cur;
        if (s + 1 < ns) issue(cur, s + 1);
        consume(now, s);
    }
#pragma unroll
    for (int tg = 0; tg < TG; tg++) red[w][tg * 4 + g][j] = acc[tg];
    __syncthreads();
    if (tid < batch * 16) {
        const uint32_t tok = tid >> 4, jj = tid & 15, row = row0 + jj;
        float sum = 0.0f;
#pragma unroll
        for (int q = 0; q < (int)C::NW; q++) sum += red[q][tok][jj];
        if (row < a.rows) a.output[(size_t)tok * a.out_stride + row] = epilogue(sum / C::DEN, row, a);
    }
}

#define CTOX_SLICE_TOK_KERNEL(name, dt, tg)                                              \
    extern "C" __global__ __launch_bounds__(CTOX_SLICE_WAVES * 64) void name(MatvecArgs a) { \
        qmatvec_slices_tok<dt, tg>(a);                                                   \
    }
CTOX_SLICE_TOK_KERNEL(ctox_q4_matvec_st4_gfx950, 1, 1)
CTOX_SLICE_TOK_KERNEL(ctox_q4_matvec_st8_gfx950, 1, 2)
CTOX_SLICE_TOK_KERNEL(ctox_q2_matvec_st4_gfx950, 0, 1)
CTOX_SLICE_TOK_KERNEL(ctox_q2_matvec_st8_gfx950, 0, 2)
