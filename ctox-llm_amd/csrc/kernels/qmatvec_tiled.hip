// Batch-1 fused matvec over the tiled weight layout (resident matrices).
//
// Same result as Q/src/backend/cpu.rs:242-310 and the same exact int8
// arithmetic as qmatvec.hip (block-diagonal MFMA over fixed-point activation
// limbs). What differs is how the weights reach the matrix cores:
//  * At prepare time every matrix is rewritten once into 16-row x 16-block
//    units whose bytes are already in MFMA B-fragment order (layout in
//    kernel_args.h). A lane's 16-byte load is its own fragment, a wave's
//    load is one contiguous, aligned KiB, and nothing is staged in LDS.
//  * A wave owns one 16-block column chunk for all its row tiles: the
//    chunk's activation fragments (4 groups x 4 quarters) and epilogue
//    constants sit in registers. They are either loaded from a prep
//    kernel's output or (AB = 1) built from x and s_in by the workgroup's
//    four waves (one group each, exchanged through LDS), so a batch-1
//    dispatch is a single launch.
//  * Each wave takes up to U row tiles of its chunk; every
//    load of all of them is issued before the first MFMA (straight-line
//    code, loads past the wave's tiles fall outside the buffer range and
//    return zeros without memory traffic).
//  * Splitting K into chunks spreads any matrix evenly over the CUs. The
//    chunk sums of a row tile are added in chunk order (deterministic) by
//    the last chunk's waves when the whole launch is resident at once, else
//    by the chunk that arrives last at the tile's count.
#include "kernel_args.h"
#include "lds_barrier.h"

// Cache policy of streamed weight loads: non-temporal.
#define CTOX_LOAD_NT 2
// Most producer chunk partials an in-kernel SwiGLU build sums.
#define CTOX_MAX_IN_PARTS 6

typedef unsigned int v2u __attribute__((ext_vector_type(2)));

template <int DT>
struct TlCfg {
    static constexpr uint32_t LPU = DT ? 8 : 4;  // 16-byte code loads per lane per unit
    static constexpr uint32_t CB = ctox_tile_code_bytes(DT);
    static constexpr uint32_t UB = ctox_tile_unit_bytes(DT);
    static constexpr float DEN = DT ? 15.0f : 3.0f;
};

template <int DT>
struct TileUnit {
    v4i w[TlCfg<DT>::LPU];
    v2u s;
};

// Builds the chunk's activation fragments from x (times s_in) inside the
// wave, with exactly the arithmetic of prep_block in qmatvec.hip: per
// 64-column block the fixed point X = rint(x' * 2^(22 - e)) (|x'| < 2^e),
// three balanced int8 limbs, and the epilogue constants
// {2q, 512q, 131072q, -off * sum(X) * q}, q = 2^(e - 22); a block holding a
// non-finite value gets q = NaN. Lane 16 t + m of group G holds elements
// 4m .. 4m + 3 of block 4G + t, so a block is one 16-lane row and every
// reduction stays inside it. The limbs go through a wave-private LDS area
// into the A-fragment order (the B unpack order of frag_pos). Reductions
// over a row use row16_reduce (DPP, qmatvec.hip).

// Raw inputs of one 4-block group of the in-kernel fragment build.
struct GroupIn {
    v4i a, b, w, s;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t f32_rsrc(const void *p, uint32_t floats) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, p ? (int)(floats * 4) : 0, 0x00020000);
}

// Epilogue operands of one output row (bias, s_out and, with residual sums,
// the residual input of token row `tok`; res_h rows are `rows` apart), read
// ahead of the combine so their latency overlaps the poll. Branch-free: an
// absent operand has an empty range and reads 0. Raw bits until applied.
struct EpiIn {
    uint32_t bias, s16, s32, h;
};
__device__ __forceinline__ EpiIn epi_load(const TileMatvecArgs &a, uint32_t row, uint32_t tok) {
    const bool f16 = a.s_out_kind == CTOX_KSCALE_F16, f32 = a.s_out_kind == CTOX_KSCALE_F32;
    const __amdgpu_buffer_rsrc_t s16 =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.s_out, (short)0, f16 ? (int)(a.rows * 2) : 0, 0x00020000);
    EpiIn e;
    e.bias = __builtin_amdgcn_raw_buffer_load_b32(f32_rsrc(a.bias, a.rows), row * 4, 0, 0);
    e.s16 = __builtin_amdgcn_raw_buffer_load_b16(s16, row * 2, 0, 0);
    e.s32 = __builtin_amdgcn_raw_buffer_load_b32(f32_rsrc(f32 ? a.s_out : nullptr, a.rows), row * 4, 0, 0);
    e.h = __builtin_amdgcn_raw_buffer_load_b32(f32_rsrc(a.res_sq ? a.res_h : nullptr, (tok + 1) * a.rows),
                                               (tok * a.rows + row) * 4, 0, 0);
    return e;
}
// Output epilogue: + bias, x s_out, then SiLU when asked.
__device__ __forceinline__ float epi_apply(float v, const EpiIn &e, const TileMatvecArgs &a) {
    if (a.bias) v += __uint_as_float(e.bias);
    if (a.s_out_kind == CTOX_KSCALE_F16) v *= half_bits_to_float(e.s16 & 0xffffu);
    if (a.s_out_kind == CTOX_KSCALE_F32) v *= __uint_as_float(e.s32);
    if (a.activation == 1) v = v / (1.0f + expf(-v));
    return v;
}

// Loads of one 4-block group's activation inputs (TileMatvecArgs::xmode);
// branch-free: an unused or absent input has an empty range and reads zeros,
// so no wait lands in a divergent block ahead of weight loads in flight.
// Lane 16 t + m takes columns 4m .. 4m + 3 of block 4 grp + t.
__device__ __forceinline__ void frag_group_loads(const TileMatvecArgs &a, uint32_t grp, uint32_t lane, GroupIn &in,
                                                 uint32_t xm) {
    const uint32_t cols = a.blocks * CTOX_BLOCK_LEN, dh = a.head_dim;
    const uint32_t col = (4 * grp + (lane >> 4)) * CTOX_BLOCK_LEN + 4 * (lane & 15);
    const uint32_t sbytes = a.s_in_kind == CTOX_KSCALE_F32 ? 4u : 2u;
    const __amdgpu_buffer_rsrc_t ar = f32_rsrc(a.input, xm == 2 ? a.off + cols : cols);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)a.s_in, (short)0, a.s_in_kind == CTOX_KSCALE_NONE ? 0 : (int)(cols * sbytes), 0x00020000);
    const void *bp = xm == 1 ? (const void *)a.delta : (xm == 2 ? (const void *)a.input : (const void *)a.xb);
    const uint32_t bn = xm == 1 || xm == 3 ? cols : (xm == 2 ? a.off + cols : (xm == 4 ? 2 * cols : 0u));
    const uint32_t bo = xm == 2 ? a.off + col : (xm == 4 ? (col / dh) * 2 * dh + dh + col % dh : col);
    const __amdgpu_buffer_rsrc_t br = f32_rsrc(xm == 0 ? nullptr : bp, bn);
    const __amdgpu_buffer_rsrc_t wr = f32_rsrc(xm == 1 || xm == 3 ? a.xw : nullptr, xm == 1 ? cols : dh);
    if (xm == 2 && a.a_parts > 1) {
        // SwiGLU over a producer's chunk partials: a = sum_k part_k[c],
        // b = sum_k part_k[off + c], in part order.
        const __amdgpu_buffer_rsrc_t pr = f32_rsrc(a.input, (a.a_parts - 1) * a.a_pstride + a.off + cols);
        v4i pa[CTOX_MAX_IN_PARTS], pb[CTOX_MAX_IN_PARTS];
#pragma unroll
        for (int k = 0; k < CTOX_MAX_IN_PARTS; k++) {
            const uint32_t o = (uint32_t)k < a.a_parts ? k * a.a_pstride : 0x10000000u;
            pa[k] = __builtin_amdgcn_raw_buffer_load_b128(pr, (o + col) * 4, 0, 0);
            pb[k] = __builtin_amdgcn_raw_buffer_load_b128(pr, (o + a.off + col) * 4, 0, 0);
        }
        v4i sa = pa[0], sb = pb[0];
#pragma unroll
        for (int k = 1; k < CTOX_MAX_IN_PARTS; k++)
            if ((uint32_t)k < a.a_parts)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    sa[i] = __float_as_int(__int_as_float(sa[i]) + __int_as_float(pa[k][i]));
                    sb[i] = __float_as_int(__int_as_float(sb[i]) + __int_as_float(pb[k][i]));
                }
        in.a = sa;
        in.b = sb;
    } else {
        in.a = __builtin_amdgcn_raw_buffer_load_b128(ar, col * 4, 0, 0);
        in.b = __builtin_amdgcn_raw_buffer_load_b128(br, bo * 4, 0, 0);
    }
    in.w = __builtin_amdgcn_raw_buffer_load_b128(wr, (xm == 3 ? col % (dh ? dh : 1) : col) * 4, 0, 0);
    in.s = __builtin_amdgcn_raw_buffer_load_b128(sr, col * sbytes, 0, 0);
}

__device__ __forceinline__ float tl_silu(float v) { return v / (1.0f + expf(-v)); }

// Builds one group's activation fragments with exactly the arithmetic of
// prep_block in qmatvec.hip: per 64-column block the fixed point
// X = rint(x' * 2^(22 - e)) (|x'| < 2^e), three balanced int8 limbs, and the
// epilogue constants {2q, 512q, 131072q, -off * sum(X) * q}, q = 2^(e - 22);
// a block holding a non-finite value gets q = NaN. x' is the transformed
// input (xmode, with the row's inverse RMS `inv` for the residual norm)
// times s_in. A block is one 16-lane row, so the block reductions stay
// inside it (DPP). The limbs are written to `frag` (4 blocks x 192 bytes,
// the prep kernel's xa order); lane (g, j) receives the constants of
// block g. With `keep` the residual and normalized values of the lane's
// columns are stored (residual norm, segment-0 workgroup).
// `bstride`: bytes between the group's blocks in `frag` (192: the blocks of
// one row; M * 192: the [block][row] order of the small-M kernels); x_out /
// norm_out: this row's outputs of the residual norm. Columns past the
// matrix are built as zeros (their weights are zero padding, and a zero X
// keeps the block's offset term zero).
template <int DT>
__device__ __forceinline__ float4 frag_group_build(const TileMatvecArgs &a, uint32_t grp, uint32_t lane,
                                                   const GroupIn &in, float inv, bool keep, int8_t *frag,
                                                   uint32_t bstride, float *x_out, float *norm_out,
                                                   uint32_t xm) {
    const uint32_t g = lane >> 4, m = lane & 15;
    const bool in_matrix = (4 * grp + g) * CTOX_BLOCK_LEN + 4 * m < a.blocks * CTOX_BLOCK_LEN;
    float xa[4], yb[4], wv[4], v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        xa[i] = __int_as_float(in.a[i]);
        yb[i] = __int_as_float(in.b[i]);
        wv[i] = __int_as_float(in.w[i]);
    }
    // One uniform branch per transform, each straight-line over the lane's
    // four columns.
    if (xm == 1) {
        const uint32_t col = (4 * grp + g) * CTOX_BLOCK_LEN + 4 * m;
        const bool inside = col < a.blocks * CTOX_BLOCK_LEN;
        float h[4];
#pragma unroll
        for (int i = 0; i < 4; i++) h[i] = xa[i] + yb[i];
        if (keep && inside && x_out) *(float4 *)(x_out + col) = make_float4(h[0], h[1], h[2], h[3]);
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = h[i] * inv * (1.0f + wv[i]);
        if (keep && inside && norm_out) *(float4 *)(norm_out + col) = make_float4(v[0], v[1], v[2], v[3]);
    } else if (xm == 2) {
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = tl_silu(xa[i]) * yb[i];
    } else if (xm == 3) {
        // Per-head mean of squares: a head of head_dim columns is head_dim / 4
        // consecutive lanes (head_dim 64, 128 or 256).
        float ss = (xa[0] * xa[0] + xa[1] * xa[1]) + (xa[2] * xa[2] + xa[3] * xa[3]);
        ss = row16_reduce(ss, [](float x, float y) { return x + y; });
        if (a.head_dim >= 128) ss += __shfl_xor(ss, 16);
        if (a.head_dim >= 256) ss += __shfl_xor(ss, 32);
        const float hinv = 1.0f / sqrtf(ss / (float)a.head_dim + a.eps);
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = xa[i] * hinv * wv[i] * tl_silu(yb[i]);
    } else if (xm == 4) {
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = xa[i] * (1.0f / (1.0f + expf(-yb[i])));
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = xa[i];
    }
    if (a.s_in_kind == CTOX_KSCALE_F16) {
        v[0] *= half_bits_to_float((uint32_t)in.s[0] & 0xffffu);
        v[1] *= half_bits_to_float((uint32_t)in.s[0] >> 16);
        v[2] *= half_bits_to_float((uint32_t)in.s[1] & 0xffffu);
        v[3] *= half_bits_to_float((uint32_t)in.s[1] >> 16);
    } else if (a.s_in_kind == CTOX_KSCALE_F32) {
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] *= __int_as_float(in.s[i]);
    }
    if (!in_matrix) v[0] = v[1] = v[2] = v[3] = 0.0f;
    // A non-finite value anywhere in the block makes its quantum NaN (the
    // lane sum of a finite row can only overflow for |x'| near 2^128).
    const bool bad = !__builtin_isfinite((v[0] + v[1]) + (v[2] + v[3]));
    // Non-negative floats order like their bit patterns: integer max.
    uint32_t mb = max(max(__float_as_uint(fabsf(v[0])), __float_as_uint(fabsf(v[1]))),
                      max(__float_as_uint(fabsf(v[2])), __float_as_uint(fabsf(v[3]))));
    mb = row16_reduce(mb, [](uint32_t x, uint32_t y) { return max(x, y); });
    const float mx = __uint_as_float(mb);
    const int badi = row16_reduce((int)bad, [](int x, int y) { return x | y; });
    int ex = 0;
    if (mx > 0.0f) frexpf(mx, &ex);
    // X = rint(v * 2^(22 - e)): one fma against 1.5 * 2^23 rounds to the
    // nearest integer (ties to even) in the low mantissa bits (|X| <= 2^22).
    const bool live = mx > 0.0f && !badi;
    const float p2 = live ? ldexpf(1.0f, CTOX_XFRAC_BITS - ex) : 0.0f;
    int X[4];
    int sx = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        X[i] = __float_as_int(fmaf(v[i], p2, 12582912.0f)) - 0x4b400000;
        sx += X[i];
    }
    sx = row16_reduce(sx, [](int x, int y) { return x + y; });
    const float q = badi ? __builtin_nanf("") : (mx > 0.0f ? ldexpf(1.0f, ex - CTOX_XFRAC_BITS) : 0.0f);
    const long long off = DT ? 15 : 3;
    // Balanced limbs X = X0 + 256 X1 + 65536 X2 (X0, X1 in [-128, 127]):
    // X0 is byte 0 of X, X1 byte 1 of X + 0x80, X2 byte 2 of X + 0x8080.
    // Element 4m + i of block g goes to quarter m / 4, element 4 (m % 4) + i.
    int8_t *blkp = frag + g * bstride + (m >> 2) * 16;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int pos = frag_pos(DT, (int)(4 * (m & 3) + i));
        blkp[0 * 64 + pos] = (int8_t)X[i];
        blkp[1 * 64 + pos] = (int8_t)((X[i] + 0x80) >> 8);
        blkp[2 * 64 + pos] = (int8_t)((X[i] + 0x8080) >> 16);
    }
    return make_float4(2.0f * q, 512.0f * q, 131072.0f * q, (float)(-off * (long long)sx) * q);
}


// Cross-chunk combine. Partials are 64-bit slots (f32 bits | the launch's
// sequence number << 32) written with single agent-scope atomic stores
// (coherent across the XCDs' L2s without cache maintenance). In a launch
// the device holds at once (the host checks the occupancy), the last
// chunk's waves combine: the other chunks store and leave, and the
// combining lane polls its row's slots until every tag is this launch's,
// then adds them in chunk order. A larger launch combines by arrival
// (tile_matvec). Either way a combining wave waits only for producers that
// are resident, so the polls end; a poll count past CTOX_COMBINE_POLLS (only
// a broken invariant) yields NaN, which the engine reports, not a hang.
#define CTOX_COMBINE_POLLS (1u << 16)
__device__ __forceinline__ void combine_store(uint64_t *slot, float v, uint32_t seq) {
    __hip_atomic_store(slot, (uint64_t)__float_as_uint(v) | ((uint64_t)seq << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Row sums of T slot sets at once (the small-M kernels' token groups):
// set i adds, in chunk order over chunks k < n, slots[i][k * stride] and,
// for chunk own_k, own[i] in place of a slot (that slot is never read: with
// the last chunk combining it does not exist). A set with want[i] false is
// done at once with 0. All sets' loads of a round go out together, so T
// sets cost one round trip, not T.
template <int T>
__device__ __forceinline__ void combine_poll_n(const uint64_t *const (&slots)[T], size_t stride, uint32_t n,
                                               uint32_t own_k, uint32_t seq, const float (&own)[T],
                                               const bool (&want)[T], float (&sum)[T]) {
    constexpr int CB = 16 / T;  // slots per set and round: 16 loads in flight
    const uint32_t ns = n - 1;  // slots to read: chunks other than own_k
    bool done[T];
    bool pending = false;
#pragma unroll
    for (int t = 0; t < T; t++) {
        sum[t] = 0.0f;
        done[t] = !want[t];
        pending = pending || want[t];
    }
    for (uint32_t poll = 0; __builtin_amdgcn_ballot_w64(pending) != 0; poll++) {
        if (poll >= CTOX_COMBINE_POLLS) {
#pragma unroll
            for (int t = 0; t < T; t++)
                if (!done[t]) sum[t] = __builtin_nanf("");
            break;
        }
        if (poll) __builtin_amdgcn_s_sleep(1);
        float acc[T];
        bool all[T];
#pragma unroll
        for (int t = 0; t < T; t++) {
            acc[t] = 0.0f;
            all[t] = true;
        }
        for (uint32_t i0 = 0; i0 < ns; i0 += CB) {
            uint64_t pv[T][CB];
#pragma unroll
            for (int t = 0; t < T; t++)
#pragma unroll
                for (int i = 0; i < CB; i++) {
                    const uint32_t k = min(i0 + i, ns - 1);
                    pv[t][i] = __hip_atomic_load(&slots[t][(size_t)(k < own_k ? k : k + 1) * stride], __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
                }
#pragma unroll
            for (int t = 0; t < T; t++)
#pragma unroll
                for (int i = 0; i < CB; i++)
                    if (i0 + i < ns) {
                        if (i0 + i == own_k) acc[t] += own[t];  // own chunk comes before chunk own_k + 1
                        all[t] = all[t] && (uint32_t)(pv[t][i] >> 32) == seq;
                        acc[t] += __uint_as_float((uint32_t)pv[t][i]);
                    }
        }
        pending = false;
#pragma unroll
        for (int t = 0; t < T; t++) {
            if (own_k == ns) acc[t] += own[t];  // own chunk is the last
            if (!done[t] && all[t]) {
                sum[t] = acc[t];
                done[t] = true;
            }
            pending = pending || !done[t];
        }
    }
}

// Producer side of the residual sums: per 16-row tile, sum of (res_h + y)^2
// over its rows (the 16 lanes of one row group, DPP within the row).
__device__ __forceinline__ void residual_tile_sum(const TileMatvecArgs &a, uint32_t tile, uint32_t row, bool mine,
                                                  float y, uint32_t j, const EpiIn &e) {
    if (!a.res_sq) return;
    const float h = mine && row < a.rows ? __uint_as_float(e.h) + y : 0.0f;
    const float s = row16_reduce(h * h, [](float x, float z) { return x + z; });
    if (mine && j == 0) a.res_sq[tile] = s;
}

template <int DT, int U, int AB, int ARR, int XM = -1>
__device__ __forceinline__ void tile_matvec(const TileMatvecArgs &a) {
    using C = TlCfg<DT>;
    // XM >= 0: the input transform fixed at compile time, so each kernel
    // holds only its own transform's registers; XM = 5 is the residual norm
    // (xmode 1) with the producer's sums of squares (sq_n > 0).
    constexpr bool SQ = XM == 5;
    const uint32_t xmode = SQ ? 1u : (XM >= 0 ? (uint32_t)XM : a.xmode);
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t v = __builtin_amdgcn_readfirstlane(blockIdx.x * 4u + (threadIdx.x >> 6));
    const uint32_t c = v / a.segs, s = v - c * a.segs;
    const uint32_t t0 = s * U;
    // With AB the host makes segs a multiple of the workgroup's wave count,
    // so c is uniform over the workgroup and every wave of it reaches the
    // barrier of the shared fragment build (waves without tiles leave after).
    if (c >= a.chunks || (!AB && t0 >= a.tiles)) return;
    const uint32_t n = t0 < a.tiles ? min((uint32_t)U, a.tiles - t0) : 0u;
    const uint8_t *base = a.weights + ((size_t)c * a.tiles + min(t0, a.tiles - 1)) * C::UB;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)(n * C::UB), 0x00020000);
    const __amdgpu_buffer_rsrc_t fr = __builtin_amdgcn_make_buffer_rsrc((void *)a.xa, (short)0, (int)(a.blocks * 192), 0x00020000);
    const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc((void *)a.xc, (short)0, (int)(a.blocks * 16), 0x00020000);
    const uint32_t g = lane >> 4, j = lane & 15, limb = j & 3;
    const bool aok = (j >> 2) == g && limb < 3;

    // Activation fragments of the chunk: A lane (g, j) of quarter q carries
    // limb j % 4 of block 4G + g when j / 4 == g (zero elsewhere).
    v4i af[4][4];
    float4 kq[4];
    if (!AB) {
#pragma unroll
        for (int G = 0; G < 4; G++) {
            const uint32_t blk = c * CTOX_TILE_BLOCKS + 4 * G + g;
#pragma unroll
            for (int q = 0; q < 4; q++)
                af[G][q] = __builtin_amdgcn_raw_buffer_load_b128(fr, aok ? blk * 192 + limb * 64 + q * 16 : 0x7ffffff0u, 0, 0);
            const v4i k4 = __builtin_amdgcn_raw_buffer_load_b128(cr, blk * 16, 0, 0);
            kq[G] = make_float4(__int_as_float(k4[0]), __int_as_float(k4[1]), __int_as_float(k4[2]), __int_as_float(k4[3]));
        }
    }
    // AB: wave w of the workgroup builds group w of the chunk. The residual
    // norm first needs the whole row's sum of squares: every workgroup
    // reduces it (the row is at most 8192 floats and L2-resident) in the same
    // thread order, so all workgroups agree on it.
    const uint32_t wg_wave = threadIdx.x >> 6;
    GroupIn gin;
    v4i hx[8], hd[8];
    float sqv[2] = {0.0f, 0.0f};
    if (AB && xmode == 1 && (SQ || a.sq_n)) {
        // The producer's per-tile sums of squares (at most 512).
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const uint32_t t = threadIdx.x + 256 * k;
            sqv[k] = t < a.sq_n ? a.sq_in[t] : 0.0f;
        }
    } else if (AB && xmode == 1 && !SQ) {
        const uint32_t cols = a.blocks * CTOX_BLOCK_LEN;
        const __amdgpu_buffer_rsrc_t xr = f32_rsrc(a.input, cols), dr = f32_rsrc(a.delta, cols);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            hx[k] = __builtin_amdgcn_raw_buffer_load_b128(xr, (threadIdx.x + 256 * k) * 16, 0, 0);
            hd[k] = __builtin_amdgcn_raw_buffer_load_b128(dr, (threadIdx.x + 256 * k) * 16, 0, 0);
        }
    }
    if (AB) frag_group_loads(a, c * 4 + wg_wave, lane, gin, xmode);
    __builtin_amdgcn_sched_barrier(0);  // activation loads stay ahead of the weight loads
    TileUnit<DT> u[U];
#pragma unroll
    for (int k = 0; k < U; k++) {
#pragma unroll
        for (int i = 0; i < (int)C::LPU; i++)
            u[k].w[i] = __builtin_amdgcn_raw_buffer_load_b128(wr, lane * 16, k * C::UB + i * 1024, CTOX_LOAD_NT);
        u[k].s = __builtin_amdgcn_raw_buffer_load_b64(wr, C::CB + lane * 8, k * C::UB, CTOX_LOAD_NT);
    }
    // AB: the chunk's fragments and constants stay in LDS and are read per
    // group where they are used, which leaves the wave's registers to the
    // weight loads in flight (more waves per CU).
    __shared__ __align__(16) int8_t xs[CTOX_TILE_BLOCKS * 192];
    __shared__ float4 kqs[CTOX_TILE_BLOCKS];
    if (AB) {
        __shared__ float wss[4];
        float inv = 0.0f;
        if (xmode == 1) {
            float ss = 0.0f;
            if (SQ || a.sq_n) {
                ss = sqv[0] + sqv[1];
            } else {
#pragma unroll
                for (int k = 0; k < 8; k++) {
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float h = __int_as_float(hx[k][i]) + __int_as_float(hd[k][i]);
                        ss = fmaf(h, h, ss);
                    }
                }
            }
            ss = row16_reduce(ss, [](float x, float y) { return x + y; });
            ss += __shfl_xor(ss, 16);
            ss += __shfl_xor(ss, 32);
            if (lane == 0) wss[wg_wave] = ss;
            lds_barrier();
            inv = 1.0f / sqrtf(((wss[0] + wss[1]) + (wss[2] + wss[3])) / (float)(a.blocks * CTOX_BLOCK_LEN) + a.eps);
        }
        const bool keep = ((blockIdx.x * 4u) % a.segs) == 0;  // segment 0 of the chunk
        const float4 k = frag_group_build<DT>(a, c * 4 + wg_wave, lane, gin, inv, keep, xs + wg_wave * 768, 192,
                                              a.x_out, a.norm_out, xmode);
        if (j == 0) kqs[4 * wg_wave + g] = k;
        lds_barrier();  // orders LDS only: the weight loads stay in flight
        if (t0 >= a.tiles) return;
    }

    // Every unit is computed (a unit past the wave's tiles reads zeros): a
    // branch here would let the compiler sink its loads behind it. Per unit
    // the groups are added in order G = 0..3.
    float part[U];
#pragma unroll
    for (int k = 0; k < U; k++) part[k] = 0.0f;
#pragma unroll
    for (int G = 0; G < 4; G++) {
        v4i fg[4];
        float4 kg;
        if (AB) {
            kg = kqs[4 * G + g];
#pragma unroll
            for (int q = 0; q < 4; q++)
                fg[q] = aok ? *(const v4i *)(xs + G * 768 + g * 192 + limb * 64 + q * 16) : (v4i){0, 0, 0, 0};
        } else {
            kg = kq[G];
#pragma unroll
            for (int q = 0; q < 4; q++) fg[q] = af[G][q];
        }
#pragma unroll
        for (int k = 0; k < U; k++) {
            v4i cc = (v4i){0, 0, 0, 0};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                uint32_t w0, w1 = 0;
                if (DT) {
                    const v4i W = u[k].w[2 * G + (q >> 1)];
                    w0 = (uint32_t)W[2 * (q & 1)];
                    w1 = (uint32_t)W[2 * (q & 1) + 1];
                } else {
                    w0 = (uint32_t)u[k].w[G][q];
                }
                cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(fg[q], unpack_quarter<DT>(w0, w1), cc, 0, 0, 0);
            }
            const uint32_t sw = u[k].s[G >> 1];
            const float scale = half_bits_to_float((G & 1) ? (sw >> 16) : (sw & 0xffffu));
            // sum(c X) = C0 + 256 C1 + 65536 C2 is exact in int32 for Q2 and
            // for staged Q4 fragments (21 fraction bits): one conversion.
            // Q4 fragments built here (22 bits) combine the limbs in float.
            float f;
            if (DT && AB) {
                f = fmaf((float)cc[0], kg.x, kg.w);
                f = fmaf((float)cc[1], kg.y, f);
                f = fmaf((float)cc[2], kg.z, f);
            } else {
                f = fmaf((float)(cc[0] + (cc[1] << 8) + (cc[2] << 16)), kg.x, kg.w);
            }
            part[k] = fmaf(f, scale, part[k]);
        }
    }
#pragma unroll
    for (int k = 0; k < U; k++) {
        part[k] += __shfl_xor(part[k], 16);
        part[k] += __shfl_xor(part[k], 32);
    }
    // Lane (g, j) reports row j of the wave's tile g.
    float val = part[0];
#pragma unroll
    for (int k = 1; k < U; k++)
        if (g == (uint32_t)k) val = part[k];
    const uint32_t tile = t0 + g, row = tile * CTOX_TILE_ROWS + j;
    const bool mine = g < n;
    const size_t cstride = (size_t)a.tiles * CTOX_TILE_ROWS;
    const bool combine = a.chunks > 1 && !a.parts_out;
    if (combine && !ARR && c + 1 < a.chunks) {
        if (mine) combine_store(&a.partial[(size_t)c * cstride + row], val, a.seq);
        return;
    }
    // This wave may write rows: its epilogue operands go out now.
    const EpiIn e = epi_load(a, row, 0);
    if (a.parts_out && a.chunks > 1) {
        // Chunk partials for a consumer that adds them (no combine here).
        if (mine && row < a.rows) a.output[(size_t)c * a.out_stride + row] = epi_apply(val / C::DEN, e, a);
        return;
    }
    float sum = val;
    if (combine) {
        bool want = mine;
        if (ARR) {
            // Arrival combine: every chunk stores its tagged partial, then
            // counts itself in for the tile; the chunk that arrives last adds
            // the tile's partials in chunk order and resets the count. It
            // waits only for stores of waves that have already arrived
            // (issued before their count), so no wave waits on one not yet
            // dispatched.
            if (mine) combine_store(&a.partial[(size_t)c * cstride + row], val, a.seq);
            uint32_t old = 0;
            if (mine && j == 0)
                old = __hip_atomic_fetch_add(&a.arrive[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            old = __shfl(old, 16 * g);
            want = mine && old + 1 == a.chunks;
            if (__builtin_amdgcn_ballot_w64(want) == 0) return;
        }
        const uint64_t *const slots[1] = {&a.partial[want ? row : j]};  // in range for every lane
        const float own[1] = {val};
        const bool w1[1] = {want};
        float got[1];
        combine_poll_n<1>(slots, cstride, a.chunks, c, a.seq, own, w1, got);
        sum = got[0];
        if (ARR && want && j == 0) __hip_atomic_store(&a.arrive[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (ARR && !want) return;
    }
    const float y = mine && row < a.rows ? epi_apply(sum / C::DEN, e, a) : 0.0f;
    if (mine && row < a.rows) a.output[row] = y;
    residual_tile_sum(a, tile, row, mine, y, j, e);
}

// ctox_q{2,4}_mv_tile{U}_gfx950 take prep-staged fragments (the _x{T}
// kernels below build them from the input). The _arrive variants combine by
// arrival (launches larger than the device holds at once).
#define CTOX_TILE_KERNEL(name, dt, u, ab) \
    extern "C" __global__ __launch_bounds__(256) void name(TileMatvecArgs a) { tile_matvec<dt, u, ab, 0>(a); } \
    extern "C" __global__ __launch_bounds__(256) void name##_arrive(TileMatvecArgs a) { tile_matvec<dt, u, ab, 1>(a); }
CTOX_TILE_KERNEL(ctox_q2_mv_tile1_gfx950, 0, 1, 0)
CTOX_TILE_KERNEL(ctox_q2_mv_tile2_gfx950, 0, 2, 0)
CTOX_TILE_KERNEL(ctox_q2_mv_tile3_gfx950, 0, 3, 0)
CTOX_TILE_KERNEL(ctox_q2_mv_tile4_gfx950, 0, 4, 0)
CTOX_TILE_KERNEL(ctox_q4_mv_tile1_gfx950, 1, 1, 0)
CTOX_TILE_KERNEL(ctox_q4_mv_tile2_gfx950, 1, 2, 0)
CTOX_TILE_KERNEL(ctox_q4_mv_tile3_gfx950, 1, 3, 0)
CTOX_TILE_KERNEL(ctox_q4_mv_tile4_gfx950, 1, 4, 0)
// ctox_q{2,4}_mv_tile{U}x{T}_gfx950: the in-kernel build with the input
// transform fixed at compile time, T = xmode 0..4 (x0: the crate's fused
// matvec on a plain input) or 5 (the residual norm with the producer's sums
// of squares).
#define CTOX_TILE_XM_KERNEL(name, dt, u, xm) \
    extern "C" __global__ __launch_bounds__(256) void name(TileMatvecArgs a) { tile_matvec<dt, u, 1, 0, xm>(a); } \
    extern "C" __global__ __launch_bounds__(256) void name##_arrive(TileMatvecArgs a) { tile_matvec<dt, u, 1, 1, xm>(a); }
#define CTOX_TILE_XM_KERNELS(xm) \
    CTOX_TILE_XM_KERNEL(ctox_q2_mv_tile1x##xm##_gfx950, 0, 1, xm) \
    CTOX_TILE_XM_KERNEL(ctox_q2_mv_tile2x##xm##_gfx950, 0, 2, xm) \
    CTOX_TILE_XM_KERNEL(ctox_q2_mv_tile3x##xm##_gfx950, 0, 3, xm) \
    CTOX_TILE_XM_KERNEL(ctox_q2_mv_tile4x##xm##_gfx950, 0, 4, xm) \
    CTOX_TILE_XM_KERNEL(ctox_q4_mv_tile1x##xm##_gfx950, 1, 1, xm) \
    CTOX_TILE_XM_KERNEL(ctox_q4_mv_tile2x##xm##_gfx950, 1, 2, xm) \
    CTOX_TILE_XM_KERNEL(ctox_q4_mv_tile3x##xm##_gfx950, 1, 3, xm) \
    CTOX_TILE_XM_KERNEL(ctox_q4_mv_tile4x##xm##_gfx950, 1, 4, xm)
CTOX_TILE_XM_KERNELS(0)
CTOX_TILE_XM_KERNELS(1)
CTOX_TILE_XM_KERNELS(2)
CTOX_TILE_XM_KERNELS(3)
CTOX_TILE_XM_KERNELS(4)
CTOX_TILE_XM_KERNELS(5)



// ---------------------------------------------------------------------------
// Small-M (2..8 activation rows) tiled matvec: the MTP verify projections.
// Same waves, chunks and last-arrival combine as the batch-1 kernel, with
// token-stacked MFMAs: A rows 4t + l carry token t's limb l of one block (the
// prep kernels' xa rows, loaded into registers once per wave), B lane (g, j)
// carries quarter g of that block for row j, and C lane (g, j) accumulates
// (token 4 tg + g, row j). The tiled units give lane (g, j) all four
// quarters of block 4G + g; two permlane swap stages transpose each group's
// 4 x 4 (lane row x dword) layout into quarter g of blocks 4G .. 4G + 3.
// A wave covers all 16 blocks of its chunk for every token, so no
// cross-lane reduction is needed before the combine.
__device__ __forceinline__ void transpose4(uint32_t &r0, uint32_t &r1, uint32_t &r2, uint32_t &r3) {
    auto s02 = __builtin_amdgcn_permlane32_swap(r0, r2, false, false);
    auto s13 = __builtin_amdgcn_permlane32_swap(r1, r3, false, false);
    auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
    auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
    r0 = s01[0];
    r1 = s01[1];
    r2 = s23[0];
    r3 = s23[1];
}

// Per 16-row tile and row tok: sum over the tile's rows of (res_h + y)^2.
__device__ __forceinline__ void residual_tile_sum_m(const TileMatvecArgs &a, uint32_t tok, uint32_t tile,
                                                    uint32_t row, bool mine, float y, uint32_t j, const EpiIn &e) {
    const float h = mine && row < a.rows ? __uint_as_float(e.h) + y : 0.0f;
    const float s = row16_reduce(h * h, [](float x, float z) { return x + z; });
    if (mine && j == 0) a.res_sq[(size_t)tok * a.tiles + tile] = s;
}

// Consumer side of the next-norm staging (a.rms_sq: per-block sums of h^2
// of the staged rows, which were staged without their 1 / rms): per token
// row t < M, 1 / sqrt(sum / (blocks * 64) + eps) into inv[t]. Thread
// (t, i) = (tid / 32, tid % 32) adds entries i, i + 32, i + 64, i + 96 of
// row t; its loads go out with the prologue's and are added after `wait`.
struct RmsIn {
    float v[4];
};
__device__ __forceinline__ RmsIn rms_loads(const TileMatvecArgs &a, uint32_t M) {
    RmsIn r;
    const uint32_t t = threadIdx.x >> 5, i = threadIdx.x & 31;
    const __amdgpu_buffer_rsrc_t rs = f32_rsrc(a.rms_sq, a.rms_sq ? M * a.rms_n : 0u);
#pragma unroll
    for (int k = 0; k < 4; k++)
        r.v[k] = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(
            rs, (t < M && i + 32 * k < a.rms_n ? t * a.rms_n + i + 32 * k : 0x1fffffffu) * 4, 0, 0));
    return r;
}
__device__ __forceinline__ void rms_finish(const TileMatvecArgs &a, const RmsIn &r, float *inv) {
    float s = (r.v[0] + r.v[1]) + (r.v[2] + r.v[3]);
    s = row16_reduce(s, [](float x, float y) { return x + y; });
    s += __shfl_xor(s, 16);
    if ((threadIdx.x & 31) == 0 && (threadIdx.x >> 5) < 8)
        inv[threadIdx.x >> 5] = 1.0f / sqrtf(s / (float)(a.blocks * CTOX_BLOCK_LEN) + a.eps);
}

// Producer side of the next-norm staging (a.nx_xa): the workgroup's four
// waves hold row tiles 4 b .. 4 b + 3 of the output, i.e. 64-column block b
// of the next projection's input. Lane (g, j) has h = res_h + out of token
// rows 4 tg + g at row j of its tile; the block's values h * (1 + w) * s_in
// meet in LDS and wave w stages token rows w, w + 4 (stage_block, the prep
// kernel's arithmetic), with the block's sum of h^2 per token.
template <int TG>
__device__ __forceinline__ void stage_next_norm(const TileMatvecArgs &a, uint32_t tile, uint32_t g, uint32_t j,
                                                uint32_t M, const float (&hv)[TG], const bool (&want)[TG], float wn,
                                                float sc, uint32_t tlo, uint32_t thi) {
    __shared__ float nxv[8 * 64];
    __shared__ float nss[8 * 4];
    const uint32_t w = tile & 3, lane = threadIdx.x & 63, b = tile >> 2;
    const uint32_t row = tile * CTOX_TILE_ROWS + j;
#pragma unroll
    for (int tg = 0; tg < TG; tg++) {
        const uint32_t tok = 4 * tg + g;
        if (want[tg]) {
            a.nx_h[(size_t)tok * a.rows + row] = hv[tg];
            nxv[tok * 64 + 16 * w + j] = hv[tg] * (1.0f + wn) * sc;
        }
        const float ss = row16_reduce(hv[tg] * hv[tg], [](float x, float y) { return x + y; });
        if (j == 0 && tok < M) nss[tok * 4 + w] = ss;
    }
    lds_barrier();
    const uint32_t nb = a.rows / CTOX_BLOCK_LEN;
    // rows [tlo, thi): the ones this workgroup combined
    for (uint32_t tok = tlo + w; tok < thi; tok += 4) {
        stage_block(nxv[tok * 64 + lane], a.nx_xa + ((size_t)b * M + tok) * 192, (float4 *)a.nx_xc + (size_t)b * M + tok,
                    a.nx_dtype, lane);
        if (lane == 0)
            a.nx_sq[(size_t)tok * nb + b] = (nss[tok * 4 + 0] + nss[tok * 4 + 1]) + (nss[tok * 4 + 2] + nss[tok * 4 + 3]);
    }
}

// MR = M, the row count, is a compile-time constant: every LDS address of
// the MFMA loop is a per-lane base plus an immediate offset.
// Tail of the small-M kernels: lane (g, j) of unit k and token group tg
// holds (token 4 tg + g, row j) of the wave's tiles t0 .. t0 + n - 1 for
// chunk c. Partials [chunk][token][tiles * 16] meet as in the batch-1
// kernel: by the last chunk's waves when the launch is resident at once
// (ARR = 0), else by the chunk that arrives last at the tile's count.
// MM: the row count when the caller knows it at compile time (0 otherwise).
// At five rows with the last chunk combining (P5S), the fifth row is
// combined by the waves of chunk chunks - 2 (same tiles, another
// workgroup), so each combining wave polls one slot set in one round trip
// and stages a fifth of the next norm's rows fewer: the last chunk also
// stores its fifth-row partial, the partial buffer holding every chunk.
template <int DT, int U, int TG, int ARR, int MM = 0>
__device__ __forceinline__ void small_m_finish(const TileMatvecArgs &a, uint32_t c, uint32_t t0, uint32_t n,
                                               uint32_t g, uint32_t j, uint32_t M, const float (&acc)[U][TG],
                                               const float (&inv)[TG]) {
    using C = TlCfg<DT>;
    const size_t tstride = (size_t)a.tiles * CTOX_TILE_ROWS, cstride = tstride * M;
    if (a.parts_out) {
        // Chunk partials [chunk][token][out_stride] for a consumer that adds
        // them (no combine here).
#pragma unroll
        for (int k = 0; k < U; k++)
#pragma unroll
            for (int tg = 0; tg < TG; tg++) {
                const uint32_t tok = 4 * tg + g, row = (t0 + k) * CTOX_TILE_ROWS + j;
                const EpiIn e = epi_load(a, row, 0);
                if ((uint32_t)k < n && tok < M && row < a.rows)
                    a.output[((size_t)c * M + tok) * a.out_stride + row] = epi_apply(acc[k][tg] * inv[tg] / C::DEN, e, a);
            }
        return;
    }
    constexpr bool P5S = MM == 5 && !ARR;
    // (worth it where the combine stages the next norm or polls more than
    // one round: more than 9 chunks)
    const bool split = P5S && a.chunks > 1 && (a.nx_xa != nullptr || a.chunks > 9);
    // split: this chunk's part in the fifth-row combine (role 1: chunk
    // chunks - 2 combines row 4, role 2: the last chunk rows 0..3).
    const uint32_t role = !split ? 0u : (c + 1 == a.chunks ? 2u : (c + 2 == a.chunks ? 1u : 0u));
    if (a.chunks > 1 && !ARR && (c + 1 < a.chunks || split)) {
#pragma unroll
        for (int k = 0; k < U; k++)
#pragma unroll
            for (int tg = 0; tg < TG; tg++) {
                const uint32_t tok = 4 * tg + g, row = (t0 + k) * CTOX_TILE_ROWS + j;
                // role 1 keeps row 4, role 2 rows 0..3: their slots are the other's
                const bool keep = (role == 1 && tok == 4) || (role == 2 && tok < 4);
                if ((uint32_t)k < n && tok < M && !keep)
                    combine_store(&a.partial[c * cstride + tok * tstride + row], acc[k][tg], a.seq);
            }
        if (!split || role == 0) return;
    }
    // This wave may write rows: its epilogue operands go out now.
    EpiIn e[U][TG];
#pragma unroll
    for (int k = 0; k < U; k++)
#pragma unroll
        for (int tg = 0; tg < TG; tg++) e[k][tg] = epi_load(a, (t0 + k) * CTOX_TILE_ROWS + j, min(4 * tg + g, M - 1));
    // Next-norm staging operands of the wave's rows, read ahead of the combine.
    const uint32_t nrow = t0 * CTOX_TILE_ROWS + j;
    const uint32_t nwb = __builtin_amdgcn_raw_buffer_load_b32(f32_rsrc(a.nx_xa ? a.nx_w : nullptr, a.rows), nrow * 4, 0, 0);
    const uint32_t nsb = __builtin_amdgcn_raw_buffer_load_b16(
        __builtin_amdgcn_make_buffer_rsrc((void *)a.nx_s_in, (short)0, a.nx_xa && a.nx_s_in ? (int)(a.rows * 2) : 0,
                                          0x00020000),
        nrow * 2, 0, 0);
    bool last[U];
#pragma unroll
    for (int k = 0; k < U; k++) last[k] = true;
    if (a.chunks > 1 && ARR) {
#pragma unroll
        for (int k = 0; k < U; k++)
#pragma unroll
            for (int tg = 0; tg < TG; tg++) {
                const uint32_t tok = 4 * tg + g, row = (t0 + k) * CTOX_TILE_ROWS + j;
                if ((uint32_t)k < n && tok < M) combine_store(&a.partial[c * cstride + tok * tstride + row], acc[k][tg], a.seq);
            }
        bool any = false;
#pragma unroll
        for (int k = 0; k < U; k++) {
            uint32_t old = 0;
            if ((threadIdx.x & 63) == 0 && (uint32_t)k < n)
                old = __hip_atomic_fetch_add(&a.arrive[t0 + k], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            old = __builtin_amdgcn_readfirstlane(old);
            last[k] = (uint32_t)k < n && old + 1 == a.chunks;
            any = any || last[k];
        }
        if (!any) return;
    }
#pragma unroll
    for (int k = 0; k < U; k++) {
        if (!last[k]) continue;  // wave-uniform
        const uint32_t tile = t0 + k, row = tile * CTOX_TILE_ROWS + j;
        float sum[TG];
        bool want[TG];
#pragma unroll
        for (int tg = 0; tg < TG; tg++) {
            const uint32_t tok = 4 * tg + g;
            want[tg] = (uint32_t)k < n && tok < M && (role == 0 || (role == 1) == (tok == 4));
            sum[tg] = acc[k][tg];
        }
        if (split) {
            // One slot set: rows 0..3 (role 2) or row 4 (role 1), all chunks
            // but this one in one round.
            const uint32_t tg1 = role == 1 ? TG - 1 : 0u;
            const uint32_t tok = 4 * tg1 + g;
            const uint64_t *const sl[1] = {&a.partial[want[tg1] ? (size_t)tok * tstride + row : j]};
            const float own[1] = {acc[k][tg1]};
            const bool w1[1] = {want[tg1]};
            float got[1];
            combine_poll_n<1>(sl, cstride, a.chunks, c, a.seq, own, w1, got);
            sum[tg1] = got[0];
        } else if (a.chunks > 1) {
            // Every token group's slots in one poll.
            const uint64_t *slots[TG];
#pragma unroll
            for (int tg = 0; tg < TG; tg++) slots[tg] = &a.partial[want[tg] ? (size_t)(4 * tg + g) * tstride + row : j];
            combine_poll_n<TG>(slots, cstride, a.chunks, c, a.seq, acc[k], want, sum);
        }
        float hv[TG];
#pragma unroll
        for (int tg = 0; tg < TG; tg++) {
            const uint32_t tok = 4 * tg + g;
            const float y = want[tg] && row < a.rows ? epi_apply(sum[tg] * inv[tg] / C::DEN, e[k][tg], a) : 0.0f;
            if (want[tg] && row < a.rows) a.output[(size_t)tok * a.out_stride + row] = y;
            if (a.res_sq) residual_tile_sum_m(a, min(tok, M - 1), tile, row, want[tg], y, j, e[k][tg]);
            hv[tg] = want[tg] && row < a.rows ? __uint_as_float(e[k][tg].h) + y : 0.0f;
        }
        if (!ARR && U == 1 && a.nx_xa)
            stage_next_norm<TG>(a, tile, g, j, M, hv, want, __uint_as_float(nwb),
                                a.nx_s_in ? half_bits_to_float(nsb & 0xffffu) : 1.0f, role == 1 ? 4u : 0u,
                                role == 2 ? 4u : M);
        if (ARR && a.chunks > 1 && (threadIdx.x & 63) == 0)
            __hip_atomic_store(&a.arrive[t0 + k], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// MM = a.batch, the row count: the LDS areas hold exactly MM rows (more
// workgroups per CU).
template <int DT, int U, int MM, int ARR>
__device__ __forceinline__ void tile_matvec_m(const TileMatvecArgs &a) {
    using C = TlCfg<DT>;
    constexpr uint32_t MAXM = MM, TG = (MM + 3) / 4;
    // The chunk's staged activation rows (xa order: [block][token][192]) and
    // epilogue constants, shared by the workgroup's four waves (same chunk).
    __shared__ __align__(16) int8_t xas[CTOX_TILE_BLOCKS * MAXM * 192];
    __shared__ float4 kqs[CTOX_TILE_BLOCKS * MAXM];
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t v = __builtin_amdgcn_readfirstlane(blockIdx.x * 4u + (threadIdx.x >> 6));
    const uint32_t c = v / a.segs, s = v - c * a.segs;
    const uint32_t t0 = s * U;
    constexpr uint32_t M = MM;  // == a.batch: every LDS offset of the MFMA loop is an immediate
    if (c >= a.chunks) return;  // uniform over the workgroup (segs is a multiple of 4)
    const uint32_t n = t0 < a.tiles ? min((uint32_t)U, a.tiles - t0) : 0u;
    const uint8_t *base = a.weights + ((size_t)c * a.tiles + min(t0, a.tiles - 1)) * C::UB;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)(n * C::UB), 0x00020000);
    const uint32_t g = lane >> 4, j = lane & 15, limb = j & 3;

    // Workgroup copy of the chunk's xa rows (contiguous: 16 blocks x M x 192
    // bytes) and xc constants, issued before the weight loads, branch-free.
    const uint32_t xbytes = min(CTOX_TILE_BLOCKS, a.blocks - c * CTOX_TILE_BLOCKS) * M * 192;
    const __amdgpu_buffer_rsrc_t fr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a.xa + (size_t)c * CTOX_TILE_BLOCKS * M * 192), (short)0, (int)xbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a.xc + (size_t)c * CTOX_TILE_BLOCKS * M * 4), (short)0, (int)(xbytes / 12), 0x00020000);
    constexpr uint32_t XL = (CTOX_TILE_BLOCKS * MAXM * 192 + 4095) / 4096;  // 16-byte loads per thread
    v4i xl[XL];
#pragma unroll
    for (int i = 0; i < (int)XL; i++) xl[i] = __builtin_amdgcn_raw_buffer_load_b128(fr, (threadIdx.x + 256 * i) * 16, 0, 0);
    const v4i kv = __builtin_amdgcn_raw_buffer_load_b128(cr, threadIdx.x * 16, 0, 0);
    const RmsIn rin = rms_loads(a, M);
    __shared__ float invs[8];
    __builtin_amdgcn_sched_barrier(0);
    TileUnit<DT> u[U];
    v2u sc[U][4];
#pragma unroll
    for (int k = 0; k < U; k++) {
#pragma unroll
        for (int i = 0; i < (int)C::LPU; i++)
            u[k].w[i] = __builtin_amdgcn_raw_buffer_load_b128(wr, lane * 16, k * C::UB + i * 1024, CTOX_LOAD_NT);
        // Scales of row j for all 16 blocks: entries (g', j), g' = 0..3.
#pragma unroll
        for (int q = 0; q < 4; q++)
            sc[k][q] = __builtin_amdgcn_raw_buffer_load_b64(wr, C::CB + (q * 16 + j) * 8, k * C::UB, CTOX_LOAD_NT);
    }
#pragma unroll
    for (int i = 0; i < (int)XL; i++)
        if ((threadIdx.x + 256 * i) * 16 < CTOX_TILE_BLOCKS * MAXM * 192) *(v4i *)(xas + (threadIdx.x + 256 * i) * 16) = xl[i];
    if (threadIdx.x < CTOX_TILE_BLOCKS * MAXM)
        kqs[threadIdx.x] = make_float4(__int_as_float(kv[0]), __int_as_float(kv[1]), __int_as_float(kv[2]), __int_as_float(kv[3]));
    // Five rows: token 4's constants per lane group g (its limb g weighs
    // 2^(8 g); the offset term once, in group 0).
    __shared__ float2 kq4s[MM == 5 ? CTOX_TILE_BLOCKS * 4 : 1];
    if (MM == 5 && threadIdx.x < CTOX_TILE_BLOCKS * MAXM && threadIdx.x % MAXM == 4) {
        const uint32_t blk = threadIdx.x / MAXM;
#pragma unroll
        for (int q = 0; q < 4; q++)
            kq4s[blk * 4 + q] = q == 3 ? make_float2(0.0f, 0.0f)  // row 15 of the A operand: not token 4's
                                       : make_float2(__int_as_float(kv[0]) * (float)(1u << (8 * q)),
                                                     q == 0 ? __int_as_float(kv[3]) : 0.0f);
    }
    if (a.rms_sq) rms_finish(a, rin, invs);
    lds_barrier();
    if (t0 >= a.tiles) return;
    // Staged launches with a.rms_sq: 1 / rms of the lane's token rows.
    float inv[TG];
#pragma unroll
    for (int tg = 0; tg < (int)TG; tg++) inv[tg] = a.rms_sq ? invs[min(4 * tg + g, M - 1)] : 1.0f;

    // Tiles in load order (the compute of tile k needs only its own loads);
    // the A fragments are re-read from LDS per tile.
    float acc[U][TG];
    // Five rows (P5): one MFMA per block for all of them. Tokens 0..3 take
    // A rows 4t + l (limb l < 3) as in the four-token layout; token 4's limb
    // l takes the spare row 4l + 3 (row 15 stays zero), so lane group g
    // holds token g's limbs in C rows 0..2 and token 4's limb g in row 3.
    // Token 4's per-group parts (limb g weighted by 2^(8 g), its offset term
    // added by group 0 only) are summed over the groups once per tile.
    constexpr bool P5 = MM == 5;
    constexpr uint32_t TGC = P5 ? 1 : TG;
    float acc4[U];
#pragma unroll
    for (int k = 0; k < U; k++) {
        acc4[k] = 0.0f;
#pragma unroll
        for (int tg = 0; tg < TG; tg++) acc[k][tg] = 0.0f;
#pragma unroll
        for (int G = 0; G < 4; G++) {
            uint32_t e[4], o[4];
            if (DT) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const v4i W = u[k].w[2 * G + (q >> 1)];
                    e[q] = (uint32_t)W[2 * (q & 1)];
                    o[q] = (uint32_t)W[2 * (q & 1) + 1];
                }
                transpose4(e[0], e[1], e[2], e[3]);
                transpose4(o[0], o[1], o[2], o[3]);
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++) e[q] = (uint32_t)u[k].w[G][q];
                transpose4(e[0], e[1], e[2], e[3]);
            }
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const v4i bf = DT ? unpack_quarter<DT>(e[b], o[b]) : unpack_quarter<DT>(e[b], 0);
                const uint32_t sw = sc[k][b][G >> 1];
                const float scale = half_bits_to_float((G & 1) ? (sw >> 16) : (sw & 0xffffu));
#pragma unroll
                for (int tg = 0; tg < (int)TGC; tg++) {
                    // A lane (g, i): token 4 tg + i / 4, limb i % 4, quarter g;
                    // P5: row 4l + 3 is token 4's limb l. Rows whose C row no
                    // sum uses (limb 3, tokens past M, P5's row 15, whose
                    // constants are zero) read a valid row, so every lane's
                    // address is its base plus an immediate.
                    const bool spare = P5 && limb == 3;
                    const uint32_t tok = spare ? 4u : min(4 * tg + (j >> 2), M - 1);
                    const uint32_t lmb = spare ? min(j >> 2, 2u) : min(limb, 2u);
                    const v4i af = *(const v4i *)(xas + ((4 * G + b) * M + tok) * 192 + lmb * 64 + g * 16);
                    const v4i cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf, (v4i){0, 0, 0, 0}, 0, 0, 0);
                    const float4 kq = kqs[(4 * G + b) * M + min(4 * tg + g, M - 1)];
                    // Staged fragments: exact int32 limb sum for Q2 and Q4.
                    const float f = fmaf((float)(cc[0] + (cc[1] << 8) + (cc[2] << 16)), kq.x, kq.w);
                    acc[k][tg] = fmaf(f, scale, acc[k][tg]);
                    if (P5) {
                        const float2 k4 = kq4s[(4 * G + b) * 4 + g];
                        const float f4 = fmaf((float)cc[3], k4.x, k4.y);
                        acc4[k] = fmaf(f4, scale, acc4[k]);
                    }
                }
            }
        }
        if (P5) {
            // Token 4: groups (0 + 1) + (2 + 3); group 3's part is zero.
            const float s2 = acc4[k] + __shfl_xor(acc4[k], 16);
            acc[k][TG - 1] = s2 + __shfl_xor(s2, 32);
        }
    }
    small_m_finish<DT, U, TG, ARR, MM>(a, c, t0, n, g, j, M, acc, inv);
}

// ctox_q{2,4}_mv_tilem{M}_gfx950: M = 2..8 staged rows, one tile per wave.
#define CTOX_TILE_M_KERNEL(name, dt, u, m) \
    extern "C" __global__ __launch_bounds__(256) void name(TileMatvecArgs a) { tile_matvec_m<dt, u, m, 0>(a); } \
    extern "C" __global__ __launch_bounds__(256) void name##_arrive(TileMatvecArgs a) { tile_matvec_m<dt, u, m, 1>(a); }
CTOX_TILE_M_KERNEL(ctox_q2_mv_tilem2_gfx950, 0, 1, 2)
CTOX_TILE_M_KERNEL(ctox_q2_mv_tilem3_gfx950, 0, 1, 3)
CTOX_TILE_M_KERNEL(ctox_q2_mv_tilem4_gfx950, 0, 1, 4)
CTOX_TILE_M_KERNEL(ctox_q2_mv_tilem5_gfx950, 0, 1, 5)
CTOX_TILE_M_KERNEL(ctox_q2_mv_tilem6_gfx950, 0, 1, 6)
CTOX_TILE_M_KERNEL(ctox_q2_mv_tilem7_gfx950, 0, 1, 7)
CTOX_TILE_M_KERNEL(ctox_q2_mv_tilem8_gfx950, 0, 1, 8)
CTOX_TILE_M_KERNEL(ctox_q4_mv_tilem2_gfx950, 1, 1, 2)
CTOX_TILE_M_KERNEL(ctox_q4_mv_tilem3_gfx950, 1, 1, 3)
CTOX_TILE_M_KERNEL(ctox_q4_mv_tilem4_gfx950, 1, 1, 4)
CTOX_TILE_M_KERNEL(ctox_q4_mv_tilem5_gfx950, 1, 1, 5)
CTOX_TILE_M_KERNEL(ctox_q4_mv_tilem6_gfx950, 1, 1, 6)
CTOX_TILE_M_KERNEL(ctox_q4_mv_tilem7_gfx950, 1, 1, 7)
CTOX_TILE_M_KERNEL(ctox_q4_mv_tilem8_gfx950, 1, 1, 8)

// ---------------------------------------------------------------------------
// Small-M tiled matvec with the activation rows built in the kernel
// (ctox_q{2,4}_mv_tilemx{2,3,4,5}_gfx950, 2..5 rows): the MTP verify
// projections without a staging launch. The MFMA scheme, chunks and combine
// are those of tile_matvec_m; what differs is where the fragments come from:
//  * each wave copies its group's inputs of every row (the producer rows
//    the transform reads, 1 KiB per row and operand) straight into LDS with
//    buffer loads that write LDS (no registers held while the weight loads
//    are in flight), then issues its weight loads;
//  * after an explicit wait that leaves the weight loads outstanding, it
//    builds its group's fragments of every row (frag_group_build, the
//    batch-1 arithmetic) into the workgroup's [block][row] fragment area;
//  * the residual norm reads the producer's per-tile sums of squares of
//    every row (wave 0 copies them into LDS; one LDS barrier shares them).
// A producer with a residual in view writes those sums for every row.
// Waits until at most n vector-memory operations of this wave are
// outstanding (gfx9 s_waitcnt: vmcnt in bits 3:0 and 15:14, expcnt and
// lgkmcnt left at their maxima).
#define CTOX_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

typedef __attribute__((address_space(3))) void *lds_ptr_t;

__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, void *lds, uint32_t voff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 16, voff, 0, 0, 0);
}

// NW waves per workgroup (a multiple of 4, all on one chunk): wave w builds
// group w % 4 of rows w / 4, w / 4 + NW / 4, ... so a wider workgroup splits
// the chunk's 4 x M group builds over more waves.
template <int DT, int MR, int ARR, int NW = 4>
__device__ __forceinline__ void tile_matvec_mx(const TileMatvecArgs &a) {
    using C = TlCfg<DT>;
    constexpr uint32_t U = 1, TG = (MR + 3) / 4, INB = 2048;
    constexpr uint32_t RW = NW / 4;  // rows a group's builders step by
    constexpr uint32_t WLOADS = U * (C::LPU + 4);  // weight loads issued after the input copies
    __shared__ __align__(16) uint8_t ins[4 * MR * INB];
    __shared__ __align__(16) int8_t xas[CTOX_TILE_BLOCKS * MR * 192];
    __shared__ float4 kqs[CTOX_TILE_BLOCKS * MR];
    __shared__ __align__(16) float sqs[MR * 512];
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t v = __builtin_amdgcn_readfirstlane(blockIdx.x * (uint32_t)NW + w);
    const uint32_t c = v / a.segs, s = v - c * a.segs;
    constexpr uint32_t M = MR;
    const uint32_t t0 = s * U;
    if (c >= a.chunks) return;  // uniform over the workgroup (segs is a multiple of NW)
    const uint32_t n = t0 < a.tiles ? min(U, a.tiles - t0) : 0u;
    const uint8_t *base = a.weights + ((size_t)c * a.tiles + min(t0, a.tiles - 1)) * C::UB;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)(n * C::UB), 0x00020000);
    const uint32_t g = lane >> 4, j = lane & 15, limb = j & 3;
    const uint32_t cols = a.blocks * CTOX_BLOCK_LEN, xm = a.xmode, dh = a.head_dim ? a.head_dim : 1u;
    const uint32_t wg = w & 3, r0 = w >> 2;  // this wave's group and first row
    const uint32_t grp = c * 4 + wg, col = grp * 256 + 4 * lane;

    // Input copies (rows t < M): operand a at [0, 1 KiB), b at [1 KiB, 2 KiB)
    // of the wave's row area; an absent operand reads zeros.
    {
        const uint32_t aext = xm == 2 ? a.off + cols : cols;
        const __amdgpu_buffer_rsrc_t ar = f32_rsrc(a.input, (M - 1) * a.a_stride + aext);
        const void *bp = xm == 1 ? (const void *)a.delta : (xm == 2 ? (const void *)a.input : (const void *)a.xb);
        const uint32_t bext = xm == 1 || xm == 3 ? cols : (xm == 2 ? a.off + cols : (xm == 4 ? 2 * cols : 0u));
        const uint32_t bstr = xm == 2 ? a.a_stride : a.b_stride;
        const __amdgpu_buffer_rsrc_t br = f32_rsrc(xm == 0 ? nullptr : bp, bext ? (M - 1) * bstr + bext : 0u);
        const uint32_t bo = xm == 2 ? a.off + col : (xm == 4 ? (col / dh) * 2 * dh + dh + col % dh : col);
        for (uint32_t t = r0; t < M; t += RW) {
            uint8_t *dst = ins + (wg * MR + t) * INB;
            lds_dma16(ar, dst, (t * a.a_stride + col) * 4);
            lds_dma16(br, dst + 1024, (t * bstr + bo) * 4);
        }
        if (xm == 1 && w == 0) {
            const __amdgpu_buffer_rsrc_t sr = f32_rsrc(a.sq_in, M * a.sq_n);
            for (uint32_t t = 0; t < M; t++) {
                lds_dma16(sr, sqs + t * 512, (t * a.sq_n + 4 * lane) * 4);
                lds_dma16(sr, sqs + t * 512 + 256, (t * a.sq_n + 256 + 4 * lane) * 4);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // Row-independent operands: the norm weight and s_in of the lane's columns.
    GroupIn gin;
    {
        const uint32_t sbytes = a.s_in_kind == CTOX_KSCALE_F32 ? 4u : 2u;
        const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
            (void *)a.s_in, (short)0, a.s_in_kind == CTOX_KSCALE_NONE ? 0 : (int)(cols * sbytes), 0x00020000);
        const __amdgpu_buffer_rsrc_t wr2 = f32_rsrc(xm == 1 || xm == 3 ? a.xw : nullptr, xm == 1 ? cols : dh);
        gin.w = __builtin_amdgcn_raw_buffer_load_b128(wr2, (xm == 3 ? col % dh : col) * 4, 0, 0);
        gin.s = __builtin_amdgcn_raw_buffer_load_b128(sr, col * sbytes, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    TileUnit<DT> u[U];
    v2u sc[U][4];
#pragma unroll
    for (int k = 0; k < (int)U; k++) {
#pragma unroll
        for (int i = 0; i < (int)C::LPU; i++)
            u[k].w[i] = __builtin_amdgcn_raw_buffer_load_b128(wr, lane * 16, k * C::UB + i * 1024, CTOX_LOAD_NT);
#pragma unroll
        for (int q = 0; q < 4; q++)
            sc[k][q] = __builtin_amdgcn_raw_buffer_load_b64(wr, C::CB + (q * 16 + j) * 8, k * C::UB, CTOX_LOAD_NT);
    }
    __builtin_amdgcn_sched_barrier(0);
    CTOX_WAIT_VMCNT(WLOADS);  // the input copies and the two operand loads have landed
    __builtin_amdgcn_sched_barrier(0);
    if (xm == 1) lds_barrier();  // wave 0's copy of the sums is visible
    const bool keep = ((blockIdx.x * (uint32_t)NW) % a.segs) == 0;  // segment 0 of the chunk
    // One row at a time (not unrolled: the build's temporaries are live
    // beside the weight loads in flight).
#pragma unroll 1
    for (uint32_t t = r0; t < M; t += RW) {
        float inv = 0.0f;
        if (xm == 1) {
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint32_t idx = lane + 64 * k;
                ss += idx < a.sq_n ? sqs[t * 512 + idx] : 0.0f;
            }
            ss = row16_reduce(ss, [](float x, float y) { return x + y; });
            ss += __shfl_xor(ss, 16);
            ss += __shfl_xor(ss, 32);
            inv = 1.0f / sqrtf(ss / (float)cols + a.eps);
        }
        const uint8_t *src = ins + (wg * MR + t) * INB;
        gin.a = *(const v4i *)(src + lane * 16);
        gin.b = *(const v4i *)(src + 1024 + lane * 16);
        const float4 k = frag_group_build<DT>(a, grp, lane, gin, inv, keep, xas + ((4 * wg) * M + t) * 192, M * 192,
                                              a.x_out ? a.x_out + (size_t)t * cols : nullptr,
                                              a.norm_out ? a.norm_out + (size_t)t * cols : nullptr, a.xmode);
        if (j == 0) kqs[(4 * wg + g) * M + t] = k;
    }
    lds_barrier();  // fragments and constants of every group and row
    if (t0 >= a.tiles) return;

    // Per lane and token group: the A fragment base (row 4 tg + j / 4, limb
    // j % 4, quarter g; lanes outside the rows or on limb 3 read a valid row
    // whose C row nothing uses) and the epilogue constants' row.
    const int8_t *abase[TG];
    const float4 *kbase[TG];
#pragma unroll
    for (int tg = 0; tg < (int)TG; tg++) {
        const uint32_t tok = min(4 * tg + (j >> 2), M - 1);
        abase[tg] = xas + tok * 192 + min(limb, 2u) * 64 + g * 16;
        kbase[tg] = kqs + min(4 * tg + g, M - 1);
    }
    float acc[U][TG];
#pragma unroll
    for (int k = 0; k < (int)U; k++) {
#pragma unroll
        for (int tg = 0; tg < (int)TG; tg++) acc[k][tg] = 0.0f;
#pragma unroll
        for (int G = 0; G < 4; G++) {
            uint32_t e[4], o[4];
            if (DT) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const v4i W = u[k].w[2 * G + (q >> 1)];
                    e[q] = (uint32_t)W[2 * (q & 1)];
                    o[q] = (uint32_t)W[2 * (q & 1) + 1];
                }
                transpose4(e[0], e[1], e[2], e[3]);
                transpose4(o[0], o[1], o[2], o[3]);
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++) e[q] = (uint32_t)u[k].w[G][q];
                transpose4(e[0], e[1], e[2], e[3]);
            }
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const v4i bf = DT ? unpack_quarter<DT>(e[b], o[b]) : unpack_quarter<DT>(e[b], 0);
                const uint32_t sw = sc[k][b][G >> 1];
                const float scale = half_bits_to_float((G & 1) ? (sw >> 16) : (sw & 0xffffu));
#pragma unroll
                for (int tg = 0; tg < (int)TG; tg++) {
                    const v4i af = *(const v4i *)(abase[tg] + (4 * G + b) * M * 192);
                    const v4i cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf, (v4i){0, 0, 0, 0}, 0, 0, 0);
                    const float4 kq = kbase[tg][(4 * G + b) * M];
                    // Fragments built here: Q4 limbs combine in float (22 bits).
                    float f;
                    if (DT) {
                        f = fmaf((float)cc[0], kq.x, kq.w);
                        f = fmaf((float)cc[1], kq.y, f);
                        f = fmaf((float)cc[2], kq.z, f);
                    } else {
                        f = fmaf((float)(cc[0] + (cc[1] << 8) + (cc[2] << 16)), kq.x, kq.w);
                    }
                    acc[k][tg] = fmaf(f, scale, acc[k][tg]);
                }
            }
        }
    }
    const float inv[TG] = {};
    float one[TG];
#pragma unroll
    for (int tg = 0; tg < (int)TG; tg++) one[tg] = 1.0f + inv[tg];
    small_m_finish<DT, U, TG, ARR>(a, c, t0, n, g, j, M, acc, one);
}

#define CTOX_TILE_MX_KERNEL(name, dt, mr) \
    extern "C" __global__ __launch_bounds__(256, 2) void name(TileMatvecArgs a) { tile_matvec_mx<dt, mr, 0>(a); } \
    extern "C" __global__ __launch_bounds__(256, 2) void name##_arrive(TileMatvecArgs a) { tile_matvec_mx<dt, mr, 1>(a); }
CTOX_TILE_MX_KERNEL(ctox_q2_mv_tilemx2_gfx950, 0, 2)
CTOX_TILE_MX_KERNEL(ctox_q2_mv_tilemx3_gfx950, 0, 3)
CTOX_TILE_MX_KERNEL(ctox_q2_mv_tilemx4_gfx950, 0, 4)
CTOX_TILE_MX_KERNEL(ctox_q2_mv_tilemx5_gfx950, 0, 5)
CTOX_TILE_MX_KERNEL(ctox_q4_mv_tilemx2_gfx950, 1, 2)
CTOX_TILE_MX_KERNEL(ctox_q4_mv_tilemx3_gfx950, 1, 3)
CTOX_TILE_MX_KERNEL(ctox_q4_mv_tilemx4_gfx950, 1, 4)
CTOX_TILE_MX_KERNEL(ctox_q4_mv_tilemx5_gfx950, 1, 5)


// Rewrites crate rows (Q/src/quant.rs:20-29 block layout, rows dense) into
// the tiled layout; one workgroup per unit, lane (g, j) moves its fragment
// of each of the unit's four groups. Runs once per matrix at prepare time.
extern "C" __global__ __launch_bounds__(64) void ctox_tile_repack_gfx950(TileRepackArgs a) {
    const uint32_t u = blockIdx.x, lane = threadIdx.x;
    const uint32_t c = u / a.tiles, t = u - c * a.tiles;
    const uint32_t g = lane >> 4, j = lane & 15, row = t * CTOX_TILE_ROWS + j;
    const uint32_t bb = a.dtype ? CTOX_Q4_BLOCK_BYTES : CTOX_Q2_BLOCK_BYTES, cbytes = bb - 2;
    const uint32_t codes = ctox_tile_code_bytes(a.dtype);
    uint8_t *dst = a.dst + (size_t)u * ctox_tile_unit_bytes(a.dtype);
    for (uint32_t G = 0; G < 4; G++) {
        const uint32_t blk = c * CTOX_TILE_BLOCKS + 4 * G + g;
        const bool ok = row < a.rows && blk < a.blocks;
        const uint8_t *src = a.src + ((size_t)row * a.blocks + blk) * bb;
        for (uint32_t h = 0; h < cbytes / 16; h++)
            for (uint32_t e = 0; e < 16; e++)
                dst[G * cbytes * 64 + h * 1024 + lane * 16 + e] = ok ? src[2 + 16 * h + e] : 0;
        dst[codes + lane * 8 + 2 * G] = ok ? src[0] : 0;
        dst[codes + lane * 8 + 2 * G + 1] = ok ? src[1] : 0;
    }
}
