// Device helpers of the decode engine, gfx950.
//
//  * ctox_fill_random_gfx950: seeded synthetic tensors (counter-based
//    splitmix64 per element, so any sub-range is reproducible): Q4 / Q2
//    blocks with uniform codes and fp16 scales |N(0, sigma)|, f32 normal,
//    f32 uniform and fp16 uniform values.
//  * ctox_embed_rows_gfx950: recovered_row of a quantized matrix for token
//    ids held on the device, out[r][c] = ((scale * level) * s_in[c]) * s_out[tok]
//    (Q/src/backend/cpu.rs:474-476, Q/src/decoder.rs:531-537).
//  * ctox_norm_rows_gfx950: RMS norms over rows addressed with two-level
//    strides (row r -> (r / inner) * outer_stride + (r % inner) * inner_stride),
//    optionally adding a residual delta first (h += delta, written back):
//      mode 0  y = x * rsqrt(mean(x^2) + eps) * (1 + w)         Q/src/reference.rs:38-62
//      mode 1  y = x * rsqrt(mean(x^2) + eps) * w * silu(gate)  Q/src/reference.rs:66-93
//  * ctox_attn_gate_gfx950: values[t][h][d] *= sigmoid(gate), the gate read
//    from the [q, gate] halves of each head of q_proj's output
//    (Q/src/decoder.rs:727-737, :788; Q/src/reference.rs:502-515).
//  * ctox_swiglu_rows_gfx950: out[t][c] = silu(in[t][c]) * in[t][off + c]
//    over token rows of a fused gate|up projection (Q/src/reference.rs:96-112).
//  * ctox_copy_rows_gfx950: strided row copy.
//  * ctox_finite_check_gfx950: per-part flags of non-finite values in a
//    buffer (the engine's fail-closed check of logits).
//  * ctox_gather_rows_gfx950: byte rows gathered by index (the restricted
//    draft head's compact LM-head copy).
//  * ctox_stream_read_gfx950: a plain streaming read (the HBM floor the
//    matvec kernels are measured against): each wave reads 8 KiB with the
//    access pattern of the tiled matvec (every 16-byte load issued before
//    the first wait, non-temporal) and stores their xor.
//  * ctox_write_words_gfx950: up to 32 words carried in the kernel arguments
//    (token ids, page descriptors): ordered on the stream, no host buffer to keep alive.
#include <hip/hip_runtime.h>

#include "kernel_args.h"

__device__ __forceinline__ uint64_t eo_mix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float eo_unit(uint64_t bits) {  // [0, 1)
    return (float)(bits >> 40) * (1.0f / 16777216.0f);
}

__device__ __forceinline__ float eo_normal(uint64_t seed, uint64_t i) {
    const uint64_t r = eo_mix(seed ^ eo_mix(i));
    const float u1 = fmaxf(eo_unit(r), 1.0f / 16777216.0f), u2 = eo_unit(eo_mix(r));
    return sqrtf(-2.0f * logf(u1)) * cosf(6.28318530718f * u2);
}

__device__ __forceinline__ uint16_t eo_f16(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }

// One thread per element (kinds 2..4) or per quantized block (kinds 0, 1).
extern "C" __global__ __launch_bounds__(256) void ctox_fill_random_gfx950(FillArgs a) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.count) return;
    const uint64_t gi = i + a.index_base;
    switch (a.kind) {
    case 0:
    case 1: {
        const uint32_t bytes = a.kind == 0 ? 34 : 18;
        uint8_t *blk = (uint8_t *)a.ptr + i * bytes;
        const float sc = fabsf(eo_normal(a.seed, 2 * gi)) * a.p1;
        const uint16_t h = eo_f16(sc);
        blk[0] = (uint8_t)h;
        blk[1] = (uint8_t)(h >> 8);
        uint64_t r = eo_mix(a.seed ^ eo_mix(2 * gi + 1));
        for (uint32_t c = 0; c < bytes - 2; c++) {
            if ((c & 7) == 0 && c) r = eo_mix(r);
            blk[2 + c] = (uint8_t)(r >> (8 * (c & 7)));
        }
        break;
    }
    case 2:
        ((float *)a.ptr)[i] = a.p0 + a.p1 * eo_normal(a.seed, gi);
        break;
    case 3:
        ((uint16_t *)a.ptr)[i] = eo_f16(a.p0 + (a.p1 - a.p0) * eo_unit(eo_mix(a.seed ^ eo_mix(gi))));
        break;
    default:
        ((float *)a.ptr)[i] = a.p0 + (a.p1 - a.p0) * eo_unit(eo_mix(a.seed ^ eo_mix(gi)));
        break;
    }
}

__device__ __forceinline__ float eo_half(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// grid (ceil(cols / 256), rows)
extern "C" __global__ __launch_bounds__(256) void ctox_embed_rows_gfx950(EmbedArgs a) {
    const uint32_t c = blockIdx.x * 256 + threadIdx.x, r = blockIdx.y;
    if (c >= a.cols) return;
    const uint32_t tok = a.tokens[r];
    float v = 0.0f;
    if (tok < a.vocab) {
        const uint32_t blk = c / 64, e = c % 64;
        float n, scale;
        if (a.dtype == 1) {
            const uint8_t *b = a.weights + ((size_t)tok * (a.cols / 64) + blk) * 34;
            scale = eo_half((uint32_t)b[0] | ((uint32_t)b[1] << 8));
            const uint32_t code = (b[2 + e / 2] >> (4 * (e & 1))) & 15u;
            n = ((float)code - 7.5f) / 7.5f;
        } else {
            const uint8_t *b = a.weights + ((size_t)tok * (a.cols / 64) + blk) * 18;
            scale = eo_half((uint32_t)b[0] | ((uint32_t)b[1] << 8));
            const uint32_t code = (b[2 + e / 4] >> (2 * (e & 3))) & 3u;
            const float cb[4] = {-1.0f, -1.0f / 3.0f, 1.0f / 3.0f, 1.0f};
            n = cb[code];
        }
        const float si = a.s_in ? eo_half(a.s_in[c]) : 1.0f;
        const float so = a.s_out ? eo_half(a.s_out[tok]) : 1.0f;
        v = ((scale * n) * si) * so;
    }
    a.out[(size_t)r * a.cols + c] = v;
}

__device__ __forceinline__ float eo_silu(float v) { return v / (1.0f + expf(-v)); }

// One workgroup per row, blockDim.x = 64 * waves threads; each thread keeps its
// (up to NR_PER) columns c = tid + k * blockDim.x in registers, so every load
// of the row is in flight at once. Sums of squares reduced in a fixed order.
#define NR_PER 8
extern "C" __global__ __launch_bounds__(1024) void ctox_norm_rows_gfx950(NormRowsArgs a) {
    __shared__ float red[16];
    const uint32_t r = blockIdx.x, T = blockDim.x, tid = threadIdx.x;
    const size_t xo = (size_t)(r / a.inner) * a.x_outer + (size_t)(r % a.inner) * a.x_inner;
    float *x = a.x + xo;
    const float *dl = a.delta ? a.delta + (size_t)r * a.cols : nullptr;
    float v[NR_PER];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NR_PER; k++) {
        const uint32_t c = tid + k * T;
        v[k] = c < a.cols ? x[c] : 0.0f;
    }
    if (dl) {
#pragma unroll
        for (int k = 0; k < NR_PER; k++) {
            const uint32_t c = tid + k * T;
            if (c < a.cols) {
                float d = dl[c];
                for (uint32_t p = 1; p < a.delta_parts; p++) d += dl[(size_t)p * a.delta_stride + c];
                v[k] += d;
                x[c] = v[k];
            }
        }
    }
#pragma unroll
    for (int k = 0; k < NR_PER; k++) s += v[k] * v[k];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    float tot = 0.0f;
    for (uint32_t w = 0; w < T / 64; w++) tot += red[w];
    const float inv = 1.0f / sqrtf(tot / (float)a.cols + a.eps);
    float *y = a.out + (size_t)r * a.out_stride;
    const float *g = a.gate ? a.gate + (size_t)(r / a.inner) * a.g_outer + (size_t)(r % a.inner) * a.g_inner : nullptr;
#pragma unroll
    for (int k = 0; k < NR_PER; k++) {
        const uint32_t c = tid + k * T;
        if (c < a.cols) {
            const float n = v[k] * inv;
            y[c] = a.mode == 0 ? n * (1.0f + a.w[c]) : n * a.w[c] * eo_silu(g[c]);
        }
    }
}

extern "C" __global__ __launch_bounds__(256) void ctox_attn_gate_gfx950(AttnGateArgs a) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (uint64_t)a.rows * a.heads * a.head_dim) return;
    const uint32_t d = (uint32_t)(i % a.head_dim), h = (uint32_t)((i / a.head_dim) % a.heads);
    const uint32_t t = (uint32_t)(i / ((uint64_t)a.head_dim * a.heads));
    const float g = a.qg[(size_t)t * a.qg_stride + (size_t)h * 2 * a.head_dim + a.head_dim + d];
    a.values[i] *= 1.0f / (1.0f + expf(-g));
}

extern "C" __global__ __launch_bounds__(256) void ctox_swiglu_rows_gfx950(RowsArgs a) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (uint64_t)a.rows * a.cols) return;
    const uint32_t c = (uint32_t)(i % a.cols), t = (uint32_t)(i / a.cols);
    const float *in = a.in + (size_t)t * a.in_stride;
    a.out[(size_t)t * a.out_stride + c] = eo_silu(in[c]) * in[a.offset + c];
}

extern "C" __global__ __launch_bounds__(256) void ctox_copy_rows_gfx950(RowsArgs a) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (uint64_t)a.rows * a.cols) return;
    const uint32_t c = (uint32_t)(i % a.cols), t = (uint32_t)(i / a.cols);
    a.out[(size_t)t * a.out_stride + c] = a.in[(size_t)t * a.in_stride + a.offset + c];
}

extern "C" __global__ __launch_bounds__(64) void ctox_write_words_gfx950(WordsArgs a) {
    if (threadIdx.x < a.count) a.dst[threadIdx.x] = a.words[threadIdx.x];
}

// grid (1), 512 threads: word i of the argument block goes to its segment.
extern "C" __global__ __launch_bounds__(512) void ctox_write_segments_gfx950(SegWordsArgs a) {
    const uint32_t i = threadIdx.x;
    if (i >= a.off[a.nseg]) return;
    uint32_t sgm = 0;
    for (uint32_t k = 1; k < a.nseg; k++) sgm += i >= a.off[k];
    a.dst[sgm][i - a.off[sgm]] = a.words[i];
}

// grid (parts), 256 threads: part p checks its contiguous range of float4
// (the tail floats by the last part) and always writes flags[p].
extern "C" __global__ __launch_bounds__(256) void ctox_finite_check_gfx950(FiniteArgs a) {
    int bad = 0;
    const uint64_t n4 = a.n / 4, per = (n4 + gridDim.x - 1) / gridDim.x;
    const uint64_t b = (uint64_t)blockIdx.x * per, e = min(n4, b + per);
    const float4 *x4 = (const float4 *)a.x;
    for (uint64_t i = b + threadIdx.x; i < e; i += 256) {
        const float4 v = x4[i];
        bad |= !__builtin_isfinite(v.x) | !__builtin_isfinite(v.y) | !__builtin_isfinite(v.z) | !__builtin_isfinite(v.w);
    }
    if (blockIdx.x + 1 == gridDim.x)
        for (uint64_t i = 4 * n4 + threadIdx.x; i < a.n; i += 256) bad |= !__builtin_isfinite(a.x[i]);
    bad = __syncthreads_or(bad);
    if (threadIdx.x == 0) a.flags[blockIdx.x] = bad ? 1u : 0u;
}

// grid (rows), 256 threads: dst row r = src row ids[r], 16 bytes per thread step.
extern "C" __global__ __launch_bounds__(256) void ctox_gather_rows_gfx950(GatherRowsArgs a) {
    const uint32_t r = blockIdx.x;
    const uint8_t *src = a.src + (uint64_t)a.ids[r] * a.row_bytes;
    uint8_t *dst = a.dst + (uint64_t)r * a.row_bytes;
    for (uint64_t i = threadIdx.x; i < a.row_bytes; i += 256) dst[i] = src[i];
}

extern "C" __global__ __launch_bounds__(256) void ctox_stream_read_gfx950(StreamReadArgs a) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t w = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint64_t base = w * 8192;
    if (base >= a.bytes) return;
    const uint64_t n = a.bytes - base < 8192 ? a.bytes - base : 8192;
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void *)(a.src + base), (short)0, (int)n, 0x00020000);
    v4i v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = __builtin_amdgcn_raw_buffer_load_b128(r, lane * 16 + i * 1024, 0, 2);
    uint32_t x = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) x ^= (uint32_t)(v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o);
    if (lane == 0) a.out[w] = x;
}
