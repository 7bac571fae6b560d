// Layer glue of one Qwen3.8 decoder layer, gfx950 (fp32).
//
//  * ctox_rms_norm_gfx950: per row r of [rows][cols],
//      mode 0  y = x * rsqrt(mean(x^2) + eps) * (1 + w)            Q/src/reference.rs:38-62
//      mode 1  y = x * rsqrt(mean(x^2) + eps) * w * silu(gate)     Q/src/reference.rs:66-93
//    One workgroup per row; the sum of squares is reduced in a fixed order.
//  * ctox_swiglu_gfx950: y = silu(gate) * up                      Q/src/reference.rs:96-112
//  * ctox_sigmoid_gate_gfx950: v *= 1 / (1 + exp(-gate))           Q/src/reference.rs:502-515
//  * ctox_conv_update_gfx950: per channel, shift the causal-conv state left by
//    one, append the input, y = silu(state . weight)               Q/src/reference.rs:159-187
//  * ctox_rope_gfx950: partial rotary embedding of the first rd dims of every
//    q and k head, pairs (i, i + rd/2), token row t at position p0 + t
//                                                                  Q/src/reference.rs:115-155
#include <hip/hip_runtime.h>

#include "kernel_args.h"

__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + expf(-v)); }

extern "C" __global__ __launch_bounds__(256) void ctox_rms_norm_gfx950(NormArgs a) {
    __shared__ float red[4];
    const float *x = a.x + (size_t)blockIdx.x * a.cols;
    float s = 0.0f;
    for (uint32_t c = threadIdx.x; c < a.cols; c += 256) s += x[c] * x[c];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    const float var = ((red[0] + red[1]) + (red[2] + red[3])) / (float)a.cols;
    const float inv = 1.0f / sqrtf(var + a.eps);
    float *y = a.out + (size_t)blockIdx.x * a.cols;
    const float *gate = a.gate ? a.gate + (size_t)blockIdx.x * a.cols : nullptr;
    for (uint32_t c = threadIdx.x; c < a.cols; c += 256) {
        const float n = x[c] * inv;
        y[c] = a.mode == 0 ? n * (1.0f + a.w[c]) : n * a.w[c] * silu_f(gate[c]);
    }
}

extern "C" __global__ __launch_bounds__(256) void ctox_swiglu_gfx950(EltArgs a) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < a.n) a.out[i] = silu_f(a.a[i]) * a.b[i];
}

extern "C" __global__ __launch_bounds__(256) void ctox_sigmoid_gate_gfx950(EltArgs a) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < a.n) a.out[i] = a.a[i] * (1.0f / (1.0f + expf(-a.b[i])));
}

extern "C" __global__ __launch_bounds__(256) void ctox_conv_update_gfx950(ConvArgs a) {
    const uint32_t c = blockIdx.x * 256 + threadIdx.x;
    if (c >= a.channels) return;
    float *s = a.state + (size_t)c * a.kernel;
    const float *w = a.weight + (size_t)c * a.kernel;
    for (uint32_t t = 0; t < a.rows; t++) {
        float sum = 0.0f;
        for (uint32_t i = 0; i + 1 < a.kernel; i++) {
            const float v = s[i + 1];
            s[i] = v;
            sum += v * w[i];
        }
        const float x = a.input[(size_t)t * a.in_stride + c];
        s[a.kernel - 1] = x;
        sum += x * w[a.kernel - 1];
        a.out[(size_t)t * a.channels + c] = silu_f(sum);
    }
}

// grid (rows, qh + kh), block = rd / 2 threads (<= 256).
extern "C" __global__ __launch_bounds__(256) void ctox_rope_gfx950(RopeArgs a) {
    const uint32_t t = blockIdx.x, hh = blockIdx.y, i = threadIdx.x;
    const uint32_t half = a.rd / 2;
    if (i >= half) return;
    const float invf = powf(a.theta, -((float)(2 * i)) / (float)a.rd);
    const float angle = (float)(a.position + t) * invf;  // u64 -> f32, as `position as f32`
    const float cs = cosf(angle), sn = sinf(angle);
    float *head = hh < a.qh ? a.q + ((size_t)t * a.qh + hh) * a.hd : a.k + ((size_t)t * a.kh + (hh - a.qh)) * a.hd;
    const float l = head[i], r = head[i + half];
    head[i] = l * cs - r * sn;
    head[i + half] = r * cs + l * sn;
}
