// Decode-step glue and token selection on the device, gfx950.
//
//  * ctox_gdn_gates_gfx950: beta = 1 / (1 + exp(-b)),
//    log_decay = -exp(A_log) * softplus(a + dt_bias), softplus(x) = x for
//    x > 20 (Q/src/decoder.rs:29-35, 881-902), over [tokens][heads].
//  * ctox_repeat_heads_gfx950: out[row][h * repeats + r][:] = in[row][h][:]
//    (Q/src/decoder.rs:47-65).
//  * Greedy selection: argmax under f32::total_cmp with the later index
//    winning ties (Q/src/engine.rs:906-913). A vocabulary row is split into
//    parts reduced by separate workgroups (ctox_row_partials_gfx950, mode 0)
//    and merged in index order of the parts (ctox_argmax_final_gfx950, or the
//    greedy MTP verification ctox_verify_greedy_gfx950 of
//    Q/src/engine.rs:915-963).
//  * Speculative rejection sampling at temperature T (no counterpart in the
//    crate, whose MTP path is greedy-only): draft i is accepted iff
//    u * q(d_i) < p(d_i), p / q the temperature-scaled softmaxes of target /
//    draft row i, u the next draw of the crate's Pcg32
//    (Q/src/sampler.rs:149-174); on the first rejection the token is drawn
//    from max(0, p - q) with the next draw by the cumulative search of
//    Q/src/sampler.rs:134-143; when every draft is accepted the bonus token is
//    drawn from the bonus row's softmax. Passes: per-part softmax statistics
//    (ctox_row_partials_gfx950, mode 1, all rows in one launch), the draws and
//    accept tests on merged statistics (ctox_mtp_decide_gfx950), per-part
//    weight sums (ctox_pick_sums_gfx950) and the search itself, which scans
//    only the part where the running sum crosses the threshold
//    (ctox_pick_final_gfx950). The generator state lives in device memory and
//    is advanced in place.
#include <hip/hip_runtime.h>

#include "kernel_args.h"

extern "C" __global__ __launch_bounds__(256) void ctox_gdn_gates_gfx950(GateArgs a) {
    const uint32_t e = blockIdx.x * 256 + threadIdx.x;
    if (e >= a.tokens * a.heads) return;
    const uint32_t h = e % a.heads, t = e / a.heads;
    const size_t in = (size_t)t * a.in_stride + h;
    a.beta[e] = 1.0f / (1.0f + expf(-a.b[in]));
    const float x = a.a[in] + a.dt_bias[h];
    const float sp = x > 20.0f ? x : log1pf(expf(x));
    a.log_decay[e] = -expf(a.a_log[h]) * sp;
}

extern "C" __global__ __launch_bounds__(256) void ctox_repeat_heads_gfx950(RepeatArgs a) {
    const uint64_t e = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    const uint64_t per_row = (uint64_t)a.heads * a.repeats * a.dim;
    if (e >= per_row * a.rows) return;
    const uint64_t row = e / per_row, rem = e % per_row;
    const uint32_t hr = (uint32_t)(rem / a.dim), i = (uint32_t)(rem % a.dim);
    const uint32_t h = hr / a.repeats;
    a.out[e] = a.in[(row * a.heads + h) * a.dim + i];
}

// Order key of f32::total_cmp: signed-integer order of the bits with the
// magnitude bits flipped for negative values.
__device__ __forceinline__ int32_t total_key(float v) {
    const int32_t b = __float_as_int(v);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}
// (key, index) max with the later index winning equal keys.
__device__ __forceinline__ void take_max(int32_t &k, uint32_t &i, int32_t k2, uint32_t i2) {
    if (k2 > k || (k2 == k && i2 > i)) {
        k = k2;
        i = i2;
    }
}

__device__ __forceinline__ const float *logits_row(const PartialArgs &a, uint32_t r) {
    return r < a.drafts ? a.draft + (size_t)r * a.draft_vocab
                        : (r < 2 * a.drafts ? a.target + (size_t)(r - a.drafts) * a.vocab : a.bonus);
}

// grid (rows, parts), 256 threads: one part of one row.
extern "C" __global__ __launch_bounds__(256) void ctox_row_partials_gfx950(PartialArgs a) {
    __shared__ float s0[4], s1[4];
    const uint32_t r = blockIdx.x, part = blockIdx.y;
    const float *row = logits_row(a, r);
    const uint32_t len = r < a.drafts ? a.draft_vocab : a.vocab;
    const uint32_t per = (len + a.parts - 1) / a.parts;
    const uint32_t b = part * per, e = min(len, b + per);
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    float *o = a.out + ((size_t)r * a.parts + part) * 2;
    if (a.mode == 0) {
        int32_t k = INT32_MIN;
        uint32_t idx = 0;
        bool any = false;
        for (uint32_t i = b + threadIdx.x; i < e; i += 256) {
            const int32_t ki = total_key(row[i]);
            if (!any) {
                k = ki;
                idx = i;
                any = true;
            } else {
                take_max(k, idx, ki, i);
            }
        }
        if (!any) idx = b;  // empty lanes keep key INT32_MIN at the part's first index
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) take_max(k, idx, __shfl_xor(k, off), __shfl_xor(idx, off));
        if (lane == 0) {
            s0[w] = __int_as_float(k);
            s1[w] = __uint_as_float(idx);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            int32_t bk = __float_as_int(s0[0]);
            uint32_t bi = __float_as_uint(s1[0]);
            for (int q = 1; q < 4; q++) take_max(bk, bi, __float_as_int(s0[q]), __float_as_uint(s1[q]));
            o[0] = __int_as_float(bk);
            o[1] = __uint_as_float(bi);
        }
        return;
    }
    const float invt = 1.0f / a.temperature;
    float m = -INFINITY;
    int bad = 0;
    for (uint32_t i = b + threadIdx.x; i < e; i += 256) {
        bad |= !__builtin_isfinite(row[i]);
        m = fmaxf(m, row[i] * invt);
    }
    // A non-finite logit anywhere in the row makes its part's sum NaN, which
    // the decision pass reports (the step fails closed).
    bad = __syncthreads_or(bad);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if (lane == 0) s0[w] = m;
    __syncthreads();
    const float mm = fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3]));
    float z = 0.0f;
    if (mm > -INFINITY)
        for (uint32_t i = b + threadIdx.x; i < e; i += 256) z += expf(row[i] * invt - mm);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) z += __shfl_xor(z, off);
    if (lane == 0) s1[w] = z;
    __syncthreads();
    if (threadIdx.x == 0) {
        o[0] = mm;
        o[1] = bad ? __builtin_nanf("") : (s1[0] + s1[1]) + (s1[2] + s1[3]);
    }
}

// Merges a row's partials across one wave (lane q holds part q, parts <= 64);
// every lane returns the result. Argmax (mode 0) or {m, z} (mode 1).
__device__ __forceinline__ uint32_t merge_argmax(const float *p, uint32_t parts) {
    const uint32_t q = threadIdx.x & 63;
    int32_t k = INT32_MIN;
    uint32_t i = 0xffffffffu;
    if (q < parts) {
        k = __float_as_int(p[2 * q]);
        i = __float_as_uint(p[2 * q + 1]);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const int32_t k2 = __shfl_xor(k, off);
        const uint32_t i2 = __shfl_xor(i, off);
        // unused lanes (index 0xffffffff) never win
        if (i2 != 0xffffffffu && (i == 0xffffffffu || k2 > k || (k2 == k && i2 > i))) {
            k = k2;
            i = i2;
        }
    }
    return i;
}
__device__ __forceinline__ void merge_stats(const float *p, uint32_t parts, float &m, float &z) {
    const uint32_t q = threadIdx.x & 63;
    const float mq = q < parts ? p[2 * q] : -INFINITY, zq = q < parts ? p[2 * q + 1] : 0.0f;
    m = mq;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    z = mq > -INFINITY ? zq * expf(mq - m) : 0.0f;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) z += __shfl_xor(z, off);
}

// grid rows, 64 threads: merges the mode-0 partials of `drafts` rows; with
// `ids` the winning index is mapped to its token (a restricted draft row).
extern "C" __global__ __launch_bounds__(64) void ctox_argmax_final_gfx950(VerifyArgs a) {
    const uint32_t t = merge_argmax(a.partials + (size_t)blockIdx.x * a.parts * 2, a.parts);
    if (threadIdx.x == 0) a.out[blockIdx.x] = a.ids ? a.ids[t] : t;
}

// From the mode-0 partials of the draft, target and bonus rows.
// out: [0] next token, [1] verified, [2] accepted count, [3 ..] accepted tokens.
extern "C" __global__ __launch_bounds__(64) void ctox_verify_greedy_gfx950(VerifyArgs a) {
    const bool lead = threadIdx.x == 0;
    uint32_t nacc = 0;
    for (uint32_t i = 0; i < a.drafts; i++) {
        const uint32_t d = merge_argmax(a.partials + (size_t)i * a.parts * 2, a.parts);
        const uint32_t t = merge_argmax(a.partials + (size_t)(a.drafts + i) * a.parts * 2, a.parts);
        if (d != t) {
            if (lead) {
                a.out[0] = t;
                a.out[1] = i + 1;
                a.out[2] = nacc;
            }
            return;
        }
        if (lead) a.out[3 + nacc] = d;
        nacc++;
    }
    const uint32_t bonus = merge_argmax(a.partials + (size_t)(2 * a.drafts) * a.parts * 2, a.parts);
    if (lead) {
        a.out[0] = bonus;
        a.out[1] = a.drafts;
        a.out[2] = nacc;
    }
}

// One wave: the greedy sampler's status words from the finite-check flags
// of its logits (status 2 on a non-finite logit, Q/src/sampler.rs:66-70,
// which the crate checks before its greedy branch).
extern "C" __global__ __launch_bounds__(64) void ctox_greedy_status_gfx950(FlagStatusArgs a) {
    uint32_t bad = 0;
    for (uint32_t i = threadIdx.x; i < a.parts; i += 64) bad |= a.flags[i];
    bad = __any(bad != 0);
    if (threadIdx.x == 0) {
        a.out[1] = bad ? 2u : 0u;
        a.out[2] = bad ? 0u : 1u;
        a.out[3] = 0u;
    }
}

__device__ __forceinline__ uint32_t pcg32_next(uint64_t &s) {
    const uint64_t old = s;
    s = old * 6364136223846793005ULL + 1442695040888963407ULL;
    const uint32_t shifted = (uint32_t)(((old >> 18) ^ old) >> 27);
    const uint32_t rot = (uint32_t)(old >> 59);
    return (shifted >> rot) | (shifted << ((32u - rot) & 31u));
}
__device__ __forceinline__ float pcg32_f32(uint64_t &s) {
    return (float)((double)pcg32_next(s) / 4294967296.0);
}

// Decision pass (one thread): replays the Pcg32 draws of the accept tests on
// merged statistics; records which weight row the cumulative search uses.
extern "C" __global__ __launch_bounds__(64) void ctox_mtp_decide_gfx950(AcceptArgs a) {
    const bool lead = threadIdx.x == 0;
    const float invt = 1.0f / a.temperature;
    uint64_t s = *a.rng;  // every lane replays the same draws
    PickState st{};
    uint32_t acc = 0;
    // Fail closed: a non-finite logit in any row (NaN part sum) ends the
    // step with no token (mode 3) and consumes no draw.
    bool finite = true;
    for (uint32_t r = 0; r < 2 * a.drafts + 1; r++) {
        float m, z;
        merge_stats(a.partials + (size_t)r * a.parts * 2, a.parts, m, z);
        finite = finite && __builtin_isfinite(z) && z > 0.0f;
    }
    if (!finite) {
        st.mode = 3;
        if (lead) *a.state = st;
        return;
    }
    for (uint32_t i = 0; i < a.drafts; i++) {
        float tm, tz, dm, dz;
        merge_stats(a.partials + (size_t)(a.drafts + i) * a.parts * 2, a.parts, tm, tz);
        merge_stats(a.partials + (size_t)i * a.parts * 2, a.parts, dm, dz);
        const uint32_t d = a.tokens[i];
        if (d >= a.vocab) {  // not a token of this vocabulary: report, consume nothing more
            st.mode = 2;
            st.accepted = acc;
            if (lead) {
                *a.state = st;
                *a.rng = s;
            }
            return;
        }
        const float p = expf(a.target[(size_t)i * a.vocab + d] * invt - tm) / tz;
        const uint32_t di = a.draft_inv ? a.draft_inv[d] : d;
        const float q = di < a.draft_vocab ? expf(a.draft[(size_t)i * a.draft_vocab + di] * invt - dm) / dz : 0.0f;
        const float u = pcg32_f32(s);
        if (u * q < p) {
            acc++;
            continue;
        }
        st.thr_draw = pcg32_f32(s);
        st.m_t = tm;
        st.z_t = tz;
        st.m_d = dm;
        st.z_d = dz;
        st.row = i;
        st.accepted = acc;
        st.mode = 0;
        if (lead) {
            *a.state = st;
            *a.rng = s;
        }
        return;
    }
    merge_stats(a.partials + (size_t)(2 * a.drafts) * a.parts * 2, a.parts, st.m_t, st.z_t);
    st.thr_draw = pcg32_f32(s);
    st.row = a.drafts;
    st.accepted = acc;
    st.mode = 1;
    if (lead) {
        *a.state = st;
        *a.rng = s;
    }
}

__device__ __forceinline__ float pick_weight(const AcceptArgs &a, const PickState &st, uint32_t t, float invt) {
    if (st.mode == 1) return expf(a.bonus[t] * invt - st.m_t) / st.z_t;
    const float p = expf(a.target[(size_t)st.row * a.vocab + t] * invt - st.m_t) / st.z_t;
    const uint32_t di = a.draft_inv ? a.draft_inv[t] : t;
    const float q = di < a.draft_vocab ? expf(a.draft[(size_t)st.row * a.draft_vocab + di] * invt - st.m_d) / st.z_d
                                       : 0.0f;
    const float r = p - q;
    return r > 0.0f ? r : 0.0f;
}

// grid parts2, 256 threads: per-part sums of the weights in index order.
extern "C" __global__ __launch_bounds__(256) void ctox_pick_sums_gfx950(AcceptArgs a) {
    __shared__ float red[4];
    const PickState st = *a.state;
    if (st.mode >= 2) return;
    const float invt = 1.0f / a.temperature;
    const uint32_t per = (a.vocab + a.parts2 - 1) / a.parts2;
    const uint32_t b = blockIdx.x * per, e = min(a.vocab, b + per);
    float z = 0.0f;
    for (uint32_t i = b + threadIdx.x; i < e; i += 256) z += pick_weight(a, st, i, invt);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) z += __shfl_xor(z, off);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = z;
    __syncthreads();
    if (threadIdx.x == 0) a.sums[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

// One workgroup (1024 threads): thr = u * total; the part where the running
// sum reaches thr is scanned element by element; the first index with w > 0
// and thr <= running sum is the token (the last positive index if rounding
// leaves thr above the total), as in the sequential search.
extern "C" __global__ __launch_bounds__(1024) void ctox_pick_final_gfx950(AcceptArgs a) {
    __shared__ float scan[1024];
    __shared__ float seg[1024];
    __shared__ uint32_t res[3];
    const PickState st = *a.state;
    const uint32_t tid = threadIdx.x;
    if (st.mode >= 2) {  // 2: a proposed token outside the vocabulary, 3: non-finite logits
        if (tid == 0) {
            a.out[0] = st.mode == 3 ? 0xfffffffeu : 0xffffffffu;
            a.out[1] = st.accepted;
        }
        return;
    }
    const float invt = 1.0f / a.temperature;
    // inclusive scan of the part sums (parts2 <= 1024)
    scan[tid] = tid < a.parts2 ? a.sums[tid] : 0.0f;
    __syncthreads();
    for (uint32_t o = 1; o < 1024; o <<= 1) {
        const float v = tid >= o ? scan[tid - o] : 0.0f;
        __syncthreads();
        scan[tid] += v;
        __syncthreads();
    }
    const float total = scan[a.parts2 - 1];
    const float thr = st.thr_draw * total;
    if (tid == 0) {
        res[0] = a.parts2;  // first part whose running sum reaches thr
        res[1] = 0xffffffffu;
        res[2] = 0;
    }
    __syncthreads();
    if (tid < a.parts2 && thr <= scan[tid]) atomicMin(&res[0], tid);
    __syncthreads();
    const uint32_t per = (a.vocab + a.parts2 - 1) / a.parts2;
    uint32_t part = res[0];
    // Scan parts from the crossing part on until an index qualifies (the
    // crossing part normally holds it; later parts only absorb rounding).
    for (; part < a.parts2; part++) {
        const uint32_t b = part * per, e = min(a.vocab, b + per);
        const float base = part ? scan[part - 1] : 0.0f;
        const uint32_t i = b + tid;
        const float wi = i < e ? pick_weight(a, st, i, invt) : 0.0f;
        seg[tid] = wi;
        __syncthreads();
        for (uint32_t o = 1; o < 1024; o <<= 1) {
            const float v = tid >= o ? seg[tid - o] : 0.0f;
            __syncthreads();
            seg[tid] += v;
            __syncthreads();
        }
        if (i < e && wi > 0.0f && thr <= base + seg[tid]) atomicMin(&res[1], i);
        __syncthreads();
        if (res[1] != 0xffffffffu) break;
    }
    // last positive index over the whole row (rounding fallback)
    if (res[1] == 0xffffffffu) {
        uint32_t last = 0;
        for (uint32_t i = tid; i < a.vocab; i += 1024)
            if (pick_weight(a, st, i, invt) > 0.0f) last = i;
        atomicMax(&res[2], last);
        __syncthreads();
    }
    if (tid == 0) {
        const uint32_t t = res[1] != 0xffffffffu ? res[1] : res[2];
        a.out[0] = st.mode == 1 && a.bonus_ids ? a.bonus_ids[t] : t;
        a.out[1] = st.accepted;
    }
}

// ---------------------------------------------------------------------------
// Top-k / top-p sampling with a caller-supplied draw: Sampler::sample_with_draw
// (Q/src/sampler.rs:65-144) for 1 <= top_k <= 256, the bound of the CUDA
// runtime's sampler (Q/kernels/cuda/q2q4_fused_matvec_sm86.cu:2647-2776).
// Candidates are ordered by scaled logit, then by token, both descending
// (the crate's sort: ties go to the later token); a candidate is the 64-bit
// key (order-preserving bits of the scaled logit << 32) | token, so one
// integer comparison orders them. Stage 1 (one workgroup per 4096 logits)
// keeps its part's top_k keys (a radix select, no sort); stage 2 selects the
// top_k of the parts' candidates the same way, sorts only those (bitonic, in
// LDS) and one thread runs the crate's sequential arithmetic over them: exp
// weights, the nucleus cut at top_p of their sum, and the cumulative search
// of draw x the nucleus total.
// out = {token, status, nucleus length, nucleus total bits}; status 0 is
// success, 2 a non-finite logit or scaled logit, 4 an invalid normalization.
__device__ __forceinline__ uint32_t topk_key(float v) {
    const uint32_t b = __float_as_uint(v);
    return b ^ ((b & 0x80000000u) ? 0xffffffffu : 0x80000000u);
}
__device__ __forceinline__ float topk_value(uint32_t k) {
    return __uint_as_float(k ^ ((k & 0x80000000u) ? 0x80000000u : 0xffffffffu));
}

// Descending bitonic sort of n (a power of two) keys in LDS.
__device__ __forceinline__ void bitonic_desc(uint64_t *sk, uint32_t n) {
    for (uint32_t k2 = 2; k2 <= n; k2 <<= 1)
        for (uint32_t j = k2 >> 1; j > 0; j >>= 1) {
            for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
                const uint32_t ixj = i ^ j;
                if (ixj > i) {
                    const uint64_t x = sk[i], y = sk[ixj];
                    const bool desc = (i & k2) == 0;
                    if (desc ? x < y : x > y) {
                        sk[i] = y;
                        sk[ixj] = x;
                    }
                }
            }
            __syncthreads();
        }
}

// Workgroup-wide selection of the k largest of the keys the threads hold
// (N per thread; 0 marks an absent key; the keys present are distinct, the
// token being part of each, and at least k of them are present): a radix
// select over the key's bytes from the top. Each pass counts, in 256 LDS
// bins, the next byte of the keys that share the bytes fixed so far; one
// wave finds the bin holding the k-th largest; the pass that finds that bin
// holding exactly the keys still missing ends the search. Returns the
// threshold: a key is among the k largest iff (key >> shift) >= (thr >> shift).
template <int N>
__device__ __forceinline__ uint64_t topk_threshold(const uint64_t (&key)[N], uint32_t k, uint32_t *hist,
                                                   uint32_t *sel, int &shift_out) {
    uint64_t prefix = 0;
    uint32_t r = k;
    int shift = 56;
    for (;;) {
        for (uint32_t i = threadIdx.x; i < 256; i += blockDim.x) hist[i] = 0;
        __syncthreads();
#pragma unroll
        for (int n = 0; n < N; n++) {
            const bool same = shift == 56 || (key[n] >> (shift + 8)) == (prefix >> (shift + 8));
            if (key[n] != 0 && same) atomicAdd(&hist[(uint32_t)(key[n] >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (threadIdx.x < 64) {
            // Lane l holds bins 255 - 4l .. 252 - 4l (descending), so the
            // lanes' inclusive prefix sums count the keys in higher bins.
            const uint32_t l = threadIdx.x;
            uint32_t c[4], t = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                c[j] = hist[255 - 4 * l - j];
                t += c[j];
            }
            uint32_t inc = t;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t y = __shfl_up(inc, o);
                if (l >= (uint32_t)o) inc += y;
            }
            uint32_t above = inc - t;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (above < r && r <= above + c[j]) {
                    sel[0] = 255 - 4 * l - j;
                    sel[1] = above;
                    sel[2] = c[j];
                }
                above += c[j];
            }
        }
        __syncthreads();
        const uint32_t b = sel[0], above = sel[1], cnt = sel[2];
        prefix |= (uint64_t)b << shift;
        r -= above;
        if (cnt == r || shift == 0) break;
        shift -= 8;
    }
    shift_out = shift;
    return prefix;
}

// Stage 1: the top_k keys of one part (unordered; zeros past the part's
// logits when it holds fewer than top_k).
extern "C" __global__ __launch_bounds__(1024) void ctox_topk_part_gfx950(TopkArgs a) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t sel[4];
    constexpr int N = CTOX_TOPK_PART / 1024;
    const uint32_t b0 = blockIdx.x * CTOX_TOPK_PART;
    const uint32_t n = min((uint32_t)CTOX_TOPK_PART, a.vocab - b0);
    int bad = 0;
    uint64_t key[N];
#pragma unroll
    for (int j = 0; j < N; j++) {
        const uint32_t i = threadIdx.x + 1024 * j;
        key[j] = 0;  // below every candidate
        if (i < n) {
            const float x = a.logits[b0 + i], v = x * a.inv_temperature;
            bad |= !__builtin_isfinite(x) | !__builtin_isfinite(v);
            key[j] = ((uint64_t)topk_key(v) << 32) | (b0 + i);
        }
    }
    if (threadIdx.x == 0) sel[3] = 0;
    bad = __syncthreads_or(bad);
    uint64_t *out = a.cand + (size_t)blockIdx.x * a.top_k;
    if (n <= a.top_k) {
#pragma unroll
        for (int j = 0; j < N; j++) {
            const uint32_t i = threadIdx.x + 1024 * j;
            if (i < a.top_k) out[i] = key[j];
        }
    } else {
        int shift = 0;
        const uint64_t thr = topk_threshold<N>(key, a.top_k, hist, sel, shift);
#pragma unroll
        for (int j = 0; j < N; j++)
            if (key[j] != 0 && (key[j] >> shift) >= (thr >> shift)) out[atomicAdd(&sel[3], 1u)] = key[j];
    }
    if (threadIdx.x == 0) a.flags[blockIdx.x] = bad ? 1u : 0u;
}

// Stage 2: the top_k of the parts' candidates, sorted (descending key, i.e.
// scaled logit then token), then the crate's sequential arithmetic.
extern "C" __global__ __launch_bounds__(1024) void ctox_topk_final_gfx950(TopkArgs a) {
    __shared__ uint64_t sk[CTOX_TOPK_MAX];
    __shared__ float w[CTOX_TOPK_MAX];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t sel[4];
    constexpr int N = CTOX_TOPK_CANDS / 1024;
    const uint32_t n = a.parts * a.top_k;
    const uint32_t len = min(a.top_k, a.vocab);
    uint32_t n2 = 1;
    while (n2 < len) n2 <<= 1;
    int bad = 0;
    uint64_t key[N];
#pragma unroll
    for (int j = 0; j < N; j++) {
        const uint32_t i = threadIdx.x + 1024 * j;
        key[j] = i < n ? a.cand[i] : 0;
    }
    for (uint32_t p = threadIdx.x; p < a.parts; p += blockDim.x) bad |= a.flags[p] != 0;
    for (uint32_t i = threadIdx.x; i < n2; i += blockDim.x) sk[i] = 0;
    if (threadIdx.x == 0) sel[3] = 0;
    bad = __syncthreads_or(bad);
    if (bad) {
        if (threadIdx.x == 0) {
            a.out[0] = 0xffffffffu;
            a.out[1] = 2;
            a.out[2] = 0;
            a.out[3] = 0;
        }
        return;
    }
    int shift = 0;
    const uint64_t kthr = topk_threshold<N>(key, len, hist, sel, shift);
#pragma unroll
    for (int j = 0; j < N; j++)
        if (key[j] != 0 && (key[j] >> shift) >= (kthr >> shift)) sk[atomicAdd(&sel[3], 1u)] = key[j];
    __syncthreads();
    bitonic_desc(sk, n2);
    if (threadIdx.x != 0) return;
    // Sampler::sample_with_draw from the sort on, in its order of operations.
    const float m = topk_value((uint32_t)(sk[0] >> 32));
    float norm = 0.0f;
    for (uint32_t r = 0; r < len; r++) {
        w[r] = expf(topk_value((uint32_t)(sk[r] >> 32)) - m);
        norm += w[r];
    }
    if (!__builtin_isfinite(norm) || norm <= 0.0f) {
        a.out[0] = 0xffffffffu;
        a.out[1] = 4;
        a.out[2] = 0;
        a.out[3] = 0;
        return;
    }
    const float cut = a.top_p * norm;
    float cum = 0.0f;
    uint32_t nuc = len;
    for (uint32_t r = 0; r < len; r++) {
        cum += w[r];
        if (cum >= cut) {
            nuc = r + 1;
            break;
        }
    }
    float total = 0.0f;
    for (uint32_t r = 0; r < nuc; r++) total += w[r];
    const float thr = a.draw * total;
    cum = 0.0f;
    uint32_t tok = (uint32_t)sk[nuc - 1];
    for (uint32_t r = 0; r < nuc; r++) {
        cum += w[r];
        if (thr <= cum) {
            tok = (uint32_t)sk[r];
            break;
        }
    }
    a.out[0] = tok;
    a.out[1] = 0;
    a.out[2] = nuc;
    a.out[3] = __float_as_uint(total);
}
