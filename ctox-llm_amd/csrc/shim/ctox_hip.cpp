// Host side of the C ABI declared in include/ctox_hip.h.
//
// A thin launcher over the HIP module API: the gfx950 code object built from
// csrc/kernels is embedded in this library, loaded with hipModuleLoadData at
// backend creation, and every kernel is started with hipModuleLaunchKernel
// with a single by-value argument block (csrc/kernels/kernel_args.h). This
// mirrors the role of the reference's driver-API runtime
// (Q/src/backend/cuda_runtime.rs:195-294, 1297-1371), not its structure.
//
// Validation restates the crate's CPU dispatcher contract
// (Q/src/backend/cpu.rs:41-173, 312-337, 478-490; Q/src/reference.rs:18-34,
// 241-263, 387-396) so that errors match kind for kind. There is no CPU
// fallback anywhere in this file: a missing device or code object fails
// closed with CTOX_ERR_UNSUPPORTED_OPERATION.
#include "ctox_hip.h"
#include "shim_internal.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../kernels/kernel_args.h"

// Static scratch of the allocation-free entry point (noalloc.hip).
extern "C" ctox_status ctox_noalloc_setup(int device);
extern "C" ctox_status ctox_noalloc_slots(int device, void *stream, uint64_t **ptr, size_t *bytes, uint32_t *seq,
                                          uint32_t **arrive, size_t *arrive_n);

// ---- embedded gfx950 code object ----
extern "C" const unsigned char ctox_hsaco_begin[];
extern "C" const unsigned char ctox_hsaco_end[];
__asm__(".section .rodata\n"
        ".balign 64\n"
        ".global ctox_hsaco_begin\n"
        "ctox_hsaco_begin:\n"
        ".incbin \"" CTOX_HSACO_PATH "\"\n"
        ".global ctox_hsaco_end\n"
        "ctox_hsaco_end:\n"
        ".byte 0\n"
        ".previous\n");

namespace {

thread_local std::string g_last_error;

ctox_status fail(ctox_status st, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return st;
}

#define HIP_TRY(expr)                                                                          \
    do {                                                                                       \
        hipError_t e_ = (expr);                                                                \
        if (e_ != hipSuccess)                                                                  \
            return fail(CTOX_ERR_INVALID_STATE, "HIP call %s failed: %s", #expr,               \
                        hipGetErrorString(e_));                                                \
    } while (0)

constexpr size_t kBlockLen = CTOX_BLOCK_LEN;

size_t block_bytes(int32_t dtype) {
    return dtype == CTOX_DTYPE_Q2B64 ? CTOX_Q2_BLOCK_BYTES
                                     : (dtype == CTOX_DTYPE_Q4B64 ? CTOX_Q4_BLOCK_BYTES : 0);
}

float f16_bits_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1f, man = h & 0x3ff, bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            int e = -1;
            do {
                man <<= 1;
                e++;
            } while ((man & 0x400) == 0);
            bits = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3ff) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

bool scale_finite(const ctox_scale_slice &s, size_t *bad) {
    for (size_t i = 0; i < s.len; i++) {
        float v = s.kind == CTOX_SCALE_F32
                      ? ((const float *)s.data)[i]
                      : f16_bits_to_f32((uint16_t)(((const uint8_t *)s.data)[2 * i] |
                                                   (((const uint8_t *)s.data)[2 * i + 1] << 8)));
        if (!std::isfinite(v)) {
            *bad = i;
            return false;
        }
    }
    return true;
}

// Checks every packed block scale of `rows` rows (the CPU dispatcher rejects
// a non-finite scale with InvalidArtifact while it walks the row,
// Q/src/backend/cpu.rs:185-190; a device kernel cannot fail per block, so the
// host checks up front).
bool block_scales_finite(const uint8_t *w, size_t rows, size_t blocks, size_t bb) {
    for (size_t r = 0; r < rows * blocks; r++) {
        const uint8_t *blk = w + r * bb;
        if (!std::isfinite(f16_bits_to_f32((uint16_t)(blk[0] | (blk[1] << 8))))) return false;
    }
    return true;
}

struct DevBuf {
    void *ptr = nullptr;
    size_t bytes = 0;
};

}  // namespace

// A matrix segment rewritten into the tiled layout (kernel_args.h).
struct TiledCopy {
    void *d = nullptr;
    uint32_t tiles = 0, chunks = 0, rows = 0, columns = 0;
};

struct ctox_hip_backend {
    int device = 0;
    char arch[64] = {0};
    hipModule_t module = nullptr;
    hipStream_t stream = nullptr;
    hipFunction_t prep = nullptr, q4_b1 = nullptr, q4_b4 = nullptr, q4_b8 = nullptr, q2_b1 = nullptr,
                  q2_b4 = nullptr, q2_b8 = nullptr, rec_row = nullptr, row_dot = nullptr,
                  gdn_scan = nullptr, gdn_chunk_prep = nullptr, gdn_chunk_scan = nullptr, gdn_chunk_scan_vec = nullptr, gates = nullptr,
                  repeat = nullptr, partials = nullptr, argmax_final = nullptr, greedy_status = nullptr, verify = nullptr, decide = nullptr,
                  pick_sums = nullptr, pick_final = nullptr, rms = nullptr, swiglu = nullptr, sgate = nullptr,
                  conv = nullptr, rope = nullptr, kv_pack = nullptr, attn_prep = nullptr, kv_demote = nullptr, gqa_part[2] = {}, gqa_part16[2] = {},
                  gqa_combine = nullptr, fill = nullptr, embed = nullptr, norm_rows = nullptr, attn_gate = nullptr,
                  swiglu_rows = nullptr, copy_rows = nullptr, write_words = nullptr, norm_prep = nullptr,
                  prep_x = nullptr, finite = nullptr, gather = nullptr, topk_part = nullptr, topk_final = nullptr, stream_read = nullptr,
                  write_segments = nullptr;
    // Batch-1 slice kernels per dtype [Q2, Q4]: [0] walks the slices, [n]
    // requests all n slices up front (n <= 3: more slices up front measured
    // slower than walking them).
    hipFunction_t sl[2][4] = {};
    // Small-M slice kernels per dtype [Q2, Q4]: [0] M = 2..4, [1] M = 5..8.
    hipFunction_t st[2][2] = {};
    // Tiled-layout batch-1 kernels per dtype [Q2, Q4] and row tiles per wave
    // (1..4), and the prepare-time repack.
    hipFunction_t tile[2][CTOX_TILE_MAXU] = {};
    // The same with the activation fragments built inside the kernel, one
    // kernel per input transform T (xmode 0..4; 5: the residual norm with
    // the producer's sums of squares): [T][q4][u - 1].
    hipFunction_t tilex[6][2][CTOX_TILE_MAXU] = {};
    // Combine by arrival: [kind][q4][u - 1], kind 0 staged, 1 + T built.
    hipFunction_t tile_arr[7][2][CTOX_TILE_MAXU] = {};
    hipFunction_t tilem[2][7] = {};      // [q4][rows - 2], 2..8 staged rows
    hipFunction_t tilem_arr[2][7] = {};  // combine by arrival
    // The same building the rows' fragments in the kernel, per row count 2..5.
    hipFunction_t tilemx[2][4] = {};
    hipFunction_t tilemx_arr[2][4] = {};  // combine by arrival
    uint64_t mx_max = (uint64_t)8 << 20;  // CTOX_MX_MAX (Mi): largest matrix the small-M launch builds rows for
    bool no_mx = false;
    bool noalloc_ok = false;  // the static scratch of ctox_hip_launch_fused_matvec_noalloc is set up
    hipFunction_t repack = nullptr;
    hipFunction_t gdn_fused = nullptr, gdn_fused_blk = nullptr;
    hipFunction_t gdn_fused1 = nullptr, gdn_fused1_blk = nullptr;  // one row
    hipFunction_t gdn_k4[2][2] = {};  // [one row][blocked]: conv kernel size 4
    bool gdn_one = true;  // CTOX_GDN_ONE=0: the one-row step runs the row-block kernel
    int cus = 0;
    uint32_t tile_u = 0;  // CTOX_TILE_U: fixed row tiles per wave (0 = planned)
    int arrive = -1;      // CTOX_ARRIVE: 1 / 0 forces the tiled combine by arrival / by the last chunk
    uint32_t tile_cap[7][2][CTOX_TILE_MAXU] = {};  // [kind][q4][u - 1]: workgroups resident at once
    uint32_t tilem_cap[2][7] = {};                  // [q4][rows - 2], same for the small-M kernels
    uint32_t tilemx_cap[2][4] = {};                 // [q4][rows - 2]
    // Tiled matvec chunk partials (64-bit slots tagged with a launch sequence
    // number; zeroed when allocated) and the last sequence number used.
    DevBuf tpart;
    DevBuf tarrive;  // batch-1 per-tile arrival counts (zero between launches)
    uint32_t tile_seq = 0;
    // Tiled copies of raw device weights (ctox_hip_register_tiled_weights).
    std::unordered_map<const void *, TiledCopy> raw_tiled;
    // Activation staging (two layouts: [0] Q2, [1] Q4) and gated-delta norms.
    DevBuf xa[2], xc[2], norms;
    // Next-norm staging written by a small-M residual producer for the
    // projection that follows it (separate from xa/xc, which the producer reads).
    DevBuf xn[2], xnc[2];
    // Token selection scratch: per-part partials, pick sums and state.
    DevBuf tok, stats;
    // Split-attention partials.
    DevBuf attn;
    // The scratch above is one set per backend: the stream of the previous
    // call (compared, never used), see pick_stream.
    hipStream_t last = nullptr;
    bool used = false;
};

struct ctox_hip_matrix {
    ctox_hip_backend *backend = nullptr;
    int32_t dtype = 0;
    size_t rows = 0, columns = 0;
    std::vector<ctox_quant_segment> segments;  // pure matrices hold one synthetic segment
    void *d_weights = nullptr;
    size_t weights_len = 0;
    void *d_s_in = nullptr;
    uint32_t s_in_kind = CTOX_KSCALE_NONE;
    void *d_s_out = nullptr;
    uint32_t s_out_kind = CTOX_KSCALE_NONE;
    float *d_bias = nullptr;
    uint32_t activation = 0;
    std::vector<uint8_t> s_in_host;  // exact s_in bytes, for fan-out sharing checks
    // Per segment: the same rows rewritten into the tiled layout (kernel_args.h).
    using Tiled = TiledCopy;
    std::vector<Tiled> tiled;
};

namespace {

ctox_status ensure(ctox_hip_backend *b, DevBuf &buf, size_t bytes, bool zero) {
    if (buf.bytes >= bytes) return CTOX_OK;
    // Grow: work queued on any stream may still read the old buffer.
    HIP_TRY(hipDeviceSynchronize());
    if (buf.ptr) HIP_TRY(hipFree(buf.ptr));
    buf.ptr = nullptr;
    buf.bytes = 0;
    size_t want = bytes < 4096 ? 4096 : bytes;
    HIP_TRY(hipMalloc(&buf.ptr, want));
    if (zero) {
        HIP_TRY(hipMemset(buf.ptr, 0, want));
        HIP_TRY(hipDeviceSynchronize());
    }
    buf.bytes = want;
    (void)b;
    return CTOX_OK;
}

template <typename Args>
ctox_status launch(hipFunction_t f, dim3 grid, dim3 block, hipStream_t s, Args args,
                   const char *name) {
    void *params[] = {&args};
    hipError_t e = hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, 0, s,
                                         params, nullptr);
    if (e != hipSuccess)
        return fail(CTOX_ERR_INVALID_STATE, "launch of %s failed: %s", name, hipGetErrorString(e));
    return CTOX_OK;
}

// Device entry points run on the caller's stream exactly as given; NULL is
// HIP's null stream, as everywhere in the HIP API. The backend's scratch
// (activation staging, combine slots, selection statistics) is one set per
// backend, so a call on a stream other than the previous call's first waits
// on the host until the device has drained: the previous stream may already
// be destroyed, so its handle is never used again. Calls that stay on one
// stream (the decode engine, a serving loop) never wait.
hipStream_t pick_stream(ctox_hip_backend *b, void *sv) {
    hipStream_t s = (hipStream_t)sv;
    if (!b) return s;
    if (b->used && s != b->last) (void)hipDeviceSynchronize();
    b->last = s;
    b->used = true;
    return s;
}

// Q/src/backend/cpu.rs:41-173 (same order of checks and error kinds).
ctox_status validate_matvec(const ctox_fused_matvec *op, bool need_input, size_t *bpr) {
    if (op->columns == 0 || op->rows == 0 || op->columns % kBlockLen != 0)
        return fail(CTOX_ERR_SHAPE,
                    "Q2/Q4 fused matvec dimensions must be non-zero and columns divisible by 64");
    if (need_input && op->input_len != op->columns)
        return fail(CTOX_ERR_SHAPE, "input has %zu, expected %zu values", op->input_len, op->columns);
    if (op->s_in.kind != CTOX_SCALE_NONE && op->s_in.len != op->columns)
        return fail(CTOX_ERR_SHAPE, "s_in length differs from columns");
    if (op->s_out.kind != CTOX_SCALE_NONE && op->s_out.len != op->rows)
        return fail(CTOX_ERR_SHAPE, "s_out length differs from rows");
    if (op->bias && op->bias_len != op->rows)
        return fail(CTOX_ERR_SHAPE, "bias length differs from rows");
    const size_t blocks = op->columns / kBlockLen;
    if (op->dtype == CTOX_DTYPE_Q2B64 || op->dtype == CTOX_DTYPE_Q4B64) {
        if (op->n_segments)
            return fail(CTOX_ERR_INVALID_ARTIFACT, "pure Q2/Q4 operation declares mixed row segments");
        const size_t expected = op->rows * blocks * block_bytes(op->dtype);
        if (op->weights_len != expected)
            return fail(CTOX_ERR_SHAPE, "weight buffer has %zu bytes, expected %zu", op->weights_len,
                        expected);
        *bpr = blocks;
        return CTOX_OK;
    }
    if (op->dtype != CTOX_DTYPE_MIXED_Q2Q4B64)
        return fail(CTOX_ERR_UNSUPPORTED_DTYPE, "unsupported quantization dtype %d", op->dtype);
    if (op->n_segments == 0)
        return fail(CTOX_ERR_INVALID_ARTIFACT, "mixed Q2/Q4 operation has no row segments");
    uint64_t row = 0, off = 0;
    for (size_t g = 0; g < op->n_segments; g++) {
        const ctox_quant_segment &s = op->segments[g];
        if (s.group_index != g || s.row_start != row || s.row_end <= s.row_start ||
            s.row_end > op->rows || s.offset != off)
            return fail(CTOX_ERR_INVALID_ARTIFACT, "mixed Q2/Q4 operation has non-contiguous segment %u",
                        s.group_index);
        const size_t sb = block_bytes(s.dtype);
        if (!sb)
            return fail(CTOX_ERR_INVALID_ARTIFACT, "mixed Q2/Q4 segment %u has invalid dtype %d",
                        s.group_index, s.dtype);
        const uint64_t expected = (s.row_end - s.row_start) * blocks * sb;
        if (s.length != expected)
            return fail(CTOX_ERR_INVALID_ARTIFACT, "mixed Q2/Q4 segment %u has %llu bytes, expected %llu",
                        s.group_index, (unsigned long long)s.length, (unsigned long long)expected);
        row = s.row_end;
        off += s.length;
    }
    if (row != op->rows || off != op->weights_len)
        return fail(CTOX_ERR_SHAPE, "mixed segments cover %llu/%zu rows and %llu/%zu bytes",
                    (unsigned long long)row, op->rows, (unsigned long long)off, op->weights_len);
    *bpr = blocks;
    return CTOX_OK;
}

ctox_status check_matrix_scales(const ctox_fused_matvec *op, size_t blocks) {
    size_t bad;
    if (op->s_in.kind != CTOX_SCALE_NONE && !scale_finite(op->s_in, &bad))
        return fail(CTOX_ERR_INVALID_ARTIFACT, "recovery scale %zu is non-finite", bad);
    if (op->s_out.kind != CTOX_SCALE_NONE && !scale_finite(op->s_out, &bad))
        return fail(CTOX_ERR_INVALID_ARTIFACT, "recovery scale %zu is non-finite", bad);
    if (op->dtype != CTOX_DTYPE_MIXED_Q2Q4B64) {
        if (!block_scales_finite(op->weights, op->rows, blocks, block_bytes(op->dtype)))
            return fail(CTOX_ERR_INVALID_ARTIFACT, "%s block scale is non-finite",
                        op->dtype == CTOX_DTYPE_Q2B64 ? "Q2" : "Q4");
    } else {
        for (size_t g = 0; g < op->n_segments; g++) {
            const ctox_quant_segment &s = op->segments[g];
            if (!block_scales_finite(op->weights + s.offset, s.row_end - s.row_start, blocks,
                                     block_bytes(s.dtype)))
                return fail(CTOX_ERR_INVALID_ARTIFACT, "%s block scale is non-finite",
                            s.dtype == CTOX_DTYPE_Q2B64 ? "Q2" : "Q4");
        }
    }
    return CTOX_OK;
}

ctox_status upload(const void *host, size_t bytes, void **dev) {
    *dev = nullptr;
    if (!bytes) return CTOX_OK;
    HIP_TRY(hipMalloc(dev, bytes));
    HIP_TRY(hipMemcpy(*dev, host, bytes, hipMemcpyHostToDevice));
    return CTOX_OK;
}

uint32_t kernel_scale_kind(int32_t kind) {
    return kind == CTOX_SCALE_F32 ? CTOX_KSCALE_F32
                                  : (kind == CTOX_SCALE_F16LE ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE);
}

size_t packed_row_bytes(int32_t dtype, size_t columns) { return columns / kBlockLen * block_bytes(dtype); }

// Converts `batch` activation rows into the MFMA A-fragment layout `layout`
// (0 = Q2 element order, 1 = Q4 element order).
ctox_status run_prep(ctox_hip_backend *b, int layout, const float *d_input, size_t columns,
                     size_t batch, const void *d_s_in, uint32_t s_in_kind, hipStream_t s) {
    const size_t blocks = columns / kBlockLen;
    const size_t tgroups = (batch + 3) / 4;
    ctox_status st = ensure(b, b->xa[layout], blocks * batch * 192, false);
    if (!st) st = ensure(b, b->xc[layout], blocks * batch * 4 * sizeof(float), false);
    if (st) return st;
    PrepArgs a{};
    a.input = d_input;
    a.s_in = d_s_in;
    a.xa = (int8_t *)b->xa[layout].ptr;
    a.xc = (float *)b->xc[layout].ptr;
    a.columns = (uint32_t)columns;
    a.batch = (uint32_t)batch;
    a.dtype = (uint32_t)layout;
    a.s_in_kind = s_in_kind;
    a.tgroups = (uint32_t)tgroups;
    return launch(b->prep, dim3((unsigned)blocks, (unsigned)batch), dim3(64), s, a,
                  "ctox_prep_activation_gfx950");
}

// Input transform of the in-kernel fragment build (TileMatvecArgs::xmode).
struct TileXform {
    uint32_t xmode = 0;
    const float *b = nullptr, *w = nullptr, *delta = nullptr;
    float *x_out = nullptr, *norm_out = nullptr;
    uint32_t off = 0, head_dim = 0;
    float eps = 0.0f;
    const float *res_h = nullptr;  // producer: residual the output is added to
    float *res_sq = nullptr;       // producer: per-tile sums of (res_h + out)^2
    const float *sq_in = nullptr;  // consumer (xmode 1): those sums
    uint32_t sq_n = 0;
    bool parts_out = false;        // batch 1: chunk partials to output [chunks][rows]
    uint32_t a_parts = 0, a_pstride = 0;  // xmode 2: input as producer chunk partials
    uint32_t a_stride = 0, b_stride = 0;  // small M: floats between rows of the input and of b / delta
};

// Caller-provided combine slots (the allocation-free entry point's static
// device scratch) in place of the backend's grown buffer, with their tag.
struct PartialSlots {
    uint64_t *p = nullptr;
    size_t bytes = 0;
    uint32_t seq = 0;
    uint32_t *arrive = nullptr;  // batch-1 arrival counts
    size_t arrive_n = 0;
};

// Small-M rows the in-kernel fragment build takes (ctox_q*_mv_tilemx*).
constexpr size_t kMaxBuildRows = 5;
size_t max_build_rows(const ctox_hip_backend *b) { return b->no_mx ? 1 : kMaxBuildRows; }
// Every workgroup of a chunk rebuilds the chunk's rows (5 rows: about 3 us
// per workgroup, measured per wave), so the in-kernel build pays off only
// for small matrices, up to 8 Mi weights. Staged rows measured faster from
// o_proj / out_proj (5120 x 6144, 5 rows: 12.3 us built in the kernel
// against 9.2 us + the staging launch; the 27B MTP step 7.50 against 7.35 ms)
// upwards.
bool build_in_kernel(const ctox_hip_backend *b, size_t batch, size_t rows, size_t columns) {
    return batch >= 2 && batch <= max_build_rows(b) && (uint64_t)rows * columns <= b->mx_max;
}

ctox_status run_tile_matvec(ctox_hip_backend *b, int32_t dtype, const TiledCopy &t, size_t rows, size_t columns,
                            const void *d_s_out, uint32_t s_out_kind, const float *d_bias, float *d_output, uint32_t act,
                            hipStream_t s, const float *d_input = nullptr, const void *d_s_in = nullptr,
                            uint32_t s_in_kind = CTOX_KSCALE_NONE, const TileXform *xf = nullptr,
                            const PartialSlots *ps = nullptr);

// Staging of the next (1 + w) RMS-normed projection by a small-M residual
// producer (TileMatvecArgs::nx_xa): the next norm weight, the next matrix's
// f16 s_in and packed dtype, where h = residual + output goes, and where the
// per-block sums of h^2 go ([batch][rows / 64]).
struct NextNorm {
    const float *w = nullptr;
    const uint16_t *s_in = nullptr;
    int32_t dtype = 0;
    float *h_out = nullptr;
    float *sq_out = nullptr;
};

// Staged input of a small-M launch other than the backend's xa/xc, with
// the consumer side of a next-norm staging (rms_sq: per-block sums of h^2).
struct StagedIn {
    const int8_t *xa = nullptr;
    const float *xc = nullptr;
    const float *rms_sq = nullptr;
    uint32_t rms_n = 0;
    float eps = 0.0f;
};

ctox_status run_tile_matvec_m(ctox_hip_backend *b, int32_t dtype, const TiledCopy &t, size_t rows, size_t columns,
                              size_t batch, const void *d_s_out, uint32_t s_out_kind, const float *d_bias,
                              float *d_output, size_t out_stride, uint32_t act, hipStream_t s,
                              const float *res_h = nullptr, float *res_sq = nullptr, bool parts_out = false,
                              const NextNorm *nx = nullptr, bool *staged = nullptr, const StagedIn *in = nullptr);

ctox_status run_tile_matvec_mx(ctox_hip_backend *b, int32_t dtype, const TiledCopy &t, size_t rows, size_t columns,
                               size_t batch, const void *d_s_out, uint32_t s_out_kind, const float *d_bias,
                               float *d_output, size_t out_stride, uint32_t act, hipStream_t s, const float *d_input,
                               const void *d_s_in, uint32_t s_in_kind, const TileXform &xf,
                               const PartialSlots *ps = nullptr);

// One launch over `rows` packed rows of one dtype (a pure matrix or one
// mixed segment), output rows written at d_output[m*out_stride + r], with
// the activation already staged in `layout`.
// split: split K into one partial per slice where the batch-1 slice kernel
// applies (outputs [parts][rows]; *parts reports the count, 1 otherwise).
ctox_status run_matvec(ctox_hip_backend *b, int layout, int32_t dtype, const void *d_weights, size_t rows,
                       size_t columns, size_t batch, const void *d_s_out, uint32_t s_out_kind,
                       const float *d_bias, float *d_output, size_t out_stride, uint32_t act,
                       hipStream_t s, bool split = false, uint32_t *parts = nullptr, const float *res_h = nullptr,
                       float *res_sq = nullptr, const NextNorm *nx = nullptr, bool *staged = nullptr) {
    if (parts) *parts = 1;
    const size_t groups = (rows + CTOX_MV_ROWS - 1) / CTOX_MV_ROWS;
    const size_t tgroups = (batch + 3) / 4;
    if (groups > 0x7fffffffu) return fail(CTOX_ERR_SHAPE, "matrix too large for one launch");
    MatvecArgs a{};
    a.weights = (const uint8_t *)d_weights;
    a.weights_len = (uint64_t)rows * packed_row_bytes(dtype, columns);
    a.xa = (const int8_t *)b->xa[layout].ptr;
    a.xc = (const float *)b->xc[layout].ptr;
    a.s_out = d_s_out;
    a.bias = d_bias;
    a.output = d_output;
    a.rows = (uint32_t)rows;
    a.columns = (uint32_t)columns;
    a.batch = (uint32_t)batch;
    a.out_stride = (uint32_t)out_stride;
    a.s_out_kind = s_out_kind;
    a.activation = act;
    const bool q4 = dtype == CTOX_DTYPE_Q4B64;
    // Registered raw weights: the tiled kernels over the staged activation.
    if (!b->raw_tiled.empty()) {
        auto it = b->raw_tiled.find(d_weights);
        if (it != b->raw_tiled.end() && it->second.rows == rows && it->second.columns == columns)
            return batch == 1 ? run_tile_matvec(b, dtype, it->second, rows, columns, d_s_out, s_out_kind, d_bias,
                                                d_output, act, s)
                              : run_tile_matvec_m(b, dtype, it->second, rows, columns, batch, d_s_out, s_out_kind,
                                                  d_bias, d_output, out_stride, act, s, res_h, res_sq, false, nx,
                                                  staged);
    }
    // Batch 1 on rows of whole 16-byte units: the slice kernels (all slices
    // requested up front when there are at most three, else walked).
    const size_t rb = packed_row_bytes(dtype, columns);
    if (batch == 1 && rb % 16 == 0 && ((uintptr_t)d_weights & 15) == 0) {
        const size_t ns = (columns / kBlockLen + ctox_slice_blocks(q4) - 1) / ctox_slice_blocks(q4);
        // Split K for tile counts that leave CUs idle: two slices per part.
        if (split && ns > 2 && !d_bias && act == 0 && ns <= 65535 && groups < 2 * (size_t)b->cus) {
            const uint32_t np = (uint32_t)((ns + 1) / 2);
            a.part_stride = (uint32_t)rows;
            if (parts) *parts = np;
            return launch(b->sl[q4 ? 1 : 0][2], dim3((unsigned)groups, np), dim3(CTOX_SLICE_WAVES * 64), s, a,
                          "ctox_q*_matvec_sl2_gfx950");
        }
        hipFunction_t f = b->sl[q4 ? 1 : 0][ns <= 3 ? ns : 0];
        return launch(f, dim3((unsigned)groups), dim3(CTOX_SLICE_WAVES * 64), s, a, "ctox_q*_matvec_sl*_gfx950");
    }
    if (batch >= 2 && rb % 16 == 0 && ((uintptr_t)d_weights & 15) == 0) {
        hipFunction_t f = b->st[q4 ? 1 : 0][tgroups == 1 ? 0 : 1];
        return launch(f, dim3((unsigned)groups), dim3(CTOX_SLICE_WAVES * 64), s, a, "ctox_q*_matvec_st*_gfx950");
    }
    hipFunction_t f = q4 ? (batch == 1 ? b->q4_b1 : (tgroups == 1 ? b->q4_b4 : b->q4_b8))
                         : (batch == 1 ? b->q2_b1 : (tgroups == 1 ? b->q2_b4 : b->q2_b8));
    return launch(f, dim3((unsigned)groups), dim3(256), s, a, "ctox_q*_matvec_gfx950");
}

// Tag of the next tiled launch's partial slots: never 0 (the value of a
// freshly zeroed slot) and never one still present in the buffer (on wrap
// the slots are zeroed again).
uint32_t next_tile_seq(ctox_hip_backend *b) {
    if (++b->tile_seq == 0) {
        if (b->tpart.ptr) {
            (void)hipDeviceSynchronize();
            (void)hipMemset(b->tpart.ptr, 0, b->tpart.bytes);
            (void)hipDeviceSynchronize();
        }
        b->tile_seq = 1;
    }
    return b->tile_seq;
}

// One launch of the tiled batch-1 matvec over a prepared segment. Plan: the
// chunks x tiles units are spread so that one pass of about twelve waves per
// CU covers them, at most CTOX_TILE_MAXU row tiles per wave. With d_input
// set the kernel builds the activation fragments itself (no prep launch);
// otherwise it reads the ones staged in the backend's xa/xc.
ctox_status run_tile_matvec(ctox_hip_backend *b, int32_t dtype, const TiledCopy &t, size_t rows,
                            size_t columns, const void *d_s_out, uint32_t s_out_kind, const float *d_bias,
                            float *d_output, uint32_t act, hipStream_t s, const float *d_input,
                            const void *d_s_in, uint32_t s_in_kind, const TileXform *xf, const PartialSlots *ps) {
    const int q4 = dtype == CTOX_DTYPE_Q4B64 ? 1 : 0;
    const size_t units = (size_t)t.tiles * t.chunks;
    // Row tiles per wave: enough that the launch has about 16 units per CU
    // (measured on the 27B decode step against 12 / 20 / 24 per CU: 16 gives
    // gate|up three tiles per wave instead of four and keeps the
    // in-projections at two; 4.12 against 4.15 ms per token).
    const size_t slots = (size_t)(b->cus > 0 ? b->cus : 256) * 16;
    uint32_t u = b->tile_u ? b->tile_u : (uint32_t)std::min<size_t>(CTOX_TILE_MAXU, std::max<size_t>(1, (units + slots - 1) / slots));
    uint32_t segs = (t.tiles + u - 1) / u;
    // The in-kernel fragment build shares one chunk per workgroup of four waves.
    if (d_input) segs = (segs + 3) & ~3u;
    const size_t waves = (size_t)segs * t.chunks;
    if ((waves + 3) / 4 > 0x7fffffffu) return fail(CTOX_ERR_SHAPE, "matrix too large for one launch");
    // Chunks meet in one of two ways. When every workgroup of the launch is
    // resident at once, the last chunk's waves combine (they wait only for
    // resident producers, whatever the dispatch order). Otherwise by
    // arrival: every chunk stores its partial and counts itself in, and the
    // last to arrive for a tile combines, waiting only for chunks that have
    // already arrived.
    const bool combine = t.chunks > 1 && !(xf && xf->parts_out);
    const size_t wgs = ((size_t)segs * t.chunks + 3) / 4;
    // kind: 0 staged fragments, else 1 + the input transform of the build
    // (5: the residual norm with the producer's sums of squares).
    const uint32_t xm = xf ? xf->xmode : 0u;
    const int kind = !d_input ? 0 : 1 + (xm == 1 && xf->sq_in && xf->sq_n ? 5 : (int)xm);
    const bool arrive = combine && (b->arrive >= 0 ? b->arrive != 0 : wgs > b->tile_cap[kind][q4][u - 1]);
    const size_t slot_bytes = (size_t)(arrive ? t.chunks : t.chunks - 1) * t.tiles * CTOX_TILE_ROWS * sizeof(uint64_t);
    if (ps && combine && (slot_bytes > ps->bytes || (arrive && t.tiles > ps->arrive_n)))
        return fail(CTOX_ERR_MEMORY_BUDGET, "combine slots need %zu bytes, the static scratch holds %zu", slot_bytes,
                    ps->bytes);
    if (combine && !ps) {
        ctox_status st = ensure(b, b->tpart, slot_bytes, true);
        if (!st && arrive) st = ensure(b, b->tarrive, (size_t)t.tiles * sizeof(uint32_t), true);
        if (st) return st;
    }
    TileMatvecArgs a{};
    a.arrive = arrive ? (ps ? ps->arrive : (uint32_t *)b->tarrive.ptr) : nullptr;
    a.weights = (const uint8_t *)t.d;
    a.xa = (const int8_t *)b->xa[q4].ptr;
    a.xc = (const float *)b->xc[q4].ptr;
    a.s_out = d_s_out;
    a.bias = d_bias;
    a.output = d_output;
    a.partial = ps ? ps->p : (uint64_t *)b->tpart.ptr;
    a.seq = ps ? ps->seq : next_tile_seq(b);
    a.rows = (uint32_t)rows;
    a.blocks = (uint32_t)(columns / kBlockLen);
    a.tiles = t.tiles;
    a.chunks = t.chunks;
    a.segs = segs;
    a.tpw = u;
    a.s_out_kind = s_out_kind;
    a.activation = act;
    a.input = d_input;
    a.s_in = d_s_in;
    a.s_in_kind = s_in_kind;
    if (xf) {
        a.xmode = xf->xmode;
        a.xb = xf->b;
        a.xw = xf->w;
        a.delta = xf->delta;
        a.x_out = xf->x_out;
        a.norm_out = xf->norm_out;
        a.off = xf->off;
        a.head_dim = xf->head_dim;
        a.eps = xf->eps;
        a.res_h = xf->res_h;
        a.res_sq = xf->res_sq;
        a.sq_in = xf->sq_in;
        a.sq_n = xf->sq_in ? xf->sq_n : 0u;
        a.parts_out = xf->parts_out && t.chunks > 1 ? 1u : 0u;
        a.out_stride = (uint32_t)rows;  // part stride of parts_out
        a.a_parts = xf->a_parts;
        a.a_pstride = xf->a_pstride;
    }
    hipFunction_t f = arrive ? b->tile_arr[kind][q4][u - 1]
                             : (kind ? b->tilex[kind - 1][q4][u - 1] : b->tile[q4][u - 1]);
    return launch(f, dim3((unsigned)((waves + 3) / 4)), dim3(256), s, a, "ctox_q*_mv_tile*_gfx950");
}

// One launch of the small-M tiled matvec (2..8 rows staged in xa/xc).
// parts_out: chunk partials [chunk][batch][out_stride] instead of the combine.
ctox_status run_tile_matvec_m(ctox_hip_backend *b, int32_t dtype, const TiledCopy &t, size_t rows, size_t columns,
                              size_t batch, const void *d_s_out, uint32_t s_out_kind, const float *d_bias,
                              float *d_output, size_t out_stride, uint32_t act, hipStream_t s, const float *res_h,
                              float *res_sq, bool parts_out, const NextNorm *nx, bool *staged, const StagedIn *in) {
    if (staged) *staged = false;
    const int q4 = dtype == CTOX_DTYPE_Q4B64 ? 1 : 0;
    const uint32_t u = 1;
    const uint32_t segs = (((t.tiles + u - 1) / u) + 3) & ~3u;
    const size_t waves = (size_t)segs * t.chunks;
    if (batch < 2 || batch > 8) return fail(CTOX_ERR_SHAPE, "small-M launch takes 2..8 rows");
    if (waves / 4 > 0x7fffffffu || out_stride > 0xffffffffu) return fail(CTOX_ERR_SHAPE, "matrix too large for one launch");
    // Chunks meet as in the batch-1 launch: by the last chunk when the
    // device holds every workgroup at once, else by arrival.
    parts_out = parts_out && t.chunks > 1;
    const bool arrive =
        t.chunks > 1 && !parts_out && (b->arrive >= 0 ? b->arrive != 0 : waves / 4 > b->tilem_cap[q4][batch - 2]);
    if (t.chunks > 1 && !parts_out) {
        // (five rows: the last chunk stores its fifth-row partial too)
        const size_t slot_chunks = arrive || batch == 5 ? t.chunks : t.chunks - 1;
        ctox_status st = ensure(b, b->tpart, slot_chunks * batch * t.tiles * CTOX_TILE_ROWS * sizeof(uint64_t), true);
        if (!st && arrive) st = ensure(b, b->tarrive, (size_t)t.tiles * sizeof(uint32_t), true);
        if (st) return st;
    }
    TileMatvecArgs a{};
    a.arrive = arrive ? (uint32_t *)b->tarrive.ptr : nullptr;
    a.weights = (const uint8_t *)t.d;
    a.xa = in && in->xa ? in->xa : (const int8_t *)b->xa[q4].ptr;
    a.xc = in && in->xc ? in->xc : (const float *)b->xc[q4].ptr;
    if (in && in->rms_sq) {
        a.rms_sq = in->rms_sq;
        a.rms_n = in->rms_n;
        a.eps = in->eps;
    }
    // Next-norm staging: the last chunk's workgroups hold whole 64-row blocks
    // (one tile per wave, four waves, rows a multiple of 64).
    if (nx && res_h && res_sq && !arrive && !parts_out && rows % kBlockLen == 0 && batch <= 8 &&
        segs == t.tiles) {
        const int nl = nx->dtype == CTOX_DTYPE_Q4B64 ? 1 : 0;
        const size_t nblk = rows / kBlockLen;
        ctox_status st = ensure(b, b->xn[nl], nblk * batch * 192, false);
        if (!st) st = ensure(b, b->xnc[nl], nblk * batch * 4 * sizeof(float), false);
        if (st) return st;
        a.nx_xa = (int8_t *)b->xn[nl].ptr;
        a.nx_xc = (float *)b->xnc[nl].ptr;
        a.nx_h = nx->h_out;
        a.nx_w = nx->w;
        a.nx_s_in = nx->s_in;
        a.nx_sq = nx->sq_out;
        a.nx_dtype = (uint32_t)nl;
        if (staged) *staged = true;
    }
    a.s_out = d_s_out;
    a.bias = d_bias;
    a.output = d_output;
    a.partial = (uint64_t *)b->tpart.ptr;
    a.seq = next_tile_seq(b);
    a.rows = (uint32_t)rows;
    a.blocks = (uint32_t)(columns / kBlockLen);
    a.tiles = t.tiles;
    a.chunks = t.chunks;
    a.segs = segs;
    a.tpw = u;
    a.s_out_kind = s_out_kind;
    a.activation = act;
    a.batch = (uint32_t)batch;
    a.out_stride = (uint32_t)out_stride;
    a.res_h = res_h;
    a.res_sq = res_sq;
    a.parts_out = parts_out ? 1u : 0u;
    return launch(arrive ? b->tilem_arr[q4][batch - 2] : b->tilem[q4][batch - 2], dim3((unsigned)(waves / 4)), dim3(256), s, a, "ctox_q*_mv_tilem*_gfx950");
}

// One launch of the small-M tiled matvec that builds its 2..5 rows'
// fragments from d_input (and the transform's operands in xf) itself.
ctox_status run_tile_matvec_mx(ctox_hip_backend *b, int32_t dtype, const TiledCopy &t, size_t rows, size_t columns,
                               size_t batch, const void *d_s_out, uint32_t s_out_kind, const float *d_bias,
                               float *d_output, size_t out_stride, uint32_t act, hipStream_t s, const float *d_input,
                               const void *d_s_in, uint32_t s_in_kind, const TileXform &xf, const PartialSlots *ps) {
    const int q4 = dtype == CTOX_DTYPE_Q4B64 ? 1 : 0;
    const uint32_t u = 1;
    const uint32_t segs = (((t.tiles + u - 1) / u) + 3) & ~3u;
    const size_t waves = (size_t)segs * t.chunks;
    if (batch < 2 || batch > kMaxBuildRows) return fail(CTOX_ERR_SHAPE, "in-kernel row build takes 2..5 rows");
    if (waves / 4 > 0x7fffffffu || out_stride > 0xffffffffu) return fail(CTOX_ERR_SHAPE, "matrix too large for one launch");
    const bool arrive =
        t.chunks > 1 && (b->arrive >= 0 ? b->arrive != 0 : waves / 4 > b->tilemx_cap[q4][batch - 2]);
    const size_t slot_bytes =
        (size_t)(arrive ? t.chunks : t.chunks - 1) * batch * t.tiles * CTOX_TILE_ROWS * sizeof(uint64_t);
    if (ps && t.chunks > 1 && (slot_bytes > ps->bytes || (arrive && t.tiles > ps->arrive_n)))
        return fail(CTOX_ERR_MEMORY_BUDGET, "combine slots need %zu bytes, the static scratch holds %zu", slot_bytes,
                    ps->bytes);
    if (t.chunks > 1 && !ps) {
        ctox_status st = ensure(b, b->tpart, slot_bytes, true);
        if (!st && arrive) st = ensure(b, b->tarrive, (size_t)t.tiles * sizeof(uint32_t), true);
        if (st) return st;
    }
    TileMatvecArgs a{};
    a.arrive = arrive ? (ps ? ps->arrive : (uint32_t *)b->tarrive.ptr) : nullptr;
    a.weights = (const uint8_t *)t.d;
    a.s_out = d_s_out;
    a.bias = d_bias;
    a.output = d_output;
    a.partial = ps ? ps->p : (uint64_t *)b->tpart.ptr;
    a.seq = ps ? ps->seq : next_tile_seq(b);
    a.rows = (uint32_t)rows;
    a.blocks = (uint32_t)(columns / kBlockLen);
    a.tiles = t.tiles;
    a.chunks = t.chunks;
    a.segs = segs;
    a.tpw = u;
    a.s_out_kind = s_out_kind;
    a.activation = act;
    a.input = d_input;
    a.s_in = d_s_in;
    a.s_in_kind = s_in_kind;
    a.xmode = xf.xmode;
    a.xb = xf.b;
    a.xw = xf.w;
    a.delta = xf.delta;
    a.x_out = xf.x_out;
    a.norm_out = xf.norm_out;
    a.off = xf.off;
    a.head_dim = xf.head_dim;
    a.eps = xf.eps;
    a.res_h = xf.res_h;
    a.res_sq = xf.res_sq;
    a.sq_in = xf.sq_in;
    a.sq_n = xf.sq_in ? xf.sq_n : 0u;
    a.batch = (uint32_t)batch;
    a.out_stride = (uint32_t)out_stride;
    a.a_stride = xf.a_stride;
    a.b_stride = xf.b_stride;
    return launch(arrive ? b->tilemx_arr[q4][batch - 2] : b->tilemx[q4][batch - 2], dim3((unsigned)(waves / 4)), dim3(256), s, a,
                  "ctox_q*_mv_tilemx*_gfx950");
}

// The registered tiled copy of raw weights, or NULL.
const TiledCopy *registered(ctox_hip_backend *b, const void *d_weights, size_t rows, size_t columns) {
    if (b->raw_tiled.empty()) return nullptr;
    auto it = b->raw_tiled.find(d_weights);
    if (it == b->raw_tiled.end() || it->second.rows != rows || it->second.columns != columns) return nullptr;
    return &it->second;
}

// `prepped` marks the layouts already staged for this input in this call
// sequence (fan-out shares them).
ctox_status dispatch_matrix(ctox_hip_backend *b, const ctox_hip_matrix *m, const float *d_input,
                            size_t batch, float *d_output, hipStream_t s, bool prepped[2],
                            uint32_t act) {
    size_t si = 0;
    for (const ctox_quant_segment &seg : m->segments) {
        const void *w = (const uint8_t *)m->d_weights + seg.offset;
        const int layout = seg.dtype == CTOX_DTYPE_Q4B64 ? 1 : 0;
        if (batch == 1 && si < m->tiled.size()) {
            // Batch 1: one launch, activation fragments built in the kernel.
            const size_t r0 = seg.row_start, nrows = seg.row_end - seg.row_start;
            const void *so = nullptr;
            if (m->s_out_kind == CTOX_KSCALE_F32) so = (const float *)m->d_s_out + r0;
            if (m->s_out_kind == CTOX_KSCALE_F16) so = (const uint16_t *)m->d_s_out + r0;
            ctox_status st = run_tile_matvec(b, seg.dtype, m->tiled[si], nrows, m->columns, so, m->s_out_kind,
                                             m->d_bias ? m->d_bias + r0 : nullptr, d_output + r0, act, s, d_input,
                                             m->d_s_in, m->s_in_kind);
            if (st) return st;
            si++;
            continue;
        }
        if (build_in_kernel(b, batch, seg.row_end - seg.row_start, m->columns) && si < m->tiled.size()) {
            // 2..5 rows: fragments built in the kernel (no staging launch).
            const size_t r0 = seg.row_start, nrows = seg.row_end - seg.row_start;
            const void *so = nullptr;
            if (m->s_out_kind == CTOX_KSCALE_F32) so = (const float *)m->d_s_out + r0;
            if (m->s_out_kind == CTOX_KSCALE_F16) so = (const uint16_t *)m->d_s_out + r0;
            TileXform xf;
            xf.a_stride = (uint32_t)m->columns;
            ctox_status st = run_tile_matvec_mx(b, seg.dtype, m->tiled[si], nrows, m->columns, batch, so, m->s_out_kind,
                                                m->d_bias ? m->d_bias + r0 : nullptr, d_output + r0, m->rows, act, s,
                                                d_input, m->d_s_in, m->s_in_kind, xf);
            if (st) return st;
            si++;
            continue;
        }
        if (!prepped[layout]) {
            ctox_status st = run_prep(b, layout, d_input, m->columns, batch, m->d_s_in, m->s_in_kind, s);
            if (st) return st;
            prepped[layout] = true;
        }
        const size_t r0 = seg.row_start, nrows = seg.row_end - seg.row_start;
        const void *so = nullptr;
        if (m->s_out_kind == CTOX_KSCALE_F32) so = (const float *)m->d_s_out + r0;
        if (m->s_out_kind == CTOX_KSCALE_F16) so = (const uint16_t *)m->d_s_out + r0;
        if (si < m->tiled.size()) {
            ctox_status st = run_tile_matvec_m(b, seg.dtype, m->tiled[si], nrows, m->columns, batch, so, m->s_out_kind,
                                               m->d_bias ? m->d_bias + r0 : nullptr, d_output + r0, m->rows, act, s);
            if (st) return st;
            si++;
            continue;
        }
        si++;
        ctox_status st = run_matvec(b, layout, seg.dtype, w, nrows, m->columns, batch, so, m->s_out_kind,
                                    m->d_bias ? m->d_bias + r0 : nullptr, d_output + r0, m->rows, act, s);
        if (st) return st;
    }
    return CTOX_OK;
}

ctox_status check_finite_host(const float *v, size_t n, const char *what) {
    for (size_t i = 0; i < n; i++)
        if (!std::isfinite(v[i]))
            return fail(CTOX_ERR_INVALID_STATE, "%s produced a non-finite value at %zu", what, i);
    return CTOX_OK;
}

}  // namespace

// ======================================================================
// lifecycle
// ======================================================================
extern "C" ctox_status ctox_hip_backend_create(int device, ctox_hip_backend **out) {
    if (!out) return fail(CTOX_ERR_SHAPE, "null output handle");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0)
        return fail(CTOX_ERR_UNSUPPORTED_OPERATION,
                    "backend hip cannot execute backend initialization: no HIP device (%s)",
                    e == hipSuccess ? "0 devices" : hipGetErrorString(e));
    if (device < 0 || device >= count)
        return fail(CTOX_ERR_UNSUPPORTED_OPERATION, "HIP device %d out of range (%d devices)", device, count);
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(CTOX_ERR_UNSUPPORTED_OPERATION,
                    "backend hip cannot execute backend initialization: device is %s, kernels are gfx950",
                    prop.gcnArchName);
    ctox_hip_backend *b = new ctox_hip_backend();
    b->device = device;
    std::snprintf(b->arch, sizeof b->arch, "%s", prop.gcnArchName);
    hipError_t le = hipSetDevice(device);
    if (le == hipSuccess) le = hipModuleLoadData(&b->module, ctox_hsaco_begin);
    // The allocation-free entry point's static scratch on this device
    // (address taken once per device, with the device current).
    if (le == hipSuccess) b->noalloc_ok = ctox_noalloc_setup(device) == CTOX_OK;
    if (le == hipSuccess) le = hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking);
    struct {
        hipFunction_t *f;
        const char *name;
    } fns[] = {{&b->prep, "ctox_prep_activation_gfx950"}, {&b->q4_b1, "ctox_q4_matvec_b1_gfx950"},
               {&b->q2_b1, "ctox_q2_matvec_b1_gfx950"},    {&b->q4_b4, "ctox_q4_matvec_b4_gfx950"},
               {&b->q4_b8, "ctox_q4_matvec_b8_gfx950"},    {&b->q2_b4, "ctox_q2_matvec_b4_gfx950"},
               {&b->q2_b8, "ctox_q2_matvec_b8_gfx950"},    {&b->rec_row, "ctox_recovered_row_gfx950"},
               {&b->row_dot, "ctox_row_dot_gfx950"},
               {&b->gdn_scan, "ctox_gdn_scan_gfx950"},    {&b->gdn_chunk_prep, "ctox_gdn_chunk_prep_gfx950"},
               {&b->gdn_chunk_scan, "ctox_gdn_chunk_scan_gfx950"},
               {&b->gdn_chunk_scan_vec, "ctox_gdn_chunk_scan_vec_gfx950"}, {&b->gates, "ctox_gdn_gates_gfx950"},
               {&b->repeat, "ctox_repeat_heads_gfx950"},   {&b->partials, "ctox_row_partials_gfx950"},
               {&b->argmax_final, "ctox_argmax_final_gfx950"}, {&b->greedy_status, "ctox_greedy_status_gfx950"}, {&b->verify, "ctox_verify_greedy_gfx950"},
               {&b->decide, "ctox_mtp_decide_gfx950"},     {&b->pick_sums, "ctox_pick_sums_gfx950"},
               {&b->pick_final, "ctox_pick_final_gfx950"},  {&b->rms, "ctox_rms_norm_gfx950"},
               {&b->swiglu, "ctox_swiglu_gfx950"},         {&b->sgate, "ctox_sigmoid_gate_gfx950"},
               {&b->conv, "ctox_conv_update_gfx950"},      {&b->rope, "ctox_rope_gfx950"},
               {&b->kv_pack, "ctox_kv_pack_q4_gfx950"}, {&b->attn_prep, "ctox_attn_prep_gfx950"},    {&b->kv_demote, "ctox_kv_demote_gfx950"},
               {&b->gqa_part[0], "ctox_paged_gqa_partial_r1_gfx950"},
               {&b->gqa_part[1], "ctox_paged_gqa_partial_r2_gfx950"},
               {&b->gqa_part16[0], "ctox_paged_gqa_partial16_r1_gfx950"},
               {&b->gqa_part16[1], "ctox_paged_gqa_partial16_r2_gfx950"},
               {&b->gqa_combine, "ctox_paged_gqa_combine_gfx950"},
               {&b->fill, "ctox_fill_random_gfx950"},      {&b->embed, "ctox_embed_rows_gfx950"},
               {&b->norm_rows, "ctox_norm_rows_gfx950"},   {&b->attn_gate, "ctox_attn_gate_gfx950"},
               {&b->swiglu_rows, "ctox_swiglu_rows_gfx950"}, {&b->copy_rows, "ctox_copy_rows_gfx950"},
               {&b->write_words, "ctox_write_words_gfx950"}, {&b->norm_prep, "ctox_norm_prep_gfx950"},
               {&b->prep_x, "ctox_prep_transform_gfx950"},
               {&b->sl[0][0], "ctox_q2_matvec_sl_gfx950"}, {&b->sl[0][1], "ctox_q2_matvec_sl1_gfx950"},
               {&b->sl[0][2], "ctox_q2_matvec_sl2_gfx950"}, {&b->sl[0][3], "ctox_q2_matvec_sl3_gfx950"},
               {&b->sl[1][0], "ctox_q4_matvec_sl_gfx950"}, {&b->sl[1][1], "ctox_q4_matvec_sl1_gfx950"},
               {&b->sl[1][2], "ctox_q4_matvec_sl2_gfx950"}, {&b->sl[1][3], "ctox_q4_matvec_sl3_gfx950"},
               {&b->st[0][0], "ctox_q2_matvec_st4_gfx950"}, {&b->st[0][1], "ctox_q2_matvec_st8_gfx950"},
               {&b->st[1][0], "ctox_q4_matvec_st4_gfx950"}, {&b->st[1][1], "ctox_q4_matvec_st8_gfx950"},
               {&b->tile[0][0], "ctox_q2_mv_tile1_gfx950"}, {&b->tile[0][1], "ctox_q2_mv_tile2_gfx950"},
               {&b->tile[0][2], "ctox_q2_mv_tile3_gfx950"}, {&b->tile[0][3], "ctox_q2_mv_tile4_gfx950"},
               {&b->tile[1][0], "ctox_q4_mv_tile1_gfx950"}, {&b->tile[1][1], "ctox_q4_mv_tile2_gfx950"},
               {&b->tile[1][2], "ctox_q4_mv_tile3_gfx950"}, {&b->tile[1][3], "ctox_q4_mv_tile4_gfx950"},
               {&b->tile_arr[0][0][0], "ctox_q2_mv_tile1_gfx950_arrive"}, {&b->tile_arr[0][0][1], "ctox_q2_mv_tile2_gfx950_arrive"},
               {&b->tile_arr[0][0][2], "ctox_q2_mv_tile3_gfx950_arrive"}, {&b->tile_arr[0][0][3], "ctox_q2_mv_tile4_gfx950_arrive"},
               {&b->tile_arr[0][1][0], "ctox_q4_mv_tile1_gfx950_arrive"}, {&b->tile_arr[0][1][1], "ctox_q4_mv_tile2_gfx950_arrive"},
               {&b->tile_arr[0][1][2], "ctox_q4_mv_tile3_gfx950_arrive"}, {&b->tile_arr[0][1][3], "ctox_q4_mv_tile4_gfx950_arrive"},
               {&b->tilemx[0][0], "ctox_q2_mv_tilemx2_gfx950"}, {&b->tilemx[0][1], "ctox_q2_mv_tilemx3_gfx950"},
               {&b->tilemx[0][2], "ctox_q2_mv_tilemx4_gfx950"}, {&b->tilemx[0][3], "ctox_q2_mv_tilemx5_gfx950"},
               {&b->tilemx[1][0], "ctox_q4_mv_tilemx2_gfx950"}, {&b->tilemx[1][1], "ctox_q4_mv_tilemx3_gfx950"},
               {&b->tilemx[1][2], "ctox_q4_mv_tilemx4_gfx950"}, {&b->tilemx[1][3], "ctox_q4_mv_tilemx5_gfx950"},
               {&b->tilemx_arr[0][0], "ctox_q2_mv_tilemx2_gfx950_arrive"}, {&b->tilemx_arr[0][1], "ctox_q2_mv_tilemx3_gfx950_arrive"},
               {&b->tilemx_arr[0][2], "ctox_q2_mv_tilemx4_gfx950_arrive"}, {&b->tilemx_arr[0][3], "ctox_q2_mv_tilemx5_gfx950_arrive"},
               {&b->tilemx_arr[1][0], "ctox_q4_mv_tilemx2_gfx950_arrive"}, {&b->tilemx_arr[1][1], "ctox_q4_mv_tilemx3_gfx950_arrive"},
               {&b->tilemx_arr[1][2], "ctox_q4_mv_tilemx4_gfx950_arrive"}, {&b->tilemx_arr[1][3], "ctox_q4_mv_tilemx5_gfx950_arrive"},
               {&b->repack, "ctox_tile_repack_gfx950"}, {&b->gdn_fused, "ctox_gdn_fused_gfx950"}, {&b->gdn_fused_blk, "ctox_gdn_fused_blk_gfx950"},
               {&b->gdn_fused1, "ctox_gdn_fused1_gfx950"}, {&b->gdn_fused1_blk, "ctox_gdn_fused1_blk_gfx950"},
               {&b->gdn_k4[0][0], "ctox_gdn_fused_k4_gfx950"}, {&b->gdn_k4[0][1], "ctox_gdn_fused_blk_k4_gfx950"},
               {&b->gdn_k4[1][0], "ctox_gdn_fused1_k4_gfx950"}, {&b->gdn_k4[1][1], "ctox_gdn_fused1_blk_k4_gfx950"},
               {&b->finite, "ctox_finite_check_gfx950"}, {&b->gather, "ctox_gather_rows_gfx950"}, {&b->stream_read, "ctox_stream_read_gfx950"},
               {&b->write_segments, "ctox_write_segments_gfx950"},
               {&b->topk_part, "ctox_topk_part_gfx950"}, {&b->topk_final, "ctox_topk_final_gfx950"}};
    for (auto &f : fns) {
        if (le != hipSuccess) break;
        le = hipModuleGetFunction(f.f, b->module, f.name);
        if (le != hipSuccess) {
            ctox_hip_backend_destroy(b);
            return fail(CTOX_ERR_UNSUPPORTED_OPERATION, "kernel %s missing from code object: %s", f.name,
                        hipGetErrorString(le));
        }
    }
    // The in-kernel build kernels, one per input transform.
    for (int x = 0; x < 6 && le == hipSuccess; x++)
        for (int q = 0; q < 2 && le == hipSuccess; q++)
            for (int u = 0; u < CTOX_TILE_MAXU && le == hipSuccess; u++)
                for (int arr = 0; arr < 2 && le == hipSuccess; arr++) {
                    char name[64];
                    std::snprintf(name, sizeof name, "ctox_q%d_mv_tile%dx%d_gfx950%s", q ? 4 : 2, u + 1, x,
                                  arr ? "_arrive" : "");
                    le = hipModuleGetFunction(arr ? &b->tile_arr[1 + x][q][u] : &b->tilex[x][q][u], b->module, name);
                    if (le != hipSuccess) {
                        ctox_hip_backend_destroy(b);
                        return fail(CTOX_ERR_UNSUPPORTED_OPERATION, "kernel %s missing from code object: %s", name,
                                    hipGetErrorString(le));
                    }
                }
    // The small-M kernels for staged rows, one per row count 2..8.
    for (int q = 0; q < 2 && le == hipSuccess; q++)
        for (int m = 0; m < 7 && le == hipSuccess; m++)
            for (int arr = 0; arr < 2 && le == hipSuccess; arr++) {
                char name[64];
                std::snprintf(name, sizeof name, "ctox_q%d_mv_tilem%d_gfx950%s", q ? 4 : 2, m + 2, arr ? "_arrive" : "");
                le = hipModuleGetFunction(arr ? &b->tilem_arr[q][m] : &b->tilem[q][m], b->module, name);
                if (le != hipSuccess) {
                    ctox_hip_backend_destroy(b);
                    return fail(CTOX_ERR_UNSUPPORTED_OPERATION, "kernel %s missing from code object: %s", name,
                                hipGetErrorString(le));
                }
            }
    if (le != hipSuccess) {
        ctox_hip_backend_destroy(b);
        return fail(CTOX_ERR_UNSUPPORTED_OPERATION, "HIP module setup failed: %s", hipGetErrorString(le));
    }
    b->cus = prop.multiProcessorCount;
    // CTOX_SMALL_M_BUILD=0: 2..5-row projections stage their fragments in a
    // separate launch (the tilem kernels) instead of building them in-kernel.
    if (const char *m = std::getenv("CTOX_SMALL_M_BUILD")) b->no_mx = std::atoi(m) == 0;
    if (const char *m = std::getenv("CTOX_ARRIVE")) b->arrive = std::atoi(m) != 0;
    if (const char *m = std::getenv("CTOX_GDN_ONE")) b->gdn_one = std::atoi(m) != 0;
    if (const char *m = std::getenv("CTOX_MX_MAX")) b->mx_max = (uint64_t)std::atoll(m) << 20;
    // How many workgroups of each tiled kernel the device holds at once:
    // launches within it may combine by the last chunk's waves (every
    // producer is resident whatever the dispatch order); larger ones combine
    // by arrival.
    auto cap = [&](hipFunction_t f) {
        int n = 0;
        if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, 256, 0) != hipSuccess) n = 0;
        return (uint32_t)std::max(0, n) * (uint32_t)b->cus;
    };
    for (int q = 0; q < 2; q++) {
        for (int u = 0; u < CTOX_TILE_MAXU; u++) {
            b->tile_cap[0][q][u] = cap(b->tile[q][u]);
            for (int x = 0; x < 6; x++) b->tile_cap[1 + x][q][u] = cap(b->tilex[x][q][u]);
        }
        for (int m = 0; m < 7; m++) b->tilem_cap[q][m] = cap(b->tilem[q][m]);
        for (int r = 0; r < 4; r++) b->tilemx_cap[q][r] = cap(b->tilemx[q][r]);
    }
    if (const char *u = std::getenv("CTOX_TILE_U")) {
        const int v = std::atoi(u);
        if (v >= 1 && v <= CTOX_TILE_MAXU) b->tile_u = (uint32_t)v;
    }
    *out = b;
    return CTOX_OK;
}

extern "C" void ctox_hip_backend_destroy(ctox_hip_backend *b) {
    if (!b) return;
    (void)hipSetDevice(b->device);
    (void)hipDeviceSynchronize();
    DevBuf *bufs[] = {&b->xa[0], &b->xa[1], &b->xc[0], &b->xc[1], &b->xn[0], &b->xn[1], &b->xnc[0], &b->xnc[1],
                      &b->norms, &b->tok, &b->stats, &b->attn, &b->tpart, &b->tarrive};
    for (auto &kv : b->raw_tiled)
        if (kv.second.d) (void)hipFree(kv.second.d);
    for (DevBuf *d : bufs)
        if (d->ptr) (void)hipFree(d->ptr);
    if (b->stream) (void)hipStreamDestroy(b->stream);
    if (b->module) (void)hipModuleUnload(b->module);
    delete b;
}

extern "C" const char *ctox_hip_backend_kind(const ctox_hip_backend *) { return "hip"; }
extern "C" const char *ctox_hip_backend_promotion_state(const ctox_hip_backend *) { return "experimental"; }
extern "C" const char *ctox_hip_backend_profile(const ctox_hip_backend *) { return "gfx950-mfma-i8"; }
extern "C" const char *ctox_hip_last_error(void) { return g_last_error.c_str(); }

// Error text of the engine translation unit (same thread-local slot).
void ctox_set_last_error(const char *msg) { g_last_error = msg; }

extern "C" ctox_status ctox_hip_synchronize(ctox_hip_backend *b) {
    if (!b) return fail(CTOX_ERR_INVALID_STATE, "null backend");
    HIP_TRY(hipStreamSynchronize(b->stream));
    return CTOX_OK;
}

// ======================================================================
// resident matrices
// ======================================================================
namespace {
// Rewrites every segment of a resident matrix into the tiled layout on the
// device (one pass at prepare time; the crate-layout copy stays for batch > 1).
ctox_status tile_copy(ctox_hip_backend *b, int32_t dtype, const void *d_src, size_t rows, size_t columns,
                      hipStream_t s, TiledCopy &t) {
    const uint32_t blocks = (uint32_t)(columns / kBlockLen);
    t.rows = (uint32_t)rows;
    t.columns = (uint32_t)columns;
    t.tiles = (uint32_t)((rows + CTOX_TILE_ROWS - 1) / CTOX_TILE_ROWS);
    t.chunks = (blocks + CTOX_TILE_BLOCKS - 1) / CTOX_TILE_BLOCKS;
    const uint32_t q4 = dtype == CTOX_DTYPE_Q4B64 ? 1 : 0;
    const size_t units = (size_t)t.tiles * t.chunks;
    if (units > 0x7fffffffu || units * ctox_tile_unit_bytes(q4) > 0x7ffffff0u)
        return fail(CTOX_ERR_SHAPE, "matrix too large to tile");
    HIP_TRY(hipMalloc(&t.d, units * ctox_tile_unit_bytes(q4)));
    TileRepackArgs a{};
    a.src = (const uint8_t *)d_src;
    a.dst = (uint8_t *)t.d;
    a.rows = (uint32_t)rows;
    a.blocks = blocks;
    a.tiles = t.tiles;
    a.chunks = t.chunks;
    a.dtype = q4;
    return launch(b->repack, dim3((unsigned)units), dim3(64), s, a, "ctox_tile_repack_gfx950");
}

// Rewrites every segment of a resident matrix into the tiled layout on the
// device (one pass at prepare time; the crate-layout copy stays for batch > 1).
ctox_status tile_segments(ctox_hip_backend *b, ctox_hip_matrix *m) {
    for (const ctox_quant_segment &seg : m->segments) {
        TiledCopy t;
        ctox_status st = tile_copy(b, seg.dtype, (const uint8_t *)m->d_weights + seg.offset,
                                   seg.row_end - seg.row_start, m->columns, pick_stream(b, b->stream), t);
        if (t.d) m->tiled.push_back(t);
        if (st) return st;
    }
    HIP_TRY(hipStreamSynchronize(b->stream));
    return CTOX_OK;
}

ctox_status prepare_impl(ctox_hip_backend *b, const ctox_fused_matvec *op, ctox_hip_matrix **out) {
    size_t blocks;
    ctox_status st = validate_matvec(op, false, &blocks);
    if (!st) st = check_matrix_scales(op, blocks);
    if (st) return st;
    HIP_TRY(hipSetDevice(b->device));
    ctox_hip_matrix *m = new ctox_hip_matrix();
    m->backend = b;
    m->dtype = op->dtype;
    m->rows = op->rows;
    m->columns = op->columns;
    if (op->dtype == CTOX_DTYPE_MIXED_Q2Q4B64) {
        m->segments.assign(op->segments, op->segments + op->n_segments);
    } else {
        ctox_quant_segment s{0, 0, op->rows, op->dtype, 0, op->weights_len};
        m->segments.push_back(s);
    }
    m->weights_len = op->weights_len;
    st = upload(op->weights, op->weights_len, &m->d_weights);
    if (!st && op->s_in.kind != CTOX_SCALE_NONE) {
        const size_t bytes = op->s_in.len * (op->s_in.kind == CTOX_SCALE_F32 ? 4 : 2);
        st = upload(op->s_in.data, bytes, &m->d_s_in);
        m->s_in_kind = kernel_scale_kind(op->s_in.kind);
        m->s_in_host.assign((const uint8_t *)op->s_in.data, (const uint8_t *)op->s_in.data + bytes);
    }
    if (!st && op->s_out.kind != CTOX_SCALE_NONE) {
        st = upload(op->s_out.data, op->s_out.len * (op->s_out.kind == CTOX_SCALE_F32 ? 4 : 2), &m->d_s_out);
        m->s_out_kind = kernel_scale_kind(op->s_out.kind);
    }
    if (!st && op->bias) st = upload(op->bias, op->rows * sizeof(float), (void **)&m->d_bias);
    if (!st) st = tile_segments(b, m);
    if (st) {
        ctox_hip_matrix_destroy(m);
        return st;
    }
    m->activation = (uint32_t)op->activation;
    *out = m;
    return CTOX_OK;
}
}  // namespace

extern "C" ctox_status ctox_hip_matrix_prepare(ctox_hip_backend *b, const ctox_fused_matvec *op,
                                               ctox_hip_matrix **out) {
    if (!b || !op || !out) return fail(CTOX_ERR_SHAPE, "null argument");
    *out = nullptr;
    return prepare_impl(b, op, out);
}

extern "C" void ctox_hip_matrix_destroy(ctox_hip_matrix *m) {
    if (!m) return;
    (void)hipSetDevice(m->backend->device);
    (void)hipDeviceSynchronize();
    if (m->d_weights) (void)hipFree(m->d_weights);
    if (m->d_s_in) (void)hipFree(m->d_s_in);
    if (m->d_s_out) (void)hipFree(m->d_s_out);
    if (m->d_bias) (void)hipFree(m->d_bias);
    for (auto &t : m->tiled)
        if (t.d) (void)hipFree(t.d);
    delete m;
}

extern "C" size_t ctox_hip_matrix_rows(const ctox_hip_matrix *m) { return m ? m->rows : 0; }
extern "C" size_t ctox_hip_matrix_columns(const ctox_hip_matrix *m) { return m ? m->columns : 0; }
extern "C" const void *ctox_hip_matrix_device_weights(const ctox_hip_matrix *m) {
    return m ? m->d_weights : nullptr;
}

extern "C" ctox_status ctox_hip_matrix_dispatch(ctox_hip_backend *b, const ctox_hip_matrix *m,
                                                const float *d_input, size_t batch, float *d_output,
                                                void *stream) {
    if (!b || !m || !d_input || !d_output) return fail(CTOX_ERR_SHAPE, "null argument");
    if (batch == 0 || batch > CTOX_MAX_BATCH)
        return fail(CTOX_ERR_SHAPE, "batch %zu outside 1..%d", batch, CTOX_MAX_BATCH);
    bool prepped[2] = {false, false};
    return dispatch_matrix(b, m, d_input, batch, d_output, pick_stream(b, stream), prepped, m->activation);
}

extern "C" ctox_status ctox_hip_matrix_dispatch_fanout(ctox_hip_backend *b,
                                                       const ctox_hip_matrix *const *ms, size_t n,
                                                       const float *d_input, size_t batch,
                                                       float *const *d_outputs, void *stream) {
    if (!b || !ms || !d_input || !d_outputs) return fail(CTOX_ERR_SHAPE, "null argument");
    if (n == 0) return fail(CTOX_ERR_SHAPE, "fan-out requires at least one projection");
    if (batch == 0 || batch > CTOX_MAX_BATCH)
        return fail(CTOX_ERR_SHAPE, "batch %zu outside 1..%d", batch, CTOX_MAX_BATCH);
    for (size_t i = 1; i < n; i++)
        if (ms[i]->columns != ms[0]->columns || ms[i]->s_in_kind != ms[0]->s_in_kind ||
            ms[i]->s_in_host != ms[0]->s_in_host)
            return fail(CTOX_ERR_SHAPE, "fan-out projections must share columns and s_in");
    bool prepped[2] = {false, false};
    hipStream_t s = pick_stream(b, stream);
    for (size_t i = 0; i < n; i++) {
        ctox_status st = dispatch_matrix(b, ms[i], d_input, batch, d_outputs[i], s, prepped, ms[i]->activation);
        if (st) return st;
    }
    return CTOX_OK;
}

extern "C" ctox_status ctox_hip_launch_fused_matvec(ctox_hip_backend *b, int32_t dtype,
                                                    const void *d_weights, const float *d_input,
                                                    const uint16_t *d_s_in, const uint16_t *d_s_out,
                                                    const float *d_bias, float *d_output, uint32_t rows,
                                                    uint32_t columns, uint32_t activation, uint32_t batch,
                                                    void *stream) {
    if (!b || !d_weights || !d_input || !d_output) return fail(CTOX_ERR_SHAPE, "null argument");
    if (dtype != CTOX_DTYPE_Q2B64 && dtype != CTOX_DTYPE_Q4B64)
        return fail(CTOX_ERR_UNSUPPORTED_DTYPE, "raw launch takes pure Q2_B64 or Q4_B64 weights");
    if (rows == 0 || columns == 0 || columns % kBlockLen)
        return fail(CTOX_ERR_SHAPE, "Q2/Q4 fused matvec dimensions must be non-zero and columns divisible by 64");
    if (batch == 0 || batch > CTOX_MAX_BATCH)
        return fail(CTOX_ERR_SHAPE, "batch %u outside 1..%d", batch, CTOX_MAX_BATCH);
    if (activation > 1) return fail(CTOX_ERR_SHAPE, "activation %u is not identity (0) or SiLU (1)", activation);
    hipStream_t s = pick_stream(b, stream);
    const int layout = dtype == CTOX_DTYPE_Q4B64 ? 1 : 0;
    if (const TiledCopy *t = registered(b, d_weights, rows, columns)) {
        if (batch == 1)
            return run_tile_matvec(b, dtype, *t, rows, columns, d_s_out, d_s_out ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE,
                                   d_bias, d_output, activation, s, d_input, d_s_in,
                                   d_s_in ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE);
        if (build_in_kernel(b, batch, rows, columns)) {
            TileXform xf;
            xf.a_stride = columns;
            return run_tile_matvec_mx(b, dtype, *t, rows, columns, batch, d_s_out,
                                      d_s_out ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE, d_bias, d_output, rows, activation,
                                      s, d_input, d_s_in, d_s_in ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE, xf);
        }
    }
    ctox_status st = run_prep(b, layout, d_input, columns, batch, d_s_in,
                              d_s_in ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE, s);
    if (st) return st;
    return run_matvec(b, layout, dtype, d_weights, rows, columns, batch, d_s_out,
                      d_s_out ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE, d_bias, d_output, rows, activation, s);
}

extern "C" ctox_status ctox_hip_launch_fused_matvec_noalloc(ctox_hip_backend *b, int32_t dtype,
                                                            const void *d_weights, const float *d_input,
                                                            const uint16_t *d_s_in, const uint16_t *d_s_out,
                                                            const float *d_bias, float *d_output, uint32_t rows,
                                                            uint32_t columns, uint32_t activation, uint32_t batch,
                                                            void *stream) {
    if (!b || !d_weights || !d_input || !d_output) return fail(CTOX_ERR_SHAPE, "null argument");
    if (dtype != CTOX_DTYPE_Q2B64 && dtype != CTOX_DTYPE_Q4B64)
        return fail(CTOX_ERR_UNSUPPORTED_DTYPE, "raw launch takes pure Q2_B64 or Q4_B64 weights");
    if (rows == 0 || columns == 0 || columns % kBlockLen)
        return fail(CTOX_ERR_SHAPE, "Q2/Q4 fused matvec dimensions must be non-zero and columns divisible by 64");
    if (batch == 0 || batch > kMaxBuildRows) return fail(CTOX_ERR_SHAPE, "allocation-free launch takes 1..5 rows");
    if (activation > 1) return fail(CTOX_ERR_SHAPE, "activation %u is not identity (0) or SiLU (1)", activation);
    if (!b->noalloc_ok) return fail(CTOX_ERR_INVALID_STATE, "the static scratch of this device is not set up");
    const TiledCopy *t = registered(b, d_weights, rows, columns);
    if (!t) return fail(CTOX_ERR_UNSUPPORTED_OPERATION, "allocation-free launch needs registered tiled weights");
    hipStream_t s = pick_stream(b, stream);
    PartialSlots ps;
    if (ctox_noalloc_slots(b->device, s, &ps.p, &ps.bytes, &ps.seq, &ps.arrive, &ps.arrive_n) != CTOX_OK)
        return fail(CTOX_ERR_INVALID_STATE, "static scratch unavailable");
    const uint32_t sk = d_s_in ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE, ok = d_s_out ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE;
    if (batch == 1)
        return run_tile_matvec(b, dtype, *t, rows, columns, d_s_out, ok, d_bias, d_output, activation, s, d_input,
                               d_s_in, sk, nullptr, &ps);
    TileXform xf;
    xf.a_stride = columns;
    return run_tile_matvec_mx(b, dtype, *t, rows, columns, batch, d_s_out, ok, d_bias, d_output, rows, activation, s,
                              d_input, d_s_in, sk, xf, &ps);
}

extern "C" ctox_status ctox_hip_register_tiled_weights(ctox_hip_backend *b, int32_t dtype, const void *d_weights,
                                                       uint32_t rows, uint32_t columns, void *stream) {
    if (!b || !d_weights) return fail(CTOX_ERR_SHAPE, "null argument");
    if (dtype != CTOX_DTYPE_Q2B64 && dtype != CTOX_DTYPE_Q4B64)
        return fail(CTOX_ERR_UNSUPPORTED_DTYPE, "tiled registration takes pure Q2_B64 or Q4_B64 weights");
    if (rows == 0 || columns == 0 || columns % kBlockLen)
        return fail(CTOX_ERR_SHAPE, "Q2/Q4 fused matvec dimensions must be non-zero and columns divisible by 64");
    ctox_hip_unregister_tiled_weights(b, d_weights);
    TiledCopy t;
    ctox_status st = tile_copy(b, dtype, d_weights, rows, columns, pick_stream(b, stream), t);
    if (st) {
        if (t.d) {
            (void)hipStreamSynchronize(pick_stream(b, stream));
            (void)hipFree(t.d);
        }
        return st;
    }
    b->raw_tiled[d_weights] = t;
    return CTOX_OK;
}

extern "C" void ctox_hip_unregister_tiled_weights(ctox_hip_backend *b, const void *d_weights) {
    if (!b) return;
    auto it = b->raw_tiled.find(d_weights);
    if (it == b->raw_tiled.end()) return;
    (void)hipDeviceSynchronize();  // launches queued on any stream may still read the copy
    if (it->second.d) (void)hipFree(it->second.d);
    b->raw_tiled.erase(it);
}

// ======================================================================
// Backend trait on host buffers
// ======================================================================
extern "C" ctox_status ctox_hip_norm_matvec_device(ctox_hip_backend *b, const float *d_x, const float *d_delta,
                                                  uint32_t delta_parts, size_t delta_part_stride,
                                                  float *d_x_out, const float *d_norm_w, float eps,
                                                  float *d_norm_out, int32_t dtype,
                                                  const void *d_weights, const uint16_t *d_s_in,
                                                  const uint16_t *d_s_out, float *d_output, uint32_t rows,
                                                  uint32_t columns, uint32_t batch, void *stream) {
    return ctox_hip_norm_matvec_sums_device(b, d_x, d_delta, delta_parts, delta_part_stride, d_x_out, d_norm_w, eps,
                                            d_norm_out, dtype, d_weights, d_s_in, d_s_out, d_output, rows, columns,
                                            batch, nullptr, 0, stream);
}

extern "C" ctox_status ctox_hip_norm_matvec_sums_device(ctox_hip_backend *b, const float *d_x, const float *d_delta,
                                                       uint32_t delta_parts, size_t delta_part_stride,
                                                       float *d_x_out, const float *d_norm_w, float eps,
                                                       float *d_norm_out, int32_t dtype, const void *d_weights,
                                                       const uint16_t *d_s_in, const uint16_t *d_s_out,
                                                       float *d_output, uint32_t rows, uint32_t columns,
                                                       uint32_t batch, const float *d_sums, uint32_t sum_count,
                                                       void *stream) {
    return ctox_hip_norm_matvec_parts_device(b, d_x, d_delta, delta_parts, delta_part_stride, d_x_out, d_norm_w, eps,
                                             d_norm_out, dtype, d_weights, d_s_in, d_s_out, d_output, rows, columns,
                                             batch, d_sums, sum_count, 1, nullptr, stream);
}

extern "C" ctox_status ctox_hip_norm_matvec_parts_device(ctox_hip_backend *b, const float *d_x, const float *d_delta,
                                                        uint32_t delta_parts, size_t delta_part_stride,
                                                        float *d_x_out, const float *d_norm_w, float eps,
                                                        float *d_norm_out, int32_t dtype, const void *d_weights,
                                                        const uint16_t *d_s_in, const uint16_t *d_s_out,
                                                        float *d_output, uint32_t rows, uint32_t columns,
                                                        uint32_t batch, const float *d_sums, uint32_t sum_count,
                                                        uint32_t max_parts, uint32_t *parts, void *stream) {
    if (parts) *parts = 1;
    if (d_sums && (sum_count != (columns + CTOX_TILE_ROWS - 1) / CTOX_TILE_ROWS || sum_count > 512))
        return fail(CTOX_ERR_SHAPE, "residual sums: one per 16 columns of the row, at most 512");
    if (!b || !d_x || !d_norm_w || !d_weights || !d_output || (d_delta && !d_x_out))
        return fail(CTOX_ERR_SHAPE, "null argument");
    if (d_delta && d_x_out == d_x) return fail(CTOX_ERR_SHAPE, "norm-matvec residual output must not alias its input");
    if (d_delta && (delta_parts == 0 || delta_parts > 8 || (delta_parts > 1 && delta_part_stride < (size_t)batch * columns) ||
                    delta_part_stride > 0xffffffffu || delta_part_stride % 4))
        return fail(CTOX_ERR_SHAPE, "norm-matvec delta parts geometry");
    if (dtype != CTOX_DTYPE_Q2B64 && dtype != CTOX_DTYPE_Q4B64)
        return fail(CTOX_ERR_UNSUPPORTED_DTYPE, "norm-matvec takes pure Q2_B64 or Q4_B64 weights");
    if (rows == 0 || columns == 0 || columns % kBlockLen || columns > 8192)
        return fail(CTOX_ERR_SHAPE, "norm-matvec columns must be a non-zero multiple of 64 up to 8192");
    if (batch == 0 || batch > CTOX_MAX_BATCH) return fail(CTOX_ERR_SHAPE, "batch %u outside 1..%d", batch, CTOX_MAX_BATCH);
    if (!std::isfinite(eps) || eps <= 0.0f) return fail(CTOX_ERR_SHAPE, "norm epsilon must be finite and positive");
    hipStream_t s = pick_stream(b, stream);
    const int layout = dtype == CTOX_DTYPE_Q4B64 ? 1 : 0;
    const size_t blocks = columns / kBlockLen;
    // Registered weights, batch 1, at most one delta part: the residual add
    // and norm are computed inside the tiled matvec (one launch).
    if (batch == 1 && (!d_delta || delta_parts == 1)) {
        if (const TiledCopy *t = registered(b, d_weights, rows, columns)) {
            TileXform xf;
            xf.xmode = 1;
            xf.w = d_norm_w;
            xf.delta = d_delta;
            xf.x_out = d_delta ? d_x_out : nullptr;
            xf.norm_out = d_norm_out;
            xf.eps = eps;
            xf.sq_in = d_sums;
            xf.sq_n = sum_count;
            // Chunk partials for a consumer that adds them, when it takes that many.
            if (parts && max_parts > 1 && t->chunks <= max_parts) {
                xf.parts_out = true;
                *parts = t->chunks;
            }
            return run_tile_matvec(b, dtype, *t, rows, columns, d_s_out, d_s_out ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE,
                                   nullptr, d_output, 0, s, d_x, d_s_in, d_s_in ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE, &xf);
        }
    }
    // Registered weights, 2..5 rows with the producer's sums of squares: one
    // launch that builds every row's fragments.
    if (build_in_kernel(b, batch, rows, columns) && d_sums && (!d_delta || delta_parts == 1)) {
        if (const TiledCopy *t = registered(b, d_weights, rows, columns)) {
            TileXform xf;
            xf.xmode = 1;
            xf.w = d_norm_w;
            xf.delta = d_delta;
            xf.x_out = d_delta ? d_x_out : nullptr;
            xf.norm_out = d_norm_out;
            xf.eps = eps;
            xf.sq_in = d_sums;
            xf.sq_n = sum_count;
            xf.a_stride = columns;
            xf.b_stride = columns;
            return run_tile_matvec_mx(b, dtype, *t, rows, columns, batch, d_s_out,
                                      d_s_out ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE, nullptr, d_output, rows, 0, s, d_x,
                                      d_s_in, d_s_in ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE, xf);
        }
    }
    ctox_status st = ensure(b, b->xa[layout], blocks * batch * 192, false);
    if (!st) st = ensure(b, b->xc[layout], blocks * batch * 4 * sizeof(float), false);
    if (st) return st;
    NormPrepArgs a{};
    a.p.s_in = d_s_in;
    a.p.xa = (int8_t *)b->xa[layout].ptr;
    a.p.xc = (float *)b->xc[layout].ptr;
    a.p.columns = columns;
    a.p.batch = batch;
    a.p.dtype = (uint32_t)layout;
    a.p.s_in_kind = d_s_in ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE;
    a.p.tgroups = (batch + 3) / 4;
    a.x = d_x;
    a.delta = d_delta;
    a.delta_parts = d_delta ? delta_parts : 0;
    a.delta_stride = (uint32_t)delta_part_stride;
    a.x_out = d_x_out;
    a.w = d_norm_w;
    a.out = d_norm_out;
    a.eps = eps;
    if (d_sums && (!d_delta || delta_parts == 1)) {
        a.sq_in = d_sums;
        a.sq_n = sum_count;
    }
    if ((st = launch(b->norm_prep, dim3((unsigned)((blocks + 3) / 4), batch), dim3(256), s, a, "ctox_norm_prep_gfx950")))
        return st;
    // Registered weights, 2..8 staged rows: chunk partials for a consumer
    // that adds them, when it takes that many.
    if (batch > 1 && parts && max_parts > 1)
        if (const TiledCopy *t = registered(b, d_weights, rows, columns))
            if (t->chunks > 1 && t->chunks <= max_parts) {
                *parts = t->chunks;
                return run_tile_matvec_m(b, dtype, *t, rows, columns, batch, d_s_out,
                                         d_s_out ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE, nullptr, d_output, rows, 0, s,
                                         nullptr, nullptr, true);
            }
    return run_matvec(b, layout, dtype, d_weights, rows, columns, batch, d_s_out,
                      d_s_out ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE, nullptr, d_output, rows, 0, s);
}

namespace {
ctox_status transform_matvec_impl(ctox_hip_backend *b, const ctox_input_transform *x, int32_t dtype,
                                  const void *d_weights, const uint16_t *d_s_in, const uint16_t *d_s_out,
                                  float *d_output, uint32_t rows, uint32_t columns, uint32_t batch, uint32_t split_k,
                                  uint32_t *parts, void *stream, const NextNorm *nx, bool *staged,
                                  bool input_staged = false) {
    if (parts) *parts = 1;
    if (staged) *staged = false;
    if (!b || !x || !x->a || !d_weights || !d_output || ((x->mode == 2 || x->mode == 3) && !x->b) ||
        (x->mode == 2 && !x->w) || (x->res_sums && !x->res_h))
        return fail(CTOX_ERR_SHAPE, "null argument");
    if (x->mode < 1 || x->mode > 3) return fail(CTOX_ERR_SHAPE, "unknown input transform %u", x->mode);
    if (x->a_parts > 1 && (x->mode != 1 || x->a_parts > 6 ||
                           x->a_part_stride < (uint64_t)(batch - 1) * x->a_stride + x->off + columns))
        return fail(CTOX_ERR_SHAPE, "input partials: swiglu only, at most 6, a_part_stride covering the rows");
    if (dtype != CTOX_DTYPE_Q2B64 && dtype != CTOX_DTYPE_Q4B64)
        return fail(CTOX_ERR_UNSUPPORTED_DTYPE, "transform-matvec takes pure Q2_B64 or Q4_B64 weights");
    if (rows == 0 || columns == 0 || columns % kBlockLen) return fail(CTOX_ERR_SHAPE, "transform-matvec dimensions");
    if (batch == 0 || batch > CTOX_MAX_BATCH) return fail(CTOX_ERR_SHAPE, "batch %u outside 1..%d", batch, CTOX_MAX_BATCH);
    if ((x->mode != 1 && (x->head_dim == 0 || columns % x->head_dim)) ||
        (x->mode == 1 && x->a_stride < x->off + columns) || (x->mode != 1 && x->a_stride < columns) ||
        (x->mode == 2 && (!std::isfinite(x->eps) || x->eps <= 0.0f || x->b_stride < columns)) ||
        (x->mode == 3 && x->b_stride < 2 * columns))
        return fail(CTOX_ERR_SHAPE, "transform-matvec input geometry");
    hipStream_t s = pick_stream(b, stream);
    const int layout = dtype == CTOX_DTYPE_Q4B64 ? 1 : 0;
    const size_t blocks = columns / kBlockLen;
    // Registered weights, batch 1: the producer runs inside the tiled matvec.
    if (batch == 1 && (x->mode != 2 || x->head_dim == 64 || x->head_dim == 128 || x->head_dim == 256) &&
        (x->mode != 3 || x->head_dim % 4 == 0)) {
        if (const TiledCopy *t = registered(b, d_weights, rows, columns)) {
            TileXform xf;
            xf.xmode = x->mode + 1;
            xf.b = x->b;
            xf.w = x->w;
            xf.off = x->off;
            xf.head_dim = x->head_dim;
            xf.eps = x->eps;
            xf.res_h = x->res_h;
            xf.res_sq = x->res_sums;
            xf.a_parts = x->a_parts > 1 ? x->a_parts : 0;
            xf.a_pstride = x->a_part_stride;
            return run_tile_matvec(b, dtype, *t, rows, columns, d_s_out, d_s_out ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE,
                                   nullptr, d_output, 0, s, x->a, d_s_in, d_s_in ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE, &xf);
        }
    }
    // Registered weights, 2..5 rows: one launch that builds every row's fragments.
    if (build_in_kernel(b, batch, rows, columns) && x->a_parts <= 1 &&
        (x->mode != 2 || x->head_dim == 64 || x->head_dim == 128 || x->head_dim == 256)) {
        if (const TiledCopy *t = registered(b, d_weights, rows, columns)) {
            TileXform xf;
            xf.xmode = x->mode + 1;
            xf.b = x->b;
            xf.w = x->w;
            xf.off = x->off;
            xf.head_dim = x->head_dim;
            xf.eps = x->eps;
            xf.res_h = x->res_h;
            xf.res_sq = x->res_sums;
            xf.a_stride = x->a_stride;
            xf.b_stride = x->b_stride;
            return run_tile_matvec_mx(b, dtype, *t, rows, columns, batch, d_s_out,
                                      d_s_out ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE, nullptr, d_output, rows, 0, s, x->a,
                                      d_s_in, d_s_in ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE, xf);
        }
    }
    const bool reg = registered(b, d_weights, rows, columns) != nullptr;
    if ((x->res_sums || x->a_parts > 1) && !reg)
        return fail(CTOX_ERR_UNSUPPORTED_OPERATION, "residual sums and input partials need registered weights");
    ctox_status st = ensure(b, b->xa[layout], blocks * batch * 192, false);
    if (!st) st = ensure(b, b->xc[layout], blocks * batch * 4 * sizeof(float), false);
    if (st) return st;
    PrepXArgs a{};
    a.p.s_in = d_s_in;
    a.p.xa = (int8_t *)b->xa[layout].ptr;
    a.p.xc = (float *)b->xc[layout].ptr;
    a.p.columns = columns;
    a.p.batch = batch;
    a.p.dtype = (uint32_t)layout;
    a.p.s_in_kind = d_s_in ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE;
    a.p.tgroups = (batch + 3) / 4;
    a.a = x->a;
    a.b = x->b;
    a.w = x->w;
    a.mode = x->mode;
    a.a_stride = x->a_stride;
    a.b_stride = x->b_stride;
    a.off = x->off;
    a.head_dim = x->head_dim;
    a.eps = x->eps;
    a.a_parts = x->a_parts > 1 ? x->a_parts : 1u;
    a.a_pstride = x->a_part_stride;
    // input_staged: the producer already wrote exactly this staging (the
    // attention combine's gate staging of the o projection).
    if (!input_staged &&
        (st = launch(b->prep_x, dim3((unsigned)blocks, batch), dim3(64), s, a, "ctox_prep_transform_gfx950")))
        return st;
    return run_matvec(b, layout, dtype, d_weights, rows, columns, batch, d_s_out,
                      d_s_out ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE, nullptr, d_output, rows, 0, s, split_k != 0, parts,
                      x->res_h, x->res_sums, nx, staged);
}
}  // namespace

extern "C" ctox_status ctox_hip_transform_matvec_device(ctox_hip_backend *b, const ctox_input_transform *x,
                                                       int32_t dtype, const void *d_weights, const uint16_t *d_s_in,
                                                       const uint16_t *d_s_out, float *d_output, uint32_t rows,
                                                       uint32_t columns, uint32_t batch, uint32_t split_k,
                                                       uint32_t *parts, void *stream) {
    return transform_matvec_impl(b, x, dtype, d_weights, d_s_in, d_s_out, d_output, rows, columns, batch, split_k,
                                 parts, stream, nullptr, nullptr);
}

ctox_status ctox_delta_matvec_stage_next(ctox_hip_backend *b, const ctox_input_transform *x, int32_t dtype,
                                         const void *d_weights, const uint16_t *d_s_in, const uint16_t *d_s_out,
                                         float *d_output, uint32_t rows, uint32_t columns, uint32_t batch,
                                         const float *next_norm_w, const uint16_t *next_s_in, int32_t next_dtype,
                                         float *next_h_out, float *next_sq_out, bool *staged, void *stream,
                                         bool input_staged) {
    if (staged) *staged = false;
    if (input_staged && !ctox_small_m_staged(b, d_weights, batch, rows, columns))
        return fail(CTOX_ERR_INVALID_STATE, "a prestaged input needs the staged small-M path");
    if (!next_norm_w || !next_h_out || !next_sq_out || !staged || !x || !x->res_h || !x->res_sums)
        return fail(CTOX_ERR_SHAPE, "next-norm staging: null argument");
    if (next_dtype != CTOX_DTYPE_Q2B64 && next_dtype != CTOX_DTYPE_Q4B64)
        return fail(CTOX_ERR_UNSUPPORTED_DTYPE, "next-norm staging takes a pure Q2_B64 or Q4_B64 matrix");
    NextNorm nx;
    nx.w = next_norm_w;
    nx.s_in = next_s_in;
    nx.dtype = next_dtype;
    nx.h_out = next_h_out;
    nx.sq_out = next_sq_out;
    return transform_matvec_impl(b, x, dtype, d_weights, d_s_in, d_s_out, d_output, rows, columns, batch, 0, nullptr,
                                 stream, batch >= 2 && batch <= 8 ? &nx : nullptr, staged, input_staged);
}

ctox_status ctox_norm_matvec_prestaged(ctox_hip_backend *b, int32_t dtype, const void *d_weights,
                                       const uint16_t *d_s_out, float *d_output, uint32_t rows, uint32_t columns,
                                       uint32_t batch, const float *sq, float eps, uint32_t max_parts, uint32_t *parts,
                                       void *stream) {
    if (parts) *parts = 1;
    if (!b || !d_weights || !d_output || !sq) return fail(CTOX_ERR_SHAPE, "null argument");
    if (batch < 2 || batch > 8 || columns % kBlockLen || columns / kBlockLen > 128)
        return fail(CTOX_ERR_SHAPE, "prestaged norm-matvec: 2..8 rows, at most 8192 columns");
    const TiledCopy *t = registered(b, d_weights, rows, columns);
    if (!t) return fail(CTOX_ERR_UNSUPPORTED_OPERATION, "prestaged norm-matvec needs registered weights");
    const int nl = dtype == CTOX_DTYPE_Q4B64 ? 1 : 0;
    if (b->xn[nl].bytes < columns / kBlockLen * batch * 192)
        return fail(CTOX_ERR_INVALID_STATE, "no next-norm staging of this size");
    hipStream_t s = pick_stream(b, stream);
    StagedIn in;
    in.xa = (const int8_t *)b->xn[nl].ptr;
    in.xc = (const float *)b->xnc[nl].ptr;
    in.rms_sq = sq;
    in.rms_n = (uint32_t)(columns / kBlockLen);
    in.eps = eps;
    bool parts_out = false;
    if (parts && max_parts > 1 && t->chunks > 1 && t->chunks <= max_parts) {
        parts_out = true;
        *parts = t->chunks;
    }
    return run_tile_matvec_m(b, dtype, *t, rows, columns, batch, d_s_out, d_s_out ? CTOX_KSCALE_F16 : CTOX_KSCALE_NONE,
                             nullptr, d_output, rows, 0, s, nullptr, nullptr, parts_out, nullptr, nullptr, &in);
}

extern "C" ctox_status ctox_hip_fused_matvec(ctox_hip_backend *b, const ctox_fused_matvec *op, float *output,
                                             size_t output_len) {
    if (!b || !op || !output) return fail(CTOX_ERR_SHAPE, "null argument");
    size_t blocks;
    ctox_status st = validate_matvec(op, true, &blocks);
    if (st) return st;
    if (output_len != op->rows) return fail(CTOX_ERR_SHAPE, "output holds %zu, expected %zu", output_len, op->rows);
    ctox_hip_matrix *m = nullptr;
    st = prepare_impl(b, op, &m);
    if (st) return st;
    float *d_in = nullptr, *d_out = nullptr;
    hipError_t e = hipMalloc((void **)&d_in, op->columns * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&d_out, op->rows * sizeof(float));
    if (e == hipSuccess)
        e = hipMemcpyAsync(d_in, op->input, op->columns * sizeof(float), hipMemcpyHostToDevice, pick_stream(b, b->stream));
    if (e == hipSuccess) {
        bool prepped[2] = {false, false};
        st = dispatch_matrix(b, m, d_in, 1, d_out, b->stream, prepped, (uint32_t)op->activation);
        if (!st) e = hipMemcpyAsync(output, d_out, op->rows * sizeof(float), hipMemcpyDeviceToHost, b->stream);
        if (!st && e == hipSuccess) e = hipStreamSynchronize(b->stream);
    }
    if (d_in) (void)hipFree(d_in);
    if (d_out) (void)hipFree(d_out);
    ctox_hip_matrix_destroy(m);
    if (e != hipSuccess) return fail(CTOX_ERR_INVALID_STATE, "HIP fused matvec failed: %s", hipGetErrorString(e));
    if (st) return st;
    return check_finite_host(output, op->rows, "fused matvec");
}

extern "C" ctox_status ctox_hip_fused_matvec_fanout(ctox_hip_backend *b, const ctox_fused_matvec *ops,
                                                    size_t n, float *const *outputs) {
    if (!b || !ops || !outputs) return fail(CTOX_ERR_SHAPE, "null argument");
    if (n == 0) return fail(CTOX_ERR_SHAPE, "HIP fan-out requires at least one projection");
    // Results equal independent calls by construction (the activation
    // conversion is a pure function of input and s_in).
    for (size_t i = 0; i < n; i++) {
        ctox_status st = ctox_hip_fused_matvec(b, &ops[i], outputs[i], ops[i].rows);
        if (st) return st;
    }
    return CTOX_OK;
}

extern "C" ctox_status ctox_hip_recovered_row(ctox_hip_backend *b, const ctox_recovered_row *op, float *output,
                                              size_t output_len) {
    if (!b || !op || !output) return fail(CTOX_ERR_SHAPE, "null argument");
    // Q/src/backend/cpu.rs:312-337
    if (op->columns == 0 || op->columns % kBlockLen)
        return fail(CTOX_ERR_SHAPE, "recovered row columns must be non-zero and divisible by 64");
    if (op->s_in.len != op->columns || !std::isfinite(op->s_out) || op->s_in.kind == CTOX_SCALE_NONE)
        return fail(CTOX_ERR_SHAPE, "recovered row scale contract differs");
    const size_t bb = block_bytes(op->dtype);
    if (!bb) return fail(CTOX_ERR_UNSUPPORTED_DTYPE, "unsupported quantization dtype %d", op->dtype);
    const size_t expected = op->columns / kBlockLen * bb;
    if (op->weights_len != expected)
        return fail(CTOX_ERR_SHAPE, "recovered row has %zu packed bytes, expected %zu", op->weights_len, expected);
    if (output_len != op->columns) return fail(CTOX_ERR_SHAPE, "output holds %zu, expected %zu", output_len, op->columns);
    if (!block_scales_finite(op->weights, 1, op->columns / kBlockLen, bb))
        return fail(CTOX_ERR_INVALID_ARTIFACT, "recovered row block scale is non-finite");
    size_t bad;
    if (!scale_finite(op->s_in, &bad))
        return fail(CTOX_ERR_INVALID_ARTIFACT, "recovery scale %zu is non-finite", bad);
    HIP_TRY(hipSetDevice(b->device));
    void *d_w = nullptr, *d_s = nullptr, *d_o = nullptr;
    ctox_status st = upload(op->weights, op->weights_len, &d_w);
    const size_t sbytes = op->s_in.len * (op->s_in.kind == CTOX_SCALE_F32 ? 4 : 2);
    if (!st) st = upload(op->s_in.data, sbytes, &d_s);
    if (!st && hipMalloc(&d_o, op->columns * sizeof(float)) != hipSuccess)
        st = fail(CTOX_ERR_INVALID_STATE, "hipMalloc failed");
    if (!st) {
        RecoveredRowArgs a{};
        a.weights = (const uint8_t *)d_w;
        a.s_in = d_s;
        a.output = (float *)d_o;
        a.columns = (uint32_t)op->columns;
        a.dtype = op->dtype == CTOX_DTYPE_Q4B64 ? 1u : 0u;
        a.s_in_kind = kernel_scale_kind(op->s_in.kind);
        a.s_out = op->s_out;
        st = launch(b->rec_row, dim3((unsigned)((op->columns + 255) / 256)), dim3(256), pick_stream(b, b->stream), a,
                    "ctox_recovered_row_gfx950");
        if (!st && (hipMemcpyAsync(output, d_o, op->columns * sizeof(float), hipMemcpyDeviceToHost, b->stream) !=
                        hipSuccess ||
                    hipStreamSynchronize(b->stream) != hipSuccess))
            st = fail(CTOX_ERR_INVALID_STATE, "recovered row readback failed");
    }
    if (d_w) (void)hipFree(d_w);
    if (d_s) (void)hipFree(d_s);
    if (d_o) (void)hipFree(d_o);
    return st;
}

extern "C" ctox_status ctox_hip_recovered_row_matvec(ctox_hip_backend *b, const ctox_recovered_row_matvec *op,
                                                     float *result) {
    if (!b || !op || !result) return fail(CTOX_ERR_SHAPE, "null argument");
    // Q/src/backend/cpu.rs:478-497
    bool finite = op->len > 0 && op->len % kBlockLen == 0 && std::isfinite(op->s_out);
    for (size_t i = 0; finite && i < op->len; i++) finite = std::isfinite(op->corrected_input[i]);
    if (!finite) return fail(CTOX_ERR_SHAPE, "recovered row matvec input or output scale is invalid");
    const size_t bb = block_bytes(op->dtype);
    if (!bb) return fail(CTOX_ERR_UNSUPPORTED_DTYPE, "unsupported quantization dtype %d", op->dtype);
    if (op->weights_len < op->len / kBlockLen * bb)
        return fail(CTOX_ERR_SHAPE, "recovered row has %zu packed bytes, expected %zu", op->weights_len,
                    op->len / kBlockLen * bb);
    if (!block_scales_finite(op->weights, 1, op->len / kBlockLen, bb))
        return fail(CTOX_ERR_INVALID_ARTIFACT, "%s block scale is non-finite",
                    op->dtype == CTOX_DTYPE_Q2B64 ? "Q2" : "Q4");
    HIP_TRY(hipSetDevice(b->device));
    void *d_w = nullptr, *d_x = nullptr, *d_r = nullptr;
    ctox_status st = upload(op->weights, op->len / kBlockLen * bb, &d_w);
    if (!st) st = upload(op->corrected_input, op->len * sizeof(float), &d_x);
    if (!st && hipMalloc(&d_r, sizeof(float)) != hipSuccess) st = fail(CTOX_ERR_INVALID_STATE, "hipMalloc failed");
    if (!st) {
        RowDotArgs a{};
        a.weights = (const uint8_t *)d_w;
        a.x = (const float *)d_x;
        a.result = (float *)d_r;
        a.len = (uint32_t)op->len;
        a.dtype = op->dtype == CTOX_DTYPE_Q4B64 ? 1u : 0u;
        a.s_out = op->s_out;
        st = launch(b->row_dot, dim3(1), dim3(64), pick_stream(b, b->stream), a, "ctox_row_dot_gfx950");
        if (!st && (hipMemcpyAsync(result, d_r, sizeof(float), hipMemcpyDeviceToHost, b->stream) != hipSuccess ||
                    hipStreamSynchronize(b->stream) != hipSuccess))
            st = fail(CTOX_ERR_INVALID_STATE, "row matvec readback failed");
    }
    if (d_w) (void)hipFree(d_w);
    if (d_x) (void)hipFree(d_x);
    if (d_r) (void)hipFree(d_r);
    if (!st && !std::isfinite(*result)) return fail(CTOX_ERR_INVALID_STATE, "row matvec produced a non-finite value");
    return st;
}

// ======================================================================
// gated delta
// ======================================================================
namespace {
ctox_status gdn_shape(size_t tokens, size_t heads, size_t kd, size_t vd) {
    if (tokens == 0 || heads == 0 || kd == 0 || vd == 0)
        return fail(CTOX_ERR_SHAPE, "delta shapes must be non-zero");
    if (kd > 16 * 16)
        return fail(CTOX_ERR_UNSUPPORTED_OPERATION,
                    "backend hip cannot execute gated delta: key_dim %zu exceeds 256", kd);
    if (tokens * heads > 0x7fffffffu) return fail(CTOX_ERR_SHAPE, "delta sequence too long");
    return CTOX_OK;
}

// key_heads = 0 means heads (no repeat); strides of 0 mean dense token rows.
ctox_status gdn_device(ctox_hip_backend *b, const float *q, const float *k, const float *v, const float *ld,
                       const float *beta, float *state, size_t tokens, size_t heads, size_t kd, size_t vd,
                       size_t chunk, float *out, hipStream_t s, size_t key_heads = 0, size_t qk_stride = 0,
                       size_t v_stride = 0) {
    ctox_status st = gdn_shape(tokens, heads, kd, vd);
    if (st) return st;
    if (key_heads == 0) key_heads = heads;
    if (qk_stride == 0) qk_stride = key_heads * kd;
    if (v_stride == 0) v_stride = heads * vd;
    // Q/src/decoder.rs:868-880: value heads repeat whole key heads.
    if (heads % key_heads || qk_stride < key_heads * kd || v_stride < heads * vd || qk_stride > 0xffffffffu ||
        v_stride > 0xffffffffu)
        return fail(CTOX_ERR_SHAPE, "delta head repeat or token strides do not fit the heads");
    // chunk >= 1 selects the chunked (WY) prefill for key/value dims up to
    // 128 and chunks up to 64 tokens; otherwise the token-serial scan.
    const bool chunked = tokens > 1 && chunk >= 1 && chunk <= 64 && kd <= 128 && vd <= 128;
    const size_t nch = chunked ? (tokens + chunk - 1) / chunk : 0;
    const size_t scratch = chunked ? heads * nch * (2 * 64 * 64 + 4 * 64) : 1;
    st = ensure(b, b->norms, scratch * sizeof(float), false);
    if (st) return st;
    GdnArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.log_decay = ld;
    a.beta = beta;
    a.state = state;
    a.out = out;
    a.norms = (float *)b->norms.ptr;
    a.tokens = (uint32_t)tokens;
    a.heads = (uint32_t)heads;
    a.key_dim = (uint32_t)kd;
    a.value_dim = (uint32_t)vd;
    a.chunk = (uint32_t)chunk;
    a.rep = (uint32_t)(heads / key_heads);
    a.qk_stride = (uint32_t)qk_stride;
    a.v_stride = (uint32_t)v_stride;
    const size_t slices = (vd + 15) / 16;
    if (chunked) {
        st = launch(b->gdn_chunk_prep, dim3((unsigned)(heads * nch)), dim3(256), s, a, "ctox_gdn_chunk_prep_gfx950");
        if (st) return st;
        // 8 * ceil(heads / 8) * slices workgroups: the kernel maps them so
        // that all slices of a head run on one XCD (surplus ones exit).
        // The vector instantiation: 16-byte branch-free loads; it needs the
        // shapes, strides and alignment below.
        const bool vec = kd % 4 == 0 && vd % 16 == 0 && qk_stride % 4 == 0 && v_stride % 4 == 0 &&
                         (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) & 15) == 0 && chunk * qk_stride < 0x1ffffff0u &&
                         chunk * v_stride < 0x1ffffff0u;
        return launch(vec ? b->gdn_chunk_scan_vec : b->gdn_chunk_scan, dim3((unsigned)(8 * ((heads + 7) / 8) * slices)),
                      dim3(256), s, a, vec ? "ctox_gdn_chunk_scan_vec_gfx950" : "ctox_gdn_chunk_scan_gfx950");
    }
    return launch(b->gdn_scan, dim3((unsigned)(heads * slices)), dim3(256), s, a, "ctox_gdn_scan_gfx950");
}

// Q/src/reference.rs:18-34
ctox_status contract(const float *v, size_t rows, size_t cols, const char *what) {
    for (size_t i = 0; i < rows * cols; i++)
        if (!std::isfinite(v[i])) return fail(CTOX_ERR_INVALID_ARTIFACT, "%s input is non-finite", what);
    return CTOX_OK;
}

ctox_status gdn_host(ctox_hip_backend *b, const float *q, const float *k, const float *v, const float *ld,
                     const float *beta, float *state, size_t tokens, size_t heads, size_t kd, size_t vd,
                     size_t chunk, float *out, bool sequence) {
    if (!b || !q || !k || !v || !ld || !beta || !state || !out) return fail(CTOX_ERR_SHAPE, "null argument");
    ctox_status st = gdn_shape(tokens, heads, kd, vd);
    if (st) return st;
    if ((st = contract(q, tokens, heads * kd, "delta query"))) return st;
    if ((st = contract(k, tokens, heads * kd, "delta key"))) return st;
    if ((st = contract(v, tokens, heads * vd, "delta value"))) return st;
    if (sequence) {
        if ((st = contract(ld, tokens, heads, "delta sequence decay"))) return st;
        if ((st = contract(beta, tokens, heads, "delta sequence beta"))) return st;
    }
    for (size_t i = 0; i < heads * kd * vd; i++)
        if (!std::isfinite(state[i])) return fail(CTOX_ERR_SHAPE, "delta state contract differs");
    for (size_t i = 0; i < tokens * heads; i++)
        if (!std::isfinite(ld[i]) || !std::isfinite(beta[i]))
            return fail(CTOX_ERR_SHAPE, "delta state contract differs");
    HIP_TRY(hipSetDevice(b->device));
    const size_t nq = tokens * heads * kd, nv = tokens * heads * vd, ns = heads * kd * vd, ng = tokens * heads;
    void *dq = nullptr, *dk = nullptr, *dv = nullptr, *dl = nullptr, *db = nullptr, *ds = nullptr, *dout = nullptr;
    st = upload(q, nq * 4, &dq);
    if (!st) st = upload(k, nq * 4, &dk);
    if (!st) st = upload(v, nv * 4, &dv);
    if (!st) st = upload(ld, ng * 4, &dl);
    if (!st) st = upload(beta, ng * 4, &db);
    if (!st) st = upload(state, ns * 4, &ds);
    if (!st && hipMalloc(&dout, nv * 4) != hipSuccess) st = fail(CTOX_ERR_INVALID_STATE, "hipMalloc failed");
    if (!st)
        st = gdn_device(b, (float *)dq, (float *)dk, (float *)dv, (float *)dl, (float *)db, (float *)ds, tokens,
                        heads, kd, vd, chunk, (float *)dout, pick_stream(b, b->stream));
    if (!st && (hipMemcpyAsync(out, dout, nv * 4, hipMemcpyDeviceToHost, b->stream) != hipSuccess ||
                hipMemcpyAsync(state, ds, ns * 4, hipMemcpyDeviceToHost, b->stream) != hipSuccess ||
                hipStreamSynchronize(b->stream) != hipSuccess))
        st = fail(CTOX_ERR_INVALID_STATE, "gated delta readback failed");
    void *all[] = {dq, dk, dv, dl, db, ds, dout};
    for (void *p : all)
        if (p) (void)hipFree(p);
    if (!st) st = check_finite_host(out, nv, "gated delta");
    return st;
}
}  // namespace

extern "C" ctox_status ctox_hip_gated_delta_step(ctox_hip_backend *b, const float *q, const float *k,
                                                 const float *v, const float *log_decay, const float *beta,
                                                 float *state, size_t heads, size_t key_dim, size_t value_dim,
                                                 float *out) {
    return gdn_host(b, q, k, v, log_decay, beta, state, 1, heads, key_dim, value_dim, 0, out, false);
}

extern "C" ctox_status ctox_hip_gated_delta_sequence(ctox_hip_backend *b, const float *q, const float *k,
                                                     const float *v, const float *log_decay,
                                                     const float *beta, float *state, size_t tokens,
                                                     size_t heads, size_t key_dim, size_t value_dim,
                                                     size_t chunk, float *out) {
    return gdn_host(b, q, k, v, log_decay, beta, state, tokens, heads, key_dim, value_dim, chunk, out, true);
}

extern "C" ctox_status ctox_hip_gated_delta_step_device(ctox_hip_backend *b, const float *q, const float *k,
                                                        const float *v, const float *log_decay,
                                                        const float *beta, float *state, size_t heads,
                                                        size_t key_dim, size_t value_dim, float *out,
                                                        void *stream) {
    if (!b || !q || !k || !v || !log_decay || !beta || !state || !out) return fail(CTOX_ERR_SHAPE, "null argument");
    return gdn_device(b, q, k, v, log_decay, beta, state, 1, heads, key_dim, value_dim, 0, out,
                      pick_stream(b, stream));
}

extern "C" ctox_status ctox_hip_gated_delta_sequence_device(ctox_hip_backend *b, const float *q, const float *k,
                                                            const float *v, const float *log_decay,
                                                            const float *beta, float *state, size_t tokens,
                                                            size_t heads, size_t key_dim, size_t value_dim,
                                                            size_t chunk, float *out, void *stream) {
    if (!b || !q || !k || !v || !log_decay || !beta || !state || !out) return fail(CTOX_ERR_SHAPE, "null argument");
    return gdn_device(b, q, k, v, log_decay, beta, state, tokens, heads, key_dim, value_dim, chunk, out,
                      pick_stream(b, stream));
}

extern "C" ctox_status ctox_hip_gated_delta_strided_device(ctox_hip_backend *b, const float *q, const float *k,
                                                           const float *v, size_t qk_stride, size_t v_stride,
                                                           const float *log_decay, const float *beta, float *state,
                                                           size_t tokens, size_t heads, size_t key_heads,
                                                           size_t key_dim, size_t value_dim, size_t chunk,
                                                           float *out, void *stream) {
    if (!b || !q || !k || !v || !log_decay || !beta || !state || !out) return fail(CTOX_ERR_SHAPE, "null argument");
    if (key_heads == 0) return fail(CTOX_ERR_SHAPE, "delta key heads must be non-zero");
    return gdn_device(b, q, k, v, log_decay, beta, state, tokens, heads, key_dim, value_dim, chunk, out,
                      pick_stream(b, stream), key_heads, qk_stride, v_stride);
}

namespace {
ctox_status gdn_fused_impl(ctox_hip_backend *b, const float *d_proj, size_t proj_stride, size_t a_off, size_t b_off,
                           const float *d_conv_w, const float *d_conv_in, float *d_conv_out, size_t kernel,
                           const float *d_a_log, const float *d_dt_bias, float *d_log_decay, float *d_beta,
                           int gates_given, const float *d_state_in, float *d_state_out, size_t snap_stride,
                           size_t conv_snap_stride, int blocked, size_t tokens, size_t heads, size_t key_heads,
                           size_t key_dim, size_t value_dim, float *d_out, void *stream) {
    if (!b || !d_proj || !d_conv_w || !d_conv_in || !d_conv_out || !d_log_decay || !d_beta || !d_state_in ||
        !d_state_out || !d_out || (!gates_given && (!d_a_log || !d_dt_bias)))
        return fail(CTOX_ERR_SHAPE, "null argument");
    ctox_status st = gdn_shape(tokens, heads, key_dim, value_dim);
    if (st) return st;
    const size_t channels = 2 * key_heads * key_dim + heads * value_dim;
    if (key_heads == 0 || heads % key_heads || key_dim > 128 || kernel == 0 || kernel > 8 ||
        proj_stride < channels || a_off + heads > proj_stride || b_off + heads > proj_stride ||
        proj_stride > 0x7fffffffu || tokens > 65536)
        return fail(CTOX_ERR_SHAPE, "fused gated delta shapes");
    // The conv windows written (every snapshot, or the final one) never
    // overlap the ones read: other workgroups still read them.
    const size_t cw = channels * kernel;
    const size_t sw = blocked ? heads * ((value_dim + 15) / 16) * 2048 : heads * key_dim * value_dim;
    if (blocked && (((uintptr_t)d_state_in | (uintptr_t)d_state_out) % 16 || (snap_stride % 4)))
        return fail(CTOX_ERR_SHAPE, "blocked gated delta state needs 16-byte alignment");
    const size_t nsnap = snap_stride ? tokens : 1;
    if ((snap_stride && (snap_stride < sw || conv_snap_stride < cw)) || (!snap_stride && conv_snap_stride))
        return fail(CTOX_ERR_SHAPE, "fused gated delta snapshot strides");
    for (size_t t = 0; t < nsnap; t++) {
        const float *o = d_conv_out + t * conv_snap_stride;
        if (o < d_conv_in + cw && d_conv_in < o + cw)
            return fail(CTOX_ERR_SHAPE, "fused gated delta conv windows must not alias");
    }
    GdnFusedArgs a{};
    a.proj = d_proj;
    a.conv_w = d_conv_w;
    a.conv_in = d_conv_in;
    a.conv_out = d_conv_out;
    a.a_log = d_a_log;
    a.dt_bias = d_dt_bias;
    a.log_decay = d_log_decay;
    a.beta = d_beta;
    a.state = (float *)d_state_in;
    a.state_out = d_state_out;
    a.snap_stride = snap_stride;
    a.conv_snap_stride = conv_snap_stride;
    a.out = d_out;
    a.tokens = (uint32_t)tokens;
    a.heads = (uint32_t)heads;
    a.key_heads = (uint32_t)key_heads;
    a.key_dim = (uint32_t)key_dim;
    a.value_dim = (uint32_t)value_dim;
    a.kernel = (uint32_t)kernel;
    a.proj_stride = (uint32_t)proj_stride;
    a.a_off = (uint32_t)a_off;
    a.b_off = (uint32_t)b_off;
    a.gates_given = gates_given ? 1u : 0u;
    a.state_blocked = blocked ? 1u : 0u;
    const size_t slices = (value_dim + 15) / 16;
    const bool one = b->gdn_one && tokens == 1;
    hipFunction_t f = kernel == 4 ? b->gdn_k4[one ? 1 : 0][a.state_blocked]
                                  : one ? (a.state_blocked ? b->gdn_fused1_blk : b->gdn_fused1)
                                        : (a.state_blocked ? b->gdn_fused_blk : b->gdn_fused);
    return launch(f, dim3((unsigned)(heads * slices)), dim3(256), pick_stream(b, stream), a, "ctox_gdn_fused_gfx950");
}
}  // namespace

extern "C" ctox_status ctox_hip_gdn_fused_device(ctox_hip_backend *b, const float *d_proj, size_t proj_stride,
                                                 size_t a_off, size_t b_off, const float *d_conv_w,
                                                 const float *d_conv_in, float *d_conv_out, size_t kernel,
                                                 const float *d_a_log, const float *d_dt_bias, float *d_log_decay,
                                                 float *d_beta, int gates_given, float *d_state, size_t tokens,
                                                 size_t heads, size_t key_heads, size_t key_dim, size_t value_dim,
                                                 float *d_out, void *stream) {
    return gdn_fused_impl(b, d_proj, proj_stride, a_off, b_off, d_conv_w, d_conv_in, d_conv_out, kernel, d_a_log,
                          d_dt_bias, d_log_decay, d_beta, gates_given, d_state, d_state, 0, 0, 0, tokens, heads,
                          key_heads, key_dim, value_dim, d_out, stream);
}

extern "C" ctox_status ctox_hip_gdn_fused_snap_device(ctox_hip_backend *b, const float *d_proj, size_t proj_stride,
                                                      size_t a_off, size_t b_off, const float *d_conv_w,
                                                      const float *d_conv_in, float *d_conv_out,
                                                      size_t conv_snap_stride, size_t kernel, const float *d_a_log,
                                                      const float *d_dt_bias, float *d_log_decay, float *d_beta,
                                                      const float *d_state_in, float *d_state_out,
                                                      size_t snap_stride, int blocked, size_t tokens, size_t heads,
                                                      size_t key_heads, size_t key_dim, size_t value_dim,
                                                      float *d_out, void *stream) {
    if (snap_stride == 0) return fail(CTOX_ERR_SHAPE, "snapshot stride must be non-zero");
    return gdn_fused_impl(b, d_proj, proj_stride, a_off, b_off, d_conv_w, d_conv_in, d_conv_out, kernel, d_a_log,
                          d_dt_bias, d_log_decay, d_beta, 0, d_state_in, d_state_out, snap_stride, conv_snap_stride,
                          blocked, tokens, heads, key_heads, key_dim, value_dim, d_out, stream);
}

// ======================================================================
// decode-step glue and token selection
// ======================================================================
namespace {
constexpr size_t kMaxDrafts = 64;
}

extern "C" ctox_status ctox_hip_gdn_gates_device(ctox_hip_backend *b, const float *d_a, const float *d_b,
                                                 const float *d_a_log, const float *d_dt_bias, size_t tokens,
                                                 size_t heads, float *d_log_decay, float *d_beta, void *stream) {
    if (!b || !d_a || !d_b || !d_a_log || !d_dt_bias || !d_log_decay || !d_beta)
        return fail(CTOX_ERR_SHAPE, "null argument");
    if (tokens == 0 || heads == 0 || tokens * heads > 0x7fffffffu) return fail(CTOX_ERR_SHAPE, "gate shapes");
    GateArgs a{d_a, d_b, d_a_log, d_dt_bias, d_log_decay, d_beta, (uint32_t)tokens, (uint32_t)heads, (uint32_t)heads, 0};
    return launch(b->gates, dim3((unsigned)((tokens * heads + 255) / 256)), dim3(256), pick_stream(b, stream), a,
                  "ctox_gdn_gates_gfx950");
}

extern "C" ctox_status ctox_hip_gdn_gates_strided_device(ctox_hip_backend *b, const float *d_a, const float *d_b,
                                                         size_t in_stride, const float *d_a_log,
                                                         const float *d_dt_bias, size_t tokens, size_t heads,
                                                         float *d_log_decay, float *d_beta, void *stream) {
    if (!b || !d_a || !d_b || !d_a_log || !d_dt_bias || !d_log_decay || !d_beta)
        return fail(CTOX_ERR_SHAPE, "null argument");
    if (tokens == 0 || heads == 0 || tokens * heads > 0x7fffffffu || in_stride < heads || in_stride > 0x7fffffffu)
        return fail(CTOX_ERR_SHAPE, "gate shapes");
    GateArgs a{d_a, d_b, d_a_log, d_dt_bias, d_log_decay, d_beta, (uint32_t)tokens, (uint32_t)heads,
               (uint32_t)in_stride, 0};
    return launch(b->gates, dim3((unsigned)((tokens * heads + 255) / 256)), dim3(256), pick_stream(b, stream), a,
                  "ctox_gdn_gates_gfx950");
}

extern "C" ctox_status ctox_hip_repeat_heads_device(ctox_hip_backend *b, const float *d_in, size_t rows,
                                                    size_t heads, size_t dim, size_t repeats, float *d_out,
                                                    void *stream) {
    if (!b || !d_in || !d_out) return fail(CTOX_ERR_SHAPE, "null argument");
    // Q/src/decoder.rs:47-65 rejects empty shapes.
    if (rows == 0 || heads == 0 || dim == 0 || repeats == 0) return fail(CTOX_ERR_SHAPE, "repeat_heads shapes must be non-zero");
    const size_t n = rows * heads * repeats * dim;
    if (n / repeats != rows * heads * dim || (n + 255) / 256 > 0x7fffffffu) return fail(CTOX_ERR_SHAPE, "repeat_heads too large");
    RepeatArgs a{d_in, d_out, (uint32_t)rows, (uint32_t)heads, (uint32_t)dim, (uint32_t)repeats};
    return launch(b->repeat, dim3((unsigned)((n + 255) / 256)), dim3(256), pick_stream(b, stream), a,
                  "ctox_repeat_heads_gfx950");
}

namespace {
// Parts per vocabulary row for the partial reductions: ~2.4k logits each.
uint32_t row_parts(size_t vocab) { return (uint32_t)std::min<size_t>(64, std::max<size_t>(1, vocab / 2048)); }
}

extern "C" ctox_status ctox_hip_greedy_tokens_device(ctox_hip_backend *b, const float *d_logits, size_t rows,
                                                     size_t vocab, uint32_t *d_tokens, void *stream) {
    return ctox_greedy_tokens_mapped(b, d_logits, rows, vocab, nullptr, d_tokens, stream);
}

ctox_status ctox_greedy_tokens_mapped(ctox_hip_backend *b, const float *d_logits, size_t rows, size_t vocab,
                                      const uint32_t *d_ids, uint32_t *d_tokens, void *stream) {
    if (!b || !d_logits || !d_tokens) return fail(CTOX_ERR_SHAPE, "null argument");
    if (vocab == 0) return fail(CTOX_ERR_INVALID_ARTIFACT, "cannot select a token from empty logits");
    if (rows == 0 || rows > 65535 || vocab > 0xffffffffu) return fail(CTOX_ERR_SHAPE, "logits shape");
    hipStream_t s = pick_stream(b, stream);
    const uint32_t parts = row_parts(vocab);
    ctox_status st = ensure(b, b->tok, rows * parts * 2 * sizeof(float), false);
    if (st) return st;
    PartialArgs p{d_logits, d_logits, d_logits, (float *)b->tok.ptr, (uint32_t)rows, (uint32_t)vocab, parts, 0, 1.0f,
                  (uint32_t)vocab};
    if ((st = launch(b->partials, dim3((unsigned)rows, parts), dim3(256), s, p, "ctox_row_partials_gfx950"))) return st;
    VerifyArgs v{(const float *)b->tok.ptr, d_tokens, (uint32_t)rows, parts, d_ids};
    return launch(b->argmax_final, dim3((unsigned)rows), dim3(64), s, v, "ctox_argmax_final_gfx950");
}

extern "C" ctox_status ctox_hip_verify_greedy_mtp_device(ctox_hip_backend *b, const float *d_draft,
                                                         const float *d_target, const float *d_bonus, size_t drafts,
                                                         size_t vocab, uint32_t *d_out, void *stream) {
    if (!b || !d_draft || !d_target || !d_bonus || !d_out) return fail(CTOX_ERR_SHAPE, "null argument");
    if (vocab == 0) return fail(CTOX_ERR_INVALID_ARTIFACT, "cannot select a token from empty logits");
    if (drafts == 0 || drafts > kMaxDrafts || vocab > 0xffffffffu) return fail(CTOX_ERR_SHAPE, "drafts outside 1..64");
    hipStream_t s = pick_stream(b, stream);
    const uint32_t parts = row_parts(vocab);
    const size_t rows = 2 * drafts + 1;
    ctox_status st = ensure(b, b->tok, rows * parts * 2 * sizeof(float), false);
    if (st) return st;
    PartialArgs p{d_draft, d_target, d_bonus, (float *)b->tok.ptr, (uint32_t)drafts, (uint32_t)vocab, parts, 0, 1.0f,
                  (uint32_t)vocab};
    if ((st = launch(b->partials, dim3((unsigned)rows, parts), dim3(256), s, p, "ctox_row_partials_gfx950"))) return st;
    VerifyArgs v{(const float *)b->tok.ptr, d_out, (uint32_t)drafts, parts};
    return launch(b->verify, dim3(1), dim3(64), s, v, "ctox_verify_greedy_gfx950");
}

extern "C" ctox_status ctox_hip_mtp_accept_restricted_device(
    ctox_hip_backend *b, const float *d_draft, size_t draft_vocab, const uint32_t *d_draft_inv, const float *d_target,
    const float *d_bonus, const uint32_t *d_bonus_ids, const uint32_t *d_tokens, size_t drafts, size_t vocab,
    float temperature, uint64_t *d_rng, uint32_t *d_out, void *stream) {
    if (!b || !d_bonus || !d_tokens || !d_rng || !d_out || (drafts && (!d_draft || !d_target)))
        return fail(CTOX_ERR_SHAPE, "null argument");
    if (!(temperature > 0.0f) || !std::isfinite(temperature) || !std::isfinite(1.0f / temperature))
        return fail(CTOX_ERR_INVALID_ARTIFACT, "sampling temperature must be finite and positive");
    if (vocab == 0) return fail(CTOX_ERR_INVALID_ARTIFACT, "cannot sample from empty logits");
    // The final search scans one part per pass with 1024 threads.
    if (drafts > kMaxDrafts || vocab > (size_t)1024 * 1024) return fail(CTOX_ERR_SHAPE, "drafts outside 0..64 or vocab above 2^20");
    if (draft_vocab == 0 || draft_vocab > vocab || (draft_vocab < vocab && drafts && !d_draft_inv))
        return fail(CTOX_ERR_SHAPE, "restricted draft rows need 1..vocab scores and the token-to-index map");
    hipStream_t s = pick_stream(b, stream);
    const uint32_t parts = row_parts(vocab);
    const uint32_t parts2 = (uint32_t)std::max<size_t>(256, (vocab + 1023) / 1024);
    const size_t rows = 2 * drafts + 1;
    const size_t state_off = ((rows * parts * 2 + parts2) * sizeof(float) + 255) & ~(size_t)255;
    ctox_status st = ensure(b, b->stats, state_off + sizeof(PickState), false);
    if (st) return st;
    float *partials = (float *)b->stats.ptr;
    AcceptArgs a{};
    a.draft = d_draft;
    a.target = d_target;
    a.bonus = d_bonus;
    a.tokens = d_tokens;
    a.partials = partials;
    a.sums = partials + rows * parts * 2;
    a.state = (PickState *)((char *)b->stats.ptr + state_off);
    a.rng = d_rng;
    a.out = d_out;
    a.draft_inv = draft_vocab < vocab ? d_draft_inv : nullptr;
    a.bonus_ids = d_bonus_ids;
    a.drafts = (uint32_t)drafts;
    a.vocab = (uint32_t)vocab;
    a.parts = parts;
    a.parts2 = parts2;
    a.temperature = temperature;
    a.draft_vocab = (uint32_t)draft_vocab;
    PartialArgs p{d_draft, d_target, d_bonus, partials, (uint32_t)drafts, (uint32_t)vocab, parts, 1, temperature,
                  (uint32_t)draft_vocab};
    if ((st = launch(b->partials, dim3((unsigned)rows, parts), dim3(256), s, p, "ctox_row_partials_gfx950"))) return st;
    if ((st = launch(b->decide, dim3(1), dim3(64), s, a, "ctox_mtp_decide_gfx950"))) return st;
    if ((st = launch(b->pick_sums, dim3(parts2), dim3(256), s, a, "ctox_pick_sums_gfx950"))) return st;
    return launch(b->pick_final, dim3(1), dim3(1024), s, a, "ctox_pick_final_gfx950");
}

extern "C" ctox_status ctox_hip_mtp_accept_device(ctox_hip_backend *b, const float *d_draft, const float *d_target,
                                                  const float *d_bonus, const uint32_t *d_tokens, size_t drafts,
                                                  size_t vocab, float temperature, uint64_t *d_rng, uint32_t *d_out,
                                                  void *stream) {
    if (!b || !d_draft || !d_target || !d_bonus || !d_tokens || !d_rng || !d_out)
        return fail(CTOX_ERR_SHAPE, "null argument");
    return ctox_hip_mtp_accept_restricted_device(b, d_draft, vocab, nullptr, d_target, d_bonus, nullptr, d_tokens,
                                                 drafts, vocab, temperature, d_rng, d_out, stream);
}

extern "C" ctox_status ctox_hip_sample_topk_topp_device(ctox_hip_backend *b, const float *d_logits, size_t vocab,
                                                        float temperature, uint32_t top_k, float top_p, float draw,
                                                        uint32_t *d_out, void *stream) {
    if (!b || !d_logits || !d_out) return fail(CTOX_ERR_SHAPE, "null argument");
    // Q/src/sampler.rs:65-78, 84-89 argument checks.
    if (vocab == 0) return fail(CTOX_ERR_INVALID_ARTIFACT, "sampler logits are empty or non-finite");
    if (!std::isfinite(draw) || !(draw >= 0.0f && draw < 1.0f))
        return fail(CTOX_ERR_INVALID_ARTIFACT, "sampler draw must be finite and in [0, 1)");
    if (!std::isfinite(temperature) || temperature < 0.0f || !std::isfinite(top_p) || !(top_p > 0.0f) || top_p > 1.0f)
        return fail(CTOX_ERR_INVALID_ARTIFACT, "sampler temperature or top_p is invalid");
    hipStream_t s = pick_stream(b, stream);
    if (temperature == 0.0f) {  // greedy: the later token wins ties (sampler.rs:76-82)
        if ((uintptr_t)d_logits % 16) return fail(CTOX_ERR_SHAPE, "greedy sampling needs 16-byte aligned logits");
        ctox_status st = ctox_hip_greedy_tokens_device(b, d_logits, 1, vocab, d_out, s);
        if (st) return st;
        // Non-finite logits are refused before the greedy branch (sampler.rs:66-70):
        // finite flags of 64 ranges, then the status words.
        constexpr uint32_t kParts = 64;
        if ((st = ensure(b, b->stats, kParts * sizeof(uint32_t), false))) return st;
        uint32_t *flags = (uint32_t *)b->stats.ptr;
        FiniteArgs fa{d_logits, flags, (uint64_t)vocab};
        if ((st = launch(b->finite, dim3(kParts), dim3(256), s, fa, "ctox_finite_check_gfx950"))) return st;
        FlagStatusArgs ga{flags, d_out, kParts};
        return launch(b->greedy_status, dim3(1), dim3(64), s, ga, "ctox_greedy_status_gfx950");
    }
    const float invt = 1.0f / temperature;
    if (!std::isfinite(invt)) return fail(CTOX_ERR_INVALID_ARTIFACT, "sampler inverse temperature must be finite");
    const size_t parts = (vocab + CTOX_TOPK_PART - 1) / CTOX_TOPK_PART;
    if (top_k == 0 || top_k > CTOX_TOPK_MAX || parts * top_k > CTOX_TOPK_CANDS || vocab > 0xffffffffu)
        return fail(CTOX_ERR_UNSUPPORTED_OPERATION,
                    "device sampling takes 1 <= top_k <= %d and parts * top_k <= %d (full-vocabulary top_p is not built)",
                    CTOX_TOPK_MAX, CTOX_TOPK_CANDS);
    const size_t flags_off = (parts * top_k * sizeof(uint64_t) + 255) & ~(size_t)255;
    ctox_status st = ensure(b, b->stats, flags_off + parts * sizeof(uint32_t), false);
    if (st) return st;
    TopkArgs a{};
    a.logits = d_logits;
    a.cand = (uint64_t *)b->stats.ptr;
    a.flags = (uint32_t *)((char *)b->stats.ptr + flags_off);
    a.out = d_out;
    a.vocab = (uint32_t)vocab;
    a.top_k = top_k;
    a.parts = (uint32_t)parts;
    a.inv_temperature = invt;
    a.top_p = top_p;
    a.draw = draw;
    if ((st = launch(b->topk_part, dim3((unsigned)parts), dim3(1024), s, a, "ctox_topk_part_gfx950"))) return st;
    return launch(b->topk_final, dim3(1), dim3(1024), s, a, "ctox_topk_final_gfx950");
}

extern "C" ctox_status ctox_hip_check_finite_device(ctox_hip_backend *b, const float *d_x, size_t n,
                                                    uint32_t *d_flags, size_t parts, void *stream) {
    if (!b || !d_x || !d_flags) return fail(CTOX_ERR_SHAPE, "null argument");
    if ((uintptr_t)d_x % 16) return fail(CTOX_ERR_SHAPE, "finite check needs a 16-byte aligned buffer");
    if (parts == 0 || parts > 1024) return fail(CTOX_ERR_SHAPE, "finite check parts outside 1..1024");
    FiniteArgs a{d_x, d_flags, (uint64_t)n};
    return launch(b->finite, dim3((unsigned)parts), dim3(256), pick_stream(b, stream), a, "ctox_finite_check_gfx950");
}

extern "C" ctox_status ctox_hip_gather_rows_device(ctox_hip_backend *b, const void *d_src, size_t src_rows,
                                                   size_t row_bytes, const uint32_t *ids, size_t rows, void *d_dst,
                                                   void *stream) {
    if (!b || !d_src || !ids || !d_dst) return fail(CTOX_ERR_SHAPE, "null argument");
    if (rows == 0 || rows > 0x7fffffffu || row_bytes == 0) return fail(CTOX_ERR_SHAPE, "gather rows geometry");
    // ids are host values: checked here, then carried to the device.
    for (size_t r = 0; r < rows; r++)
        if (ids[r] >= src_rows) return fail(CTOX_ERR_SHAPE, "gathered row %u outside %zu rows", ids[r], src_rows);
    uint32_t *d_ids = nullptr;
    HIP_TRY(hipMalloc((void **)&d_ids, rows * sizeof(uint32_t)));
    hipStream_t s = pick_stream(b, stream);
    hipError_t e = hipMemcpyAsync(d_ids, ids, rows * sizeof(uint32_t), hipMemcpyHostToDevice, s);
    ctox_status st = CTOX_OK;
    if (e != hipSuccess) st = fail(CTOX_ERR_INVALID_STATE, "gather ids upload failed: %s", hipGetErrorString(e));
    GatherRowsArgs a{(const uint8_t *)d_src, (uint8_t *)d_dst, d_ids, (uint64_t)row_bytes, (uint32_t)rows, 0};
    if (!st) st = launch(b->gather, dim3((unsigned)rows), dim3(256), s, a, "ctox_gather_rows_gfx950");
    (void)hipStreamSynchronize(s);
    (void)hipFree(d_ids);
    return st;
}

// A plain streaming read of `bytes` (a multiple of 16) with the tiled
// matvec's access pattern; d_out receives one word per 8 KiB.
extern "C" ctox_status ctox_hip_stream_read_device(ctox_hip_backend *b, const void *d_src, size_t bytes,
                                                   uint32_t *d_out, void *stream) {
    if (!b || !d_src || !d_out) return fail(CTOX_ERR_SHAPE, "null argument");
    if (bytes == 0 || bytes % 16 || bytes > ((size_t)1 << 40)) return fail(CTOX_ERR_SHAPE, "read size");
    const size_t waves = (bytes + 8191) / 8192;
    StreamReadArgs a{(const uint8_t *)d_src, d_out, (uint64_t)bytes};
    return launch(b->stream_read, dim3((unsigned)((waves + 3) / 4)), dim3(256), pick_stream(b, stream), a,
                  "ctox_stream_read_gfx950");
}

// ======================================================================
// layer glue
// ======================================================================
namespace {
ctox_status norm_launch(ctox_hip_backend *b, const float *x, const float *gate, size_t rows, size_t cols,
                        const float *w, float eps, float *out, uint32_t mode, void *stream) {
    if (!b || !x || !w || !out || (mode == 1 && !gate)) return fail(CTOX_ERR_SHAPE, "null argument");
    // Q/src/reference.rs:18-34 matrix contract and the eps check of :38-93.
    if (rows == 0 || cols == 0 || rows > 0x7fffffffu || cols > 0xffffffffu)
        return fail(CTOX_ERR_SHAPE, "norm matrix shape is empty or too large");
    if (!std::isfinite(eps) || eps <= 0.0f) return fail(CTOX_ERR_SHAPE, "norm epsilon must be finite and positive");
    NormArgs a{x, gate, w, out, (uint32_t)cols, mode, eps, 0};
    return launch(b->rms, dim3((unsigned)rows), dim3(256), pick_stream(b, stream), a, "ctox_rms_norm_gfx950");
}
ctox_status elt_launch(ctox_hip_backend *b, hipFunction_t f, const float *x, const float *y, float *out, size_t n,
                       void *stream, const char *name) {
    if (!b || !x || !y || !out) return fail(CTOX_ERR_SHAPE, "null argument");
    if (n == 0 || (n + 255) / 256 > 0x7fffffffu) return fail(CTOX_ERR_SHAPE, "%s length is empty or too large", name);
    EltArgs a{x, y, out, (uint64_t)n};
    return launch(f, dim3((unsigned)((n + 255) / 256)), dim3(256), pick_stream(b, stream), a, name);
}
}  // namespace

extern "C" ctox_status ctox_hip_rms_norm_device(ctox_hip_backend *b, const float *d_x, size_t rows, size_t cols,
                                                const float *d_w, float eps, float *d_out, void *stream) {
    return norm_launch(b, d_x, nullptr, rows, cols, d_w, eps, d_out, 0, stream);
}

extern "C" ctox_status ctox_hip_rms_norm_gated_device(ctox_hip_backend *b, const float *d_x, const float *d_gate,
                                                      size_t rows, size_t cols, const float *d_w, float eps,
                                                      float *d_out, void *stream) {
    return norm_launch(b, d_x, d_gate, rows, cols, d_w, eps, d_out, 1, stream);
}

extern "C" ctox_status ctox_hip_swiglu_device(ctox_hip_backend *b, const float *d_gate, const float *d_up, size_t n,
                                              float *d_out, void *stream) {
    return elt_launch(b, b ? b->swiglu : nullptr, d_gate, d_up, d_out, n, stream, "ctox_swiglu_gfx950");
}

extern "C" ctox_status ctox_hip_sigmoid_gate_device(ctox_hip_backend *b, float *d_values, const float *d_gate,
                                                    size_t n, void *stream) {
    return elt_launch(b, b ? b->sgate : nullptr, d_values, d_gate, d_values, n, stream, "ctox_sigmoid_gate_gfx950");
}

extern "C" ctox_status ctox_hip_causal_conv_update_device(ctox_hip_backend *b, const float *d_input, float *d_state,
                                                          const float *d_weight, size_t channels, size_t kernel,
                                                          float *d_out, void *stream) {
    if (!b || !d_input || !d_state || !d_weight || !d_out) return fail(CTOX_ERR_SHAPE, "null argument");
    if (channels == 0 || kernel == 0 || channels > 0x7fffffffu || kernel > 4096)
        return fail(CTOX_ERR_SHAPE, "conv state shape is empty or too large");
    ConvArgs a{d_input, d_state, d_weight, d_out, (uint32_t)channels, (uint32_t)kernel, 1, (uint32_t)channels};
    return launch(b->conv, dim3((unsigned)((channels + 255) / 256)), dim3(256), pick_stream(b, stream), a,
                  "ctox_conv_update_gfx950");
}

extern "C" ctox_status ctox_hip_partial_rope_device(ctox_hip_backend *b, float *d_q, float *d_k, size_t rows,
                                                    size_t q_heads, size_t k_heads, size_t head_dim,
                                                    size_t rotary_dim, uint64_t position, float theta, void *stream) {
    if (!b || !d_q || !d_k) return fail(CTOX_ERR_SHAPE, "null argument");
    // Q/src/reference.rs:115-155: the rotary dimension is even, non-zero and within the head.
    if (rotary_dim == 0 || rotary_dim > head_dim || rotary_dim % 2 || !std::isfinite(theta) || theta <= 0.0f)
        return fail(CTOX_ERR_SHAPE, "rotary dimension or theta is invalid");
    if (rows == 0 || q_heads == 0 || k_heads == 0 || rotary_dim > 512 || rows > 65535 || q_heads + k_heads > 65535 ||
        position > UINT64_MAX - rows)
        return fail(CTOX_ERR_SHAPE, "rope shape is empty or too large");
    RopeArgs a{d_q, d_k, (uint32_t)q_heads, (uint32_t)k_heads, (uint32_t)head_dim, (uint32_t)rotary_dim,
               (uint64_t)position, theta, 0};
    return launch(b->rope, dim3((unsigned)rows, (unsigned)(q_heads + k_heads)), dim3(256), pick_stream(b, stream), a,
                  "ctox_rope_gfx950");
}

// ======================================================================
// paged KV cache and attention
// ======================================================================
extern "C" ctox_status ctox_hip_kv_pack_q4_device(ctox_hip_backend *b, uint8_t *d_q4_pages, const float *d_keys,
                                                  const float *d_values, size_t token_count, size_t component_values,
                                                  uint32_t physical_slot, uint32_t first_token_in_page,
                                                  uint32_t q4_page_bytes, void *stream) {
    if (!b || !d_q4_pages || !d_keys || !d_values) return fail(CTOX_ERR_SHAPE, "null argument");
    // Q/src/kv_cache.rs:238-252: a non-zero multiple of 64 values per component.
    if (component_values == 0 || component_values % 64 || component_values > (1u << 24))
        return fail(CTOX_ERR_SHAPE, "KV component width must be a non-zero multiple of 64");
    const uint64_t token_bytes = component_values * 2 / 64 * 34;
    if (token_count == 0 || token_count > 65535 ||
        (first_token_in_page + token_count) * token_bytes > (uint64_t)q4_page_bytes)
        return fail(CTOX_ERR_SHAPE, "KV tokens do not fit the Q4 page");
    KvPackArgs a{d_q4_pages, d_keys, d_values, physical_slot, first_token_in_page, (uint32_t)component_values,
                 (uint32_t)token_bytes, q4_page_bytes};
    return launch(b->kv_pack, dim3((unsigned)(component_values * 2 / 64), (unsigned)token_count), dim3(64),
                  pick_stream(b, stream), a, "ctox_kv_pack_q4_gfx950");
}

extern "C" ctox_status ctox_hip_attn_prep_device(ctox_hip_backend *b, const float *d_proj, size_t proj_stride,
                                                const float *d_q_norm, const float *d_k_norm, size_t rows,
                                                size_t q_heads, size_t kv_heads, size_t head_dim, size_t rotary_dim,
                                                uint64_t position, float theta, float eps, uint8_t *d_q4_pages,
                                                uint32_t q4_page_bytes, const uint32_t *slots,
                                                const uint32_t *positions_in_page, float *d_q_out,
                                                uint32_t *d_words_dst, const uint32_t *words, size_t word_count,
                                                void *stream) {
    if (!b || !d_proj || !d_q_norm || !d_k_norm || !d_q4_pages || !slots || !positions_in_page || !d_q_out ||
        (word_count && (!d_words_dst || !words)))
        return fail(CTOX_ERR_SHAPE, "null argument");
    if (word_count > CTOX_ATTN_PREP_DESC_WORDS) return fail(CTOX_ERR_SHAPE, "attention prep carries at most 32 words");
    if (head_dim != 256 || rows == 0 || rows > CTOX_ATTN_PREP_ROWS || q_heads == 0 || kv_heads == 0 ||
        q_heads + 2 * kv_heads > 65535 || rotary_dim == 0 || rotary_dim % 2 || rotary_dim > head_dim ||
        proj_stride < 2 * (q_heads + kv_heads) * head_dim || proj_stride > 0xffffffffu || !std::isfinite(theta) ||
        !(theta > 0.0f) || !std::isfinite(eps) || !(eps > 0.0f))
        return fail(CTOX_ERR_SHAPE, "attention prep shapes");
    const uint64_t token_bytes = 2 * kv_heads * head_dim / 64 * 34;
    AttnPrepArgs a{};
    for (size_t t = 0; t < rows; t++) {
        if ((uint64_t)(positions_in_page[t] + 1) * token_bytes > q4_page_bytes)
            return fail(CTOX_ERR_SHAPE, "attention prep row does not fit its Q4 page");
        a.slot[t] = slots[t];
        a.pos[t] = positions_in_page[t];
    }
    a.proj = d_proj;
    a.q_norm = d_q_norm;
    a.k_norm = d_k_norm;
    a.q_out = d_q_out;
    a.q4_pages = d_q4_pages;
    a.q4_page_bytes = q4_page_bytes;
    a.position = position;
    a.proj_stride = (uint32_t)proj_stride;
    a.qh = (uint32_t)q_heads;
    a.kh = (uint32_t)kv_heads;
    a.hd = (uint32_t)head_dim;
    a.rd = (uint32_t)rotary_dim;
    a.q4_token_bytes = (uint32_t)token_bytes;
    a.eps = eps;
    a.theta = theta;
    a.desc_dst = word_count ? d_words_dst : nullptr;
    a.desc_words = (uint32_t)word_count;
    for (size_t i = 0; i < word_count; i++) a.desc[i] = words[i];
    return launch(b->attn_prep, dim3((unsigned)(q_heads + 2 * kv_heads), (unsigned)rows), dim3(64),
                  pick_stream(b, stream), a, "ctox_attn_prep_gfx950");
}

extern "C" ctox_status ctox_hip_kv_demote_device(ctox_hip_backend *b, const uint8_t *d_q4_page, uint8_t *d_q2_page,
                                                 size_t tokens, size_t blocks_per_token, void *stream) {
    if (!b || !d_q4_page || !d_q2_page) return fail(CTOX_ERR_SHAPE, "null argument");
    if (tokens == 0 || blocks_per_token == 0 || tokens > (1u << 20) || blocks_per_token > (1u << 20))
        return fail(CTOX_ERR_SHAPE, "KV page geometry is empty or too large");
    const uint64_t blocks = (uint64_t)tokens * blocks_per_token;
    KvDemoteArgs a{d_q4_page, d_q2_page, blocks};
    return launch(b->kv_demote, dim3((unsigned)((blocks * 16 + 255) / 256)), dim3(256), pick_stream(b, stream), a,
                  "ctox_kv_demote_gfx950");
}

namespace {
// The attention-gate staging of the o projection's input done by the combine.
struct GateStage {
    const float *gate = nullptr;
    uint32_t gate_stride = 0;
    const uint16_t *s_in = nullptr;
    int32_t dtype = 0;
};

ctox_status paged_gqa_impl(ctox_hip_backend *b, const float *d_query, const uint8_t *d_q2_pages,
                           const uint8_t *d_q4_pages, const ctox_paged_kv_descriptor *d_descriptors,
                           const ctox_paged_gqa_params *p, size_t rows, float *d_out, void *stream,
                           const GateStage *gs) {
    if (!b || !d_query || !d_q2_pages || !d_q4_pages || !d_descriptors || !p || !d_out)
        return fail(CTOX_ERR_SHAPE, "null argument");
    if (p->head_dim != 256) return fail(CTOX_ERR_UNSUPPORTED_OPERATION, "paged attention needs head_dim 256");
    // Q/src/reference.rs:420-440 contract: heads divide, the query rows are cached.
    if (p->key_value_heads == 0 || p->query_heads == 0 || p->query_heads % p->key_value_heads || rows == 0 ||
        rows > p->tokens || p->page_tokens == 0 || p->page_count == 0 || !std::isfinite(p->scale))
        return fail(CTOX_ERR_SHAPE, "invalid paged attention contract");
    const uint32_t group = p->query_heads / p->key_value_heads;
    if ((uint64_t)group * rows > 32)
        return fail(CTOX_ERR_UNSUPPORTED_OPERATION, "query heads per kv head times rows exceeds 32");
    const uint64_t cv = (uint64_t)p->key_value_heads * 256;
    if (p->combined_values != 2 * cv || p->q2_token_bytes != 2 * cv / 64 * 18 ||
        p->q4_token_bytes != 2 * cv / 64 * 34 || (uint64_t)p->q2_page_bytes < (uint64_t)p->page_tokens * p->q2_token_bytes ||
        (uint64_t)p->q4_page_bytes < (uint64_t)p->page_tokens * p->q4_token_bytes || p->q2_page_bytes % 4 ||
        p->q4_page_bytes % 4 || p->tokens > (1u << 30))
        return fail(CTOX_ERR_SHAPE, "paged KV geometry differs from the attention contract");
    const uint32_t queries = group * (uint32_t)rows;
    const uint32_t tiles = (p->tokens + 15) / 16;
    // Two workgroups per CU for the 16-query kernel (it fits two per CU), one for the 32-query one.
    const uint32_t per_cu = queries > 16 ? 1 : 2;
    uint32_t splits = std::max<uint32_t>(1, (uint32_t)((per_cu * b->cus + p->key_value_heads - 1) / p->key_value_heads));
    splits = std::min<uint32_t>(std::min<uint32_t>(splits, (tiles + 3) / 4), 1024);
    const uint32_t tpw = (tiles + 4 * splits - 1) / (4 * splits);
    splits = (tiles + 4 * tpw - 1) / (4 * tpw);
    const size_t part = (size_t)p->key_value_heads * splits * queries;
    ctox_status st = ensure(b, b->attn, part * (256 + 2) * sizeof(float), false);
    if (st) return st;
    float *part_out = (float *)b->attn.ptr;
    GqaArgs a{d_query, d_q2_pages, d_q4_pages, (const PagedKvDesc *)d_descriptors, part_out, part_out + part * 256,
              d_out, p->q2_page_bytes, p->q4_page_bytes, p->query_heads, group, p->tokens, (uint32_t)rows, queries,
              p->page_tokens, p->page_count, (uint32_t)cv, p->q2_token_bytes, p->q4_token_bytes, tiles, tpw, splits,
              p->scale, p->page_tokens % 16 == 0 ? 1u : 0u, 0};
    if (gs) {
        const int layout = gs->dtype == CTOX_DTYPE_Q4B64 ? 1 : 0;
        const size_t blocks = (size_t)p->query_heads * 256 / kBlockLen;
        st = ensure(b, b->xa[layout], blocks * rows * 192, false);
        if (!st) st = ensure(b, b->xc[layout], blocks * rows * 4 * sizeof(float), false);
        if (st) return st;
        a.st_xa = (int8_t *)b->xa[layout].ptr;
        a.st_xc = (float *)b->xc[layout].ptr;
        a.st_gate = gs->gate;
        a.st_gate_stride = gs->gate_stride;
        a.st_s_in = gs->s_in;
        a.st_dtype = (uint32_t)layout;
    }
    hipStream_t s = pick_stream(b, stream);
    // Page-aligned 16-token tiles run P.V on f16 MFMA; other page sizes on the fp32-MFMA kernel.
    // (its waves hold up to 64 tiles' page descriptors in registers).
    const bool f16 = p->page_tokens % 16 == 0 && tpw <= 64;
    hipFunction_t part_fn = f16 ? b->gqa_part16[queries > 16 ? 1 : 0] : b->gqa_part[queries > 16 ? 1 : 0];
    st = launch(part_fn, dim3(splits, p->key_value_heads), dim3(256), s, a,
                "ctox_paged_gqa_partial_gfx950");
    if (st) return st;
    return launch(b->gqa_combine, dim3(queries, p->key_value_heads, 4), dim3(256), s, a, "ctox_paged_gqa_combine_gfx950");
}
}  // namespace

extern "C" ctox_status ctox_hip_paged_gqa_device(ctox_hip_backend *b, const float *d_query, const uint8_t *d_q2_pages,
                                                 const uint8_t *d_q4_pages,
                                                 const ctox_paged_kv_descriptor *d_descriptors,
                                                 const ctox_paged_gqa_params *p, size_t rows, float *d_out,
                                                 void *stream) {
    return paged_gqa_impl(b, d_query, d_q2_pages, d_q4_pages, d_descriptors, p, rows, d_out, stream, nullptr);
}

ctox_status ctox_paged_gqa_stage_o_device(ctox_hip_backend *b, const float *d_query, const uint8_t *d_q2_pages,
                                          const uint8_t *d_q4_pages, const ctox_paged_kv_descriptor *d_descriptors,
                                          const ctox_paged_gqa_params *p, size_t rows, float *d_out,
                                          const float *d_gate, uint32_t gate_stride, const uint16_t *d_o_s_in,
                                          int32_t o_dtype, void *stream) {
    if (!d_gate || gate_stride < 2 * 256 * (size_t)(p ? p->query_heads : 0))
        return fail(CTOX_ERR_SHAPE, "attention gate staging geometry");
    GateStage gs;
    gs.gate = d_gate;
    gs.gate_stride = gate_stride;
    gs.s_in = d_o_s_in;
    gs.dtype = o_dtype;
    return paged_gqa_impl(b, d_query, d_q2_pages, d_q4_pages, d_descriptors, p, rows, d_out, stream, &gs);
}

bool ctox_small_m_staged(ctox_hip_backend *b, const void *d_weights, uint32_t batch, uint32_t rows, uint32_t columns) {
    return b && batch >= 2 && batch <= 8 && !build_in_kernel(b, batch, rows, columns) &&
           registered(b, d_weights, rows, columns) != nullptr;
}
static_assert(sizeof(ctox_paged_kv_descriptor) == sizeof(PagedKvDesc), "page descriptor layout");

extern "C" ctox_status ctox_hip_causal_conv_rows_device(ctox_hip_backend *b, const float *d_input, size_t in_stride,
                                                        float *d_state, const float *d_weight, size_t channels,
                                                        size_t kernel, size_t rows, float *d_out, void *stream) {
    if (!b || !d_input || !d_state || !d_weight || !d_out) return fail(CTOX_ERR_SHAPE, "null argument");
    if (channels == 0 || kernel == 0 || channels > 0x7fffffffu || kernel > 4096 || rows == 0 || rows > 65536 ||
        in_stride < channels || in_stride > 0x7fffffffu)
        return fail(CTOX_ERR_SHAPE, "conv state shape is empty or too large");
    ConvArgs a{d_input, d_state, d_weight, d_out, (uint32_t)channels, (uint32_t)kernel, (uint32_t)rows,
               (uint32_t)in_stride};
    return launch(b->conv, dim3((unsigned)((channels + 255) / 256)), dim3(256), pick_stream(b, stream), a,
                  "ctox_conv_update_gfx950");
}

// ======================================================================
// decode engine helpers
// ======================================================================
extern "C" ctox_status ctox_hip_fill_random_device(ctox_hip_backend *b, void *d_ptr, uint64_t count, uint32_t kind,
                                                   uint64_t seed, float p0, float p1, void *stream) {
    if (!b || !d_ptr) return fail(CTOX_ERR_SHAPE, "null argument");
    if (kind > 4 || !std::isfinite(p0) || !std::isfinite(p1)) return fail(CTOX_ERR_SHAPE, "invalid fill request");
    const size_t unit = kind == 0 ? 34 : kind == 1 ? 18 : kind == 3 ? 2 : 4;
    hipStream_t s = pick_stream(b, stream);
    const uint64_t chunk = (uint64_t)1 << 26;
    for (uint64_t base = 0; base < count; base += chunk) {
        const uint64_t n = std::min<uint64_t>(chunk, count - base);
        FillArgs a{(char *)d_ptr + base * unit, n, base, seed, kind, p0, p1, 0};
        ctox_status st = launch(b->fill, dim3((unsigned)((n + 255) / 256)), dim3(256), s, a, "ctox_fill_random_gfx950");
        if (st) return st;
    }
    return CTOX_OK;
}

extern "C" ctox_status ctox_hip_embedding_rows_device(ctox_hip_backend *b, int32_t dtype, const uint8_t *d_weights,
                                                      const uint16_t *d_s_in, const uint16_t *d_s_out,
                                                      const uint32_t *d_tokens, size_t rows, size_t vocab,
                                                      size_t cols, float *d_out, void *stream) {
    if (!b || !d_weights || !d_tokens || !d_out) return fail(CTOX_ERR_SHAPE, "null argument");
    if (dtype != CTOX_DTYPE_Q2B64 && dtype != CTOX_DTYPE_Q4B64) return fail(CTOX_ERR_UNSUPPORTED_DTYPE, "embedding rows must be Q2 or Q4");
    if (rows == 0 || rows > 65535 || cols == 0 || cols % 64 || cols > 0x7fffffffu || vocab == 0 || vocab > 0xffffffffu)
        return fail(CTOX_ERR_SHAPE, "embedding shape is empty or too large");
    EmbedArgs a{d_weights, d_s_in, d_s_out, d_tokens, d_out, (uint32_t)cols, (uint32_t)vocab,
                dtype == CTOX_DTYPE_Q4B64 ? 1u : 0u, 0};
    return launch(b->embed, dim3((unsigned)((cols + 255) / 256), (unsigned)rows), dim3(256), pick_stream(b, stream), a,
                  "ctox_embed_rows_gfx950");
}

extern "C" ctox_status ctox_hip_norm_rows_device(ctox_hip_backend *b, const ctox_norm_rows *d, void *stream) {
    if (!b || !d || !d->x || !d->w || !d->out || (d->mode == 1 && !d->gate)) return fail(CTOX_ERR_SHAPE, "null argument");
    if (d->rows == 0 || d->cols == 0 || d->inner == 0 || d->mode > 1)
        return fail(CTOX_ERR_SHAPE, "norm rows shape is empty or mode unknown");
    if (!std::isfinite(d->eps) || d->eps <= 0.0f) return fail(CTOX_ERR_SHAPE, "norm epsilon must be finite and positive");
    // Up to 8 columns per thread, 64..1024 threads.
    if (d->cols > 8 * 1024) return fail(CTOX_ERR_SHAPE, "norm rows wider than 8192");
    const uint32_t threads = std::min<uint32_t>(1024, 64 * ((d->cols + 511) / 512));
    if (d->delta && (d->delta_parts > 64 || (d->delta_parts > 1 && (d->delta_stride < (uint64_t)d->rows * d->cols ||
                                                                      d->delta_stride > 0xffffffffu))))
        return fail(CTOX_ERR_SHAPE, "norm rows delta parts geometry");
    NormRowsArgs a{d->x, d->delta, d->gate, d->w, d->out, d->cols, d->mode, d->eps, d->inner,
                   d->x_inner, d->x_outer, d->g_inner, d->g_outer, d->out_stride,
                   std::max<uint32_t>(1, d->delta_parts), (uint32_t)d->delta_stride};
    return launch(b->norm_rows, dim3(d->rows), dim3(threads), pick_stream(b, stream), a, "ctox_norm_rows_gfx950");
}

extern "C" ctox_status ctox_hip_attention_gate_device(ctox_hip_backend *b, float *d_values, const float *d_qg,
                                                      size_t rows, size_t heads, size_t head_dim, size_t qg_stride,
                                                      void *stream) {
    if (!b || !d_values || !d_qg) return fail(CTOX_ERR_SHAPE, "null argument");
    const uint64_t n = (uint64_t)rows * heads * head_dim;
    if (n == 0 || (n + 255) / 256 > 0x7fffffffu || qg_stride < 2 * heads * head_dim || qg_stride > 0xffffffffu)
        return fail(CTOX_ERR_SHAPE, "attention gate shape");
    AttnGateArgs a{d_values, d_qg, (uint32_t)rows, (uint32_t)heads, (uint32_t)head_dim, (uint32_t)qg_stride};
    return launch(b->attn_gate, dim3((unsigned)((n + 255) / 256)), dim3(256), pick_stream(b, stream), a,
                  "ctox_attn_gate_gfx950");
}

namespace {
ctox_status rows_launch(ctox_hip_backend *b, hipFunction_t f, const float *in, size_t in_stride, size_t offset,
                        size_t rows, size_t cols, float *out, size_t out_stride, void *stream, const char *name) {
    if (!b || !in || !out) return fail(CTOX_ERR_SHAPE, "null argument");
    const uint64_t n = (uint64_t)rows * cols;
    if (n == 0 || (n + 255) / 256 > 0x7fffffffu || in_stride > 0xffffffffu || out_stride > 0xffffffffu ||
        offset > 0xffffffffu || out_stride < cols)
        return fail(CTOX_ERR_SHAPE, "%s shape", name);
    RowsArgs a{in, out, (uint32_t)rows, (uint32_t)cols, (uint32_t)in_stride, (uint32_t)out_stride, (uint32_t)offset, 0};
    return launch(f, dim3((unsigned)((n + 255) / 256)), dim3(256), pick_stream(b, stream), a, name);
}
}  // namespace

extern "C" ctox_status ctox_hip_swiglu_rows_device(ctox_hip_backend *b, const float *d_in, size_t in_stride,
                                                   size_t up_offset, size_t rows, size_t cols, float *d_out,
                                                   size_t out_stride, void *stream) {
    if (up_offset < cols || in_stride < up_offset + cols) return fail(CTOX_ERR_SHAPE, "swiglu rows geometry");
    return rows_launch(b, b ? b->swiglu_rows : nullptr, d_in, in_stride, up_offset, rows, cols, d_out, out_stride,
                       stream, "ctox_swiglu_rows_gfx950");
}

extern "C" ctox_status ctox_hip_copy_rows_device(ctox_hip_backend *b, const float *d_in, size_t in_stride,
                                                 size_t col_offset, size_t rows, size_t cols, float *d_out,
                                                 size_t out_stride, void *stream) {
    if (in_stride < col_offset + cols) return fail(CTOX_ERR_SHAPE, "copy rows geometry");
    return rows_launch(b, b ? b->copy_rows : nullptr, d_in, in_stride, col_offset, rows, cols, d_out, out_stride,
                       stream, "ctox_copy_rows_gfx950");
}

ctox_status ctox_write_word_ranges_device(ctox_hip_backend *b, uint32_t *const *dst, const uint32_t *const *src,
                                          const size_t *count, size_t n, void *stream) {
    if (!b || (n && (!dst || !src || !count))) return fail(CTOX_ERR_SHAPE, "null argument");
    hipStream_t s = pick_stream(b, stream);
    SegWordsArgs a{};
    auto flush = [&]() -> ctox_status {
        if (a.nseg == 0) return CTOX_OK;
        const ctox_status st = launch(b->write_segments, dim3(1), dim3(512), s, a, "ctox_write_segments_gfx950");
        a = SegWordsArgs{};
        return st;
    };
    for (size_t i = 0; i < n; i++) {
        for (size_t done = 0; done < count[i];) {
            if (a.nseg == CTOX_SEG_MAX || a.off[a.nseg] == CTOX_SEG_WORDS)
                if (ctox_status st = flush()) return st;
            const size_t take = std::min<size_t>(count[i] - done, CTOX_SEG_WORDS - a.off[a.nseg]);
            a.dst[a.nseg] = dst[i] + done;
            std::memcpy(a.words + a.off[a.nseg], src[i] + done, take * sizeof(uint32_t));
            a.off[a.nseg + 1] = a.off[a.nseg] + (uint32_t)take;
            a.nseg++;
            done += take;
        }
    }
    return flush();
}

extern "C" ctox_status ctox_hip_write_words_device(ctox_hip_backend *b, uint32_t *d_dst, const uint32_t *words,
                                                   size_t count, void *stream) {
    if (!b || !d_dst || (!words && count)) return fail(CTOX_ERR_SHAPE, "null argument");
    hipStream_t s = pick_stream(b, stream);
    for (size_t i = 0; i < count; i += 32) {
        WordsArgs a{};
        a.dst = d_dst + i;
        a.count = (uint32_t)std::min<size_t>(32, count - i);
        std::memcpy(a.words, words + i, a.count * sizeof(uint32_t));
        ctox_status st = launch(b->write_words, dim3(1), dim3(64), s, a, "ctox_write_words_gfx950");
        if (st) return st;
    }
    return CTOX_OK;
}
