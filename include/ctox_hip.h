/*
 * ctox_hip.h -- C ABI of the MI355X (gfx950) HIP backend for CTOX-LLM's
 * Qwen3.8-27B decode hot path.
 *
 * This is the drop-in boundary. A host written against the crate's
 * `Backend` trait (Q/src/backend/mod.rs:153-169; Q/ = models/qwen38_27b/ in
 * the reference tree) binds these symbols over FFI exactly as the CUDA
 * candidate runtime binds its kernels through the driver API
 * (Q/src/backend/cuda_runtime.rs:195-294). All signatures use plain
 * pointers and sizes; no PyTorch or HIP C++ types cross the boundary.
 * Streams are passed as `void*` holding a `hipStream_t`; NULL is HIP's
 * null stream. Host-buffer entry points use a stream the backend owns.
 *
 * Threading: one backend handle owns one device context and is externally
 * synchronized (the reference CUDA runtime is `Rc`, not `Send`:
 * Q/src/backend/cuda_executor.rs:149-155). Calls on one handle must not
 * overlap.
 *
 * Error contract: every entry point returns a ctox_status mapped 1:1 from
 * EngineError (Q/src/error.rs:5-29). Nothing falls back to a CPU path
 * (Q/src/backend/cpu.rs:400-410); non-finite outputs of the host-buffer
 * entry points are reported as CTOX_ERR_INVALID_STATE
 * (Q/src/backend/cuda_runtime.rs:10627-10632). The message of the last
 * failure on the calling thread is returned by ctox_hip_last_error().
 */
#ifndef CTOX_HIP_H
#define CTOX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* EngineError variants, Q/src/error.rs:5-29. */
typedef enum {
    CTOX_OK = 0,
    CTOX_ERR_IO = 1,
    CTOX_ERR_JSON = 2,
    CTOX_ERR_INVALID_ARTIFACT = 3,
    CTOX_ERR_UNSUPPORTED_DTYPE = 4,
    CTOX_ERR_UNSUPPORTED_OPERATION = 5,
    CTOX_ERR_MEMORY_BUDGET = 6,
    CTOX_ERR_SHAPE = 7,
    CTOX_ERR_INVALID_STATE = 8,
    CTOX_ERR_CANCELLED = 9
} ctox_status;

/* TensorDType, Q/src/format.rs:26-33. */
typedef enum {
    CTOX_DTYPE_Q2B64 = 0,
    CTOX_DTYPE_Q4B64 = 1,
    CTOX_DTYPE_MIXED_Q2Q4B64 = 2,
    CTOX_DTYPE_F16 = 3,
    CTOX_DTYPE_F32 = 4
} ctox_dtype;

/* Activation, Q/src/backend/mod.rs:54-67. */
typedef enum { CTOX_ACT_IDENTITY = 0, CTOX_ACT_SILU = 1 } ctox_activation;

/* Option<ScaleSlice>, Q/src/backend/mod.rs:74-112. */
typedef enum { CTOX_SCALE_NONE = 0, CTOX_SCALE_F32 = 1, CTOX_SCALE_F16LE = 2 } ctox_scale_kind;

typedef struct {
    int32_t kind;      /* ctox_scale_kind */
    const void *data;  /* float* (F32) or little-endian binary16 bytes (F16Le) */
    size_t len;        /* number of values, not bytes */
} ctox_scale_slice;

/* QuantSegment, Q/src/format.rs:56-64. */
typedef struct {
    uint32_t group_index;
    uint64_t row_start;
    uint64_t row_end;
    int32_t dtype;     /* CTOX_DTYPE_Q2B64 or CTOX_DTYPE_Q4B64 */
    uint64_t offset;   /* relative to the tensor's packed payload */
    uint64_t length;
} ctox_quant_segment;

/* FusedMatVec, Q/src/backend/mod.rs:115-128. Host pointers. */
typedef struct {
    int32_t dtype;
    const uint8_t *weights;
    size_t weights_len;
    const ctox_quant_segment *segments;
    size_t n_segments;
    size_t rows;
    size_t columns;
    const float *input;
    size_t input_len;
    ctox_scale_slice s_in;
    ctox_scale_slice s_out;
    const float *bias;   /* NULL = None */
    size_t bias_len;
    int32_t activation;  /* ctox_activation */
} ctox_fused_matvec;

/* RecoveredRow, Q/src/backend/mod.rs:130-142. */
typedef struct {
    int32_t dtype;
    const uint8_t *weights;
    size_t weights_len;
    size_t columns;
    ctox_scale_slice s_in;
    float s_out;
} ctox_recovered_row;

/* RecoveredRowMatVec, Q/src/backend/mod.rs:144-151. */
typedef struct {
    int32_t dtype;
    const uint8_t *weights;
    size_t weights_len;
    const float *corrected_input;
    size_t len;
    float s_out;
} ctox_recovered_row_matvec;

typedef struct ctox_hip_backend ctox_hip_backend;
typedef struct ctox_hip_matrix ctox_hip_matrix;

/* ---- lifecycle (replaces CudaCandidateRuntime::new, cuda_runtime.rs:1297-1371) ---- */
ctox_status ctox_hip_backend_create(int device, ctox_hip_backend **out);
void ctox_hip_backend_destroy(ctox_hip_backend *backend);
/* Backend::kind / promotion_state / profile (Q/src/backend/mod.rs:153-157).
 * kind returns "hip"; promotion state is "experimental"; profile names the
 * device architecture (e.g. "gfx950-mfma"). Strings are static. */
const char *ctox_hip_backend_kind(const ctox_hip_backend *backend);
const char *ctox_hip_backend_promotion_state(const ctox_hip_backend *backend);
const char *ctox_hip_backend_profile(const ctox_hip_backend *backend);
/* Thread-local message of the last failing call ("" if none). */
const char *ctox_hip_last_error(void);
/* Blocks until all work the backend issued on its own stream is done. */
ctox_status ctox_hip_synchronize(ctox_hip_backend *backend);

/* ---- Backend trait, host buffers (Q/src/backend/mod.rs:158-168) ---- */
/* Backend::fused_matvec; `output` holds op->rows floats. */
ctox_status ctox_hip_fused_matvec(ctox_hip_backend *backend, const ctox_fused_matvec *op,
                                  float *output, size_t output_len);
/* Backend::fused_matvec_fanout; outputs[i] holds ops[i].rows floats. Results
 * equal independent fused_matvec calls (Q/src/backend/cpu.rs:444-472). */
ctox_status ctox_hip_fused_matvec_fanout(ctox_hip_backend *backend, const ctox_fused_matvec *ops,
                                         size_t n_ops, float *const *outputs);
/* Backend::recovered_row (Q/src/backend/cpu.rs:312-370); output holds columns floats. */
ctox_status ctox_hip_recovered_row(ctox_hip_backend *backend, const ctox_recovered_row *op,
                                   float *output, size_t output_len);
/* Backend::recovered_row_matvec (Q/src/backend/cpu.rs:478-497). */
ctox_status ctox_hip_recovered_row_matvec(ctox_hip_backend *backend,
                                          const ctox_recovered_row_matvec *op, float *result);

/* ---- resident matrices: prepare once, dispatch many times ----
 * Replaces CudaCandidateRuntime::prepare_* / dispatch_prepared_*
 * (Q/src/backend/cuda_runtime.rs:8341-8386, 10560-10637). The descriptor's
 * weights, segments, s_in, s_out and bias are validated exactly as the CPU
 * dispatcher does (Q/src/backend/cpu.rs:41-173) and uploaded to HBM in the
 * crate's packed CTOXQ layout, unchanged. op->input is ignored. */
ctox_status ctox_hip_matrix_prepare(ctox_hip_backend *backend, const ctox_fused_matvec *op,
                                    ctox_hip_matrix **out);
void ctox_hip_matrix_destroy(ctox_hip_matrix *matrix);
size_t ctox_hip_matrix_rows(const ctox_hip_matrix *matrix);
size_t ctox_hip_matrix_columns(const ctox_hip_matrix *matrix);
/* Device pointer to the resident packed weights (for benchmarks/tests). */
const void *ctox_hip_matrix_device_weights(const ctox_hip_matrix *matrix);

/* Batched fused matvec on device buffers: Y[m, r] = act((sum_k W[r,k] *
 * X[m,k] * s_in[k] + bias[r]) * s_out[r]) for m < batch. batch = 1 is the
 * decode matvec; 2 <= batch <= 8 is the MTP speculative-verify pass, equal to
 * `batch` independent fused_matvec calls (the crate verifies drafts with
 * sequential target steps, Q/src/decoder.rs:1344-1375; the CUDA five-row
 * verify is Q/src/backend/cuda_graph.rs:4565-4787). d_input is [batch,
 * columns] f32, d_output is [batch, rows] f32, both device memory. */
ctox_status ctox_hip_matrix_dispatch(ctox_hip_backend *backend, const ctox_hip_matrix *matrix,
                                     const float *d_input, size_t batch, float *d_output,
                                     void *stream);

/* Fan-out on device buffers: the activation is converted once and feeds
 * every matrix (Q/src/backend/cpu.rs:444-472, Q/src/fanout.rs:284-323). All
 * matrices must share `columns` and s_in. d_outputs[i] is [batch, rows_i]. */
ctox_status ctox_hip_matrix_dispatch_fanout(ctox_hip_backend *backend,
                                            const ctox_hip_matrix *const *matrices, size_t n,
                                            const float *d_input, size_t batch,
                                            float *const *d_outputs, void *stream);

/* ---- raw launch on device pointers ----
 * Same nine parameters, in the same order and meaning, as the SM86 fused
 * matvec parameter buffer (Q/src/backend/cuda.rs:73-122): weights (packed
 * pure Q2_B64 or Q4_B64 rows), input, s_in (fp16, NULL = 1.0), s_out (fp16,
 * NULL = 1.0), bias (NULL = 0), output, rows, columns, activation. Adds
 * `batch` (1..8 input rows, as the batched MMQ launch) and the stream. The
 * backend supplies the activation staging buffers. */
ctox_status ctox_hip_launch_fused_matvec(ctox_hip_backend *backend, int32_t dtype,
                                         const void *d_weights, const float *d_input,
                                         const uint16_t *d_s_in, const uint16_t *d_s_out,
                                         const float *d_bias, float *d_output, uint32_t rows,
                                         uint32_t columns, uint32_t activation, uint32_t batch,
                                         void *stream);

/* Allocation-free variant of ctox_hip_launch_fused_matvec. NO COUNTERPART
 * IN THE REFERENCE: it is for callers that cannot allocate device memory
 * (tight serving loops, harnesses that forbid hipMalloc). It must not be
 * captured into a HIP graph that is replayed: each launch tags its combine
 * slots with a number passed as a kernel argument, which a replay repeats.
 * Same arguments; the weights must have a tiled copy
 * (ctox_hip_register_tiled_weights, else CTOX_ERR_UNSUPPORTED_OPERATION) and
 * batch is 1..5. Results equal the allocating launch's, except for Q4
 * matrices of more than 8 Mi weights at 2..5 rows: there the allocating
 * launch stages 21-bit activation fragments and this one builds 22-bit
 * fragments in the kernel, so the two differ in the last bits (about 2^-21
 * relative). The cross-chunk combine slots come from a static device
 * array of CTOX_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends),
 * not from the backend's grown buffer; a matrix whose slots do not fit,
 * (chunks - 1) * batch * 16 * ceil(rows / 16) * 8 bytes with
 * chunks = ceil(columns / 1024), fails with CTOX_ERR_MEMORY_BUDGET. The call
 * allocates nothing. Every call on one GPU shares that GPU's array: calls
 * that overlap on one GPU (other streams, other threads, other backends)
 * race and must be ordered by the caller. */
#define CTOX_NOALLOC_SCRATCH_BYTES (8u << 20)
ctox_status ctox_hip_launch_fused_matvec_noalloc(ctox_hip_backend *backend, int32_t dtype, const void *d_weights,
                                                 const float *d_input, const uint16_t *d_s_in,
                                                 const uint16_t *d_s_out, const float *d_bias, float *d_output,
                                                 uint32_t rows, uint32_t columns, uint32_t activation,
                                                 uint32_t batch, void *stream);
/* Registers a tiled copy of raw packed weights already on the device
 * (pure Q2_B64 / Q4_B64, `rows` x `columns`, the crate's row layout at
 * d_weights). Batch-1 launches of the raw device entry points
 * (ctox_hip_launch_fused_matvec, ctox_hip_norm_matvec_device,
 * ctox_hip_transform_matvec_device) whose d_weights, rows and columns match a
 * registration then run the tiled-layout kernel, as resident matrices do
 * (the device-side counterpart of the CUDA runtime's prepare step,
 * Q/src/backend/cuda_runtime.rs:8341-8386). The copy is made in stream order
 * on `stream` and reflects the weights at that point; re-register after
 * changing them. Registering the same pointer again replaces the copy. */
ctox_status ctox_hip_register_tiled_weights(ctox_hip_backend *backend, int32_t dtype, const void *d_weights,
                                            uint32_t rows, uint32_t columns, void *stream);
/* Drops the tiled copy registered for d_weights (no-op when none is). */
void ctox_hip_unregister_tiled_weights(ctox_hip_backend *backend, const void *d_weights);

/* Residual add + (1 + w) RMS norm (Q/src/reference.rs:38-62) of `batch`
 * dense rows: h = d_x + d_delta (d_delta may be NULL: h = d_x), written to
 * d_x_out (required with d_delta, must not alias d_x); then the fused matvec
 * of ctox_hip_launch_fused_matvec (identity activation, no bias) on the
 * normalized rows, which also go to d_norm_out when it is set. A delta given
 * as delta_parts partial sums (d_delta + p * delta_part_stride, the output of
 * a split-K transform-matvec) is summed in part order first. The crate's
 * residual + norm -> projection pairs (Q/src/decoder.rs:640-657, :718-731,
 * :822-853) in one staging pass. columns <= 8192, delta_parts <= 8. */
ctox_status ctox_hip_norm_matvec_device(ctox_hip_backend *backend, const float *d_x, const float *d_delta,
                                        uint32_t delta_parts, size_t delta_part_stride, float *d_x_out,
                                        const float *d_norm_w, float eps, float *d_norm_out, int32_t dtype,
                                        const void *d_weights, const uint16_t *d_s_in, const uint16_t *d_s_out,
                                        float *d_output, uint32_t rows, uint32_t columns, uint32_t batch,
                                        void *stream);

/* ctox_hip_norm_matvec_device with the residual's sum of squares given as
 * per-16-row-tile partials, d_sums[batch][sum_count] (a producing
 * ctox_hip_transform_matvec_device's res_sums over d_x + d_delta), so that
 * no workgroup re-reads the whole rows for them. Used whenever the delta is
 * one part (batch 1 and 2..5 rows in the projection's launch, more rows in
 * the staging launch); with several delta parts the sums are computed from
 * the rows as before. */
ctox_status ctox_hip_norm_matvec_sums_device(ctox_hip_backend *backend, const float *d_x, const float *d_delta,
                                             uint32_t delta_parts, size_t delta_part_stride, float *d_x_out,
                                             const float *d_norm_w, float eps, float *d_norm_out, int32_t dtype,
                                             const void *d_weights, const uint16_t *d_s_in, const uint16_t *d_s_out,
                                             float *d_output, uint32_t rows, uint32_t columns, uint32_t batch,
                                             const float *d_sums, uint32_t sum_count, void *stream);

/* ctox_hip_norm_matvec_sums_device whose output may be left as partial
 * rows: on registered weights, when the K range is split into
 * n <= max_parts chunks, d_output receives n parts [n][batch][rows] (each
 * chunk's sum times s_out) whose sum in order is the projection, *parts = n,
 * and the cross-chunk combine is skipped; otherwise the result itself and
 * *parts = 1 (also for 2..5 rows built in the kernel from d_sums). For a consumer that adds them (ctox_input_transform::a_parts).
 * No crate counterpart (the crate's projection returns finished rows,
 * Q/src/backend/mod.rs:153-169). */
ctox_status ctox_hip_norm_matvec_parts_device(ctox_hip_backend *backend, const float *d_x, const float *d_delta,
                                              uint32_t delta_parts, size_t delta_part_stride, float *d_x_out,
                                              const float *d_norm_w, float eps, float *d_norm_out, int32_t dtype,
                                              const void *d_weights, const uint16_t *d_s_in, const uint16_t *d_s_out,
                                              float *d_output, uint32_t rows, uint32_t columns, uint32_t batch,
                                              const float *d_sums, uint32_t sum_count, uint32_t max_parts,
                                              uint32_t *parts, void *stream);

/* The projection of a value computed on the fly from its producer's output,
 * staged in the same pass (rows of a at t * a_stride, of b at t * b_stride):
 *   mode 1 swiglu (Q/src/reference.rs:96-112): silu(a[c]) * a[off + c];
 *   mode 2 rms_norm_gated per head of head_dim values (Q/src/reference.rs:66-93):
 *          a = core, b = gate z, w = norm weight [head_dim];
 *   mode 3 attention sigmoid gate (Q/src/decoder.rs:727-737, :788): a = attention
 *          output, b = q_proj rows holding [q, gate] per head. */
typedef struct {
    const float *a, *b, *w;
    uint32_t mode, a_stride, b_stride, off, head_dim;
    float eps;
    /* Optional (both NULL: off). When the output is a residual delta that
     * will be added to res_h [rows], res_sums receives, per 16-row tile t,
     * the sum over its rows r of (res_h[r] + out[r])^2: the sum of squares a
     * following ctox_hip_norm_matvec_sums_device needs (Q/src/reference.rs:38-62),
     * so that it need not re-read the whole residual row in every workgroup.
     * 1 row, or 2..5 rows of a matrix of at most 120 Mi weights, on
     * registered weights (row t: res_h + t * rows and
     * res_sums + t * ceil(rows / 16)); otherwise the call fails with
     * CTOX_ERR_UNSUPPORTED_OPERATION. No crate counterpart (the CPU decoder
     * adds and normalizes in one pass, Q/src/decoder.rs:636-680). */
    const float *res_h;
    float *res_sums;
    /* Mode 1 only, on registered weights: a holds a_parts (2..6) partials
     * a_part_stride floats apart (each batch rows of a_stride floats) whose
     * sum (in order) is the gate|up rows, as ctox_hip_norm_matvec_parts_device
     * leaves them (0 or 1: a is the rows themselves). */
    uint32_t a_parts, a_part_stride;
} ctox_input_transform;
/* split_k != 0 lets a batch-1 projection split its K range into one partial
 * per 1 KiB slice of a row (balancing few-row, long-K matrices over the
 * CUs): d_output then holds *parts partial outputs [parts][rows] whose sum
 * (in part order) is the result; *parts = 1 when no split was made. */
ctox_status ctox_hip_transform_matvec_device(ctox_hip_backend *backend, const ctox_input_transform *x, int32_t dtype,
                                             const void *d_weights, const uint16_t *d_s_in, const uint16_t *d_s_out,
                                             float *d_output, uint32_t rows, uint32_t columns, uint32_t batch,
                                             uint32_t split_k, uint32_t *parts, void *stream);

/* ---- gated delta (GatedDeltaNet) recurrence, fp32 state ----
 * Layouts follow Q/src/reference.rs:230-415: q, k [tokens][heads][key_dim]
 * (after Q/K head repetition), v [tokens][heads][value_dim], log_decay and
 * beta [tokens][heads], state [heads][key_dim][value_dim] row-major, updated
 * in place; out [tokens][heads][value_dim]. */
/* recurrent_gated_delta_step, Q/src/reference.rs:230-297 (host buffers). */
ctox_status ctox_hip_gated_delta_step(ctox_hip_backend *backend, const float *q, const float *k,
                                      const float *v, const float *log_decay, const float *beta,
                                      float *state, size_t heads, size_t key_dim,
                                      size_t value_dim, float *out);
/* recurrent_gated_delta_sequence, Q/src/reference.rs:377-415 (host buffers).
 * `chunk` = 0 selects the token-serial scan; chunk > 0 selects the chunked
 * prefill with that chunk length (64 for the benchmark). */
ctox_status ctox_hip_gated_delta_sequence(ctox_hip_backend *backend, const float *q,
                                          const float *k, const float *v, const float *log_decay,
                                          const float *beta, float *state, size_t tokens,
                                          size_t heads, size_t key_dim, size_t value_dim,
                                          size_t chunk, float *out);
/* Device-buffer forms of the two entry points above (same layouts). */
ctox_status ctox_hip_gated_delta_step_device(ctox_hip_backend *backend, const float *d_q,
                                             const float *d_k, const float *d_v,
                                             const float *d_log_decay, const float *d_beta,
                                             float *d_state, size_t heads, size_t key_dim,
                                             size_t value_dim, float *d_out, void *stream);
ctox_status ctox_hip_gated_delta_sequence_device(ctox_hip_backend *backend, const float *d_q,
                                                 const float *d_k, const float *d_v,
                                                 const float *d_log_decay, const float *d_beta,
                                                 float *d_state, size_t tokens, size_t heads,
                                                 size_t key_dim, size_t value_dim, size_t chunk,
                                                 float *d_out, void *stream);

/* GatedDeltaNet gates with a and b read at t * in_stride + h (token rows of a
 * fused projection output); outputs stay [tokens][heads]. */
ctox_status ctox_hip_gdn_gates_strided_device(ctox_hip_backend *backend, const float *d_a, const float *d_b,
                                              size_t in_stride, const float *d_a_log, const float *d_dt_bias,
                                              size_t tokens, size_t heads, float *d_log_decay, float *d_beta,
                                              void *stream);
/* The same recurrence reading q, k, v straight out of a fused projection /
 * convolution output: token t's q and k rows start at t * qk_stride floats,
 * v rows at t * v_stride; value head h uses key head h / (heads / key_heads),
 * which is repeat_heads (Q/src/decoder.rs:47-65, :868-880) without the copy.
 * chunk as in ctox_hip_gated_delta_sequence_device (0: token-serial scan). */
ctox_status ctox_hip_gated_delta_strided_device(ctox_hip_backend *backend, const float *d_q, const float *d_k,
                                                const float *d_v, size_t qk_stride, size_t v_stride,
                                                const float *d_log_decay, const float *d_beta, float *d_state,
                                                size_t tokens, size_t heads, size_t key_heads, size_t key_dim,
                                                size_t value_dim, size_t chunk, float *d_out, void *stream);
/* The GatedDeltaNet token mixer core of Q/src/decoder.rs:863-913 in one
 * launch over `tokens` projected rows (row t at d_proj + t * proj_stride:
 * [q (key_heads * key_dim) | k | v (heads * value_dim)] at 0, a at a_off, b at
 * b_off): causal conv + SiLU of the q, k, v channels (reference.rs:159-187)
 * from the windows in d_conv_in to d_conv_out ([channels][kernel], channels =
 * 2 key_heads key_dim + heads value_dim; must not alias d_conv_in), the gates
 * (decoder.rs:29-35, 881-902; written to d_log_decay / d_beta
 * [tokens][heads], or read from them when gates_given), and the recurrence of
 * ctox_hip_gated_delta_strided_device into d_state and d_out
 * [tokens][heads][value_dim]. key_dim <= 128, kernel <= 8. */
ctox_status ctox_hip_gdn_fused_device(ctox_hip_backend *backend, const float *d_proj, size_t proj_stride,
                                      size_t a_off, size_t b_off, const float *d_conv_w, const float *d_conv_in,
                                      float *d_conv_out, size_t kernel, const float *d_a_log, const float *d_dt_bias,
                                      float *d_log_decay, float *d_beta, int gates_given, float *d_state,
                                      size_t tokens, size_t heads, size_t key_heads, size_t key_dim,
                                      size_t value_dim, float *d_out, void *stream);
/* The same core with per-row snapshots, for the speculative verify of the
 * CUDA runtime's MTP branch (Q/src/backend/cuda_graph.rs:4565-4787 keeps a
 * restorable branch; here every row's state is kept instead of a checkpoint
 * and a replay): the state is read from d_state_in and the state after row
 * t is written at d_state_out + t * snap_stride (floats, at least
 * heads * key_dim * value_dim), the conv windows after row t at
 * d_conv_out + t * conv_snap_stride; no snapshot may overlap d_conv_in.
 * d_state_out may equal d_state_in. Gates are computed (never given).
 * blocked = 0: states [heads][key_dim][value_dim]; blocked = 1: the
 * engine's layout, per head and 16-column slice of the value dimension
 * 256 runs of 8 floats: element (h, i, j) at
 * ((h * S + j / 16) * 256 + (i % 16) * 16 + j % 16) * 8 + i / 16,
 * S = ceil(value_dim / 16), heads * S * 2048 floats per state, 16-byte
 * aligned (a wave moves 2 KiB per access instead of 64-byte pieces). */
ctox_status ctox_hip_gdn_fused_snap_device(ctox_hip_backend *backend, const float *d_proj, size_t proj_stride,
                                           size_t a_off, size_t b_off, const float *d_conv_w,
                                           const float *d_conv_in, float *d_conv_out, size_t conv_snap_stride,
                                           size_t kernel, const float *d_a_log, const float *d_dt_bias,
                                           float *d_log_decay, float *d_beta, const float *d_state_in,
                                           float *d_state_out, size_t snap_stride, int blocked, size_t tokens,
                                           size_t heads, size_t key_heads, size_t key_dim, size_t value_dim,
                                           float *d_out, void *stream);

/* ---- decode-step glue and token selection (device buffers) ---- */
/* GatedDeltaNet gates, Q/src/decoder.rs:881-902 (softplus :29-35):
 * beta = sigmoid(b), log_decay = -exp(A_log) * softplus(a + dt_bias), over
 * [tokens][heads] (A_log, dt_bias per head). */
ctox_status ctox_hip_gdn_gates_device(ctox_hip_backend *backend, const float *d_a, const float *d_b,
                                      const float *d_a_log, const float *d_dt_bias, size_t tokens,
                                      size_t heads, float *d_log_decay, float *d_beta, void *stream);
/* repeat_heads, Q/src/decoder.rs:47-65: out[row][h * repeats + r] = in[row][h]. */
ctox_status ctox_hip_repeat_heads_device(ctox_hip_backend *backend, const float *d_in, size_t rows,
                                         size_t heads, size_t dim, size_t repeats, float *d_out,
                                         void *stream);
/* Greedy token per logits row: argmax under f32::total_cmp, later index wins
 * ties (Q/src/engine.rs:906-913). d_tokens holds `rows` uint32. */
ctox_status ctox_hip_greedy_tokens_device(ctox_hip_backend *backend, const float *d_logits, size_t rows,
                                          size_t vocab, uint32_t *d_tokens, void *stream);
/* verify_greedy_mtp, Q/src/engine.rs:915-963 (full-logits branch): draft and
 * target are [drafts][vocab], bonus [vocab]. d_out receives 3 + drafts uint32:
 * next token, verified count, accepted count, accepted tokens. */
ctox_status ctox_hip_verify_greedy_mtp_device(ctox_hip_backend *backend, const float *d_draft,
                                              const float *d_target, const float *d_bonus, size_t drafts,
                                              size_t vocab, uint32_t *d_out, void *stream);
/* Speculative rejection-sampling accept at temperature > 0. No counterpart in
 * the crate (its MTP path is greedy-only, Q/src/engine.rs:583-590); draws are
 * the crate's Pcg32 (Q/src/sampler.rs:149-174), the replacement / bonus draw
 * uses the cumulative search of Q/src/sampler.rs:134-143. d_tokens: the
 * `drafts` proposed tokens; d_rng: Pcg32 state (uint64, advanced in place);
 * d_out receives 2 uint32: next token, accepted count; a proposed token
 * outside the vocabulary stops the pass with next token 0xFFFFFFFF. */
ctox_status ctox_hip_mtp_accept_device(ctox_hip_backend *backend, const float *d_draft, const float *d_target,
                                       const float *d_bonus, const uint32_t *d_tokens, size_t drafts,
                                       size_t vocab, float temperature, uint64_t *d_rng, uint32_t *d_out,
                                       void *stream);
/* The same acceptance with restricted draft rows (DraftDistribution::Restricted,
 * Q/src/engine.rs:151-200; the draft head of Q/src/decoder.rs:589-627 over the
 * release-bound draft vocabulary): draft rows hold draft_vocab scores and
 * d_draft_inv[t] (vocab entries) is token t's index in them, 0xffffffff for
 * tokens outside the draft vocabulary (q = 0 there). d_bonus_ids, when set,
 * maps a bonus-row index to its token: drafts = 0 with the bonus row a
 * restricted draft row of `vocab` = draft-vocabulary scores samples a draft
 * token. d_draft_inv may be NULL when draft_vocab == vocab. A non-finite
 * logit in any row fails closed: d_out[0] = 0xfffffffe, no draw is consumed. */
ctox_status ctox_hip_mtp_accept_restricted_device(ctox_hip_backend *backend, const float *d_draft,
                                                  size_t draft_vocab, const uint32_t *d_draft_inv,
                                                  const float *d_target, const float *d_bonus,
                                                  const uint32_t *d_bonus_ids, const uint32_t *d_tokens,
                                                  size_t drafts, size_t vocab, float temperature, uint64_t *d_rng,
                                                  uint32_t *d_out, void *stream);
/* Sampler::sample_with_draw, Q/src/sampler.rs:65-144, on device logits
 * [vocab] with the caller's draw in [0, 1): temperature 0 is greedy (the
 * later token wins ties); otherwise the top_k scaled logits (ties to the
 * later token), exp weights from their maximum, the nucleus where the
 * running weight first reaches top_p of the weights' sum, and the first
 * nucleus token whose running weight reaches draw x the nucleus total, in
 * the crate's sequential float arithmetic. As the CUDA runtime's sampler
 * (Q/kernels/cuda/q2q4_fused_matvec_sm86.cu:2647-2776), 1 <= top_k <= 256
 * (top_k = 0, the full-vocabulary nucleus, is not built:
 * CTOX_ERR_UNSUPPORTED_OPERATION), and ceil(vocab / 4096) * top_k <= 16384.
 * d_out[4] = {token, status, nucleus length, nucleus total (f32 bits)};
 * status 0 ok, 2 a non-finite logit or scaled logit, 4 an invalid
 * normalization (the crate's InvalidArtifact cases, reported on the device). */
ctox_status ctox_hip_sample_topk_topp_device(ctox_hip_backend *backend, const float *d_logits, size_t vocab,
                                             float temperature, uint32_t top_k, float top_p, float draw,
                                             uint32_t *d_out, void *stream);
/* Fail-closed check of a logits buffer (Q/src/backend/cuda_runtime.rs:10627-10632):
 * the n values are split into `parts` (1..1024) contiguous ranges and
 * d_flags[p] = 1 if range p holds a non-finite value, else 0 (every flag is
 * written). d_x 16-byte aligned. */
ctox_status ctox_hip_check_finite_device(ctox_hip_backend *backend, const float *d_x, size_t n, uint32_t *d_flags,
                                         size_t parts, void *stream);
/* dst row r = src row ids[r] (rows of row_bytes bytes; ids host values, each
 * below src_rows). Builds the restricted draft head's compact copy of the LM
 * head rows once at load (the CUDA runtime gathers them per launch instead,
 * Q/kernels/cuda/q2q4_fused_matvec_sm86.cu:607-703). Synchronizes `stream`. */
ctox_status ctox_hip_gather_rows_device(ctox_hip_backend *backend, const void *d_src, size_t src_rows,
                                        size_t row_bytes, const uint32_t *ids, size_t rows, void *d_dst,
                                        void *stream);

/* ---- layer glue (device buffers, fp32) ---- */
/* rms_norm with (1 + w) weight, Q/src/reference.rs:38-62, per row of [rows][cols]. */
ctox_status ctox_hip_rms_norm_device(ctox_hip_backend *backend, const float *d_x, size_t rows, size_t cols,
                                     const float *d_w, float eps, float *d_out, void *stream);
/* rms_norm_gated, Q/src/reference.rs:66-93: x * rsqrt(mean(x^2) + eps) * w * silu(gate). */
ctox_status ctox_hip_rms_norm_gated_device(ctox_hip_backend *backend, const float *d_x, const float *d_gate,
                                           size_t rows, size_t cols, const float *d_w, float eps, float *d_out,
                                           void *stream);
/* swiglu, Q/src/reference.rs:96-112: out = silu(gate) * up. */
ctox_status ctox_hip_swiglu_device(ctox_hip_backend *backend, const float *d_gate, const float *d_up, size_t n,
                                   float *d_out, void *stream);
/* sigmoid_gate, Q/src/reference.rs:502-515: values *= sigmoid(gate), in place. */
ctox_status ctox_hip_sigmoid_gate_device(ctox_hip_backend *backend, float *d_values, const float *d_gate,
                                         size_t n, void *stream);
/* causal_conv_silu update, Q/src/reference.rs:159-187: the [channels][kernel]
 * state shifts left by one, the input is appended, out = silu(state . weight). */
ctox_status ctox_hip_causal_conv_update_device(ctox_hip_backend *backend, const float *d_input, float *d_state,
                                               const float *d_weight, size_t channels, size_t kernel,
                                               float *d_out, void *stream);
/* causal_conv_silu_update over `rows` consecutive tokens, in order; token t's
 * input starts at t * in_stride floats (a slice of a fused projection
 * output), out is [rows][channels]. */
ctox_status ctox_hip_causal_conv_rows_device(ctox_hip_backend *backend, const float *d_input, size_t in_stride,
                                             float *d_state, const float *d_weight, size_t channels, size_t kernel,
                                             size_t rows, float *d_out, void *stream);
/* apply_partial_rope, Q/src/reference.rs:115-155, in place on q [rows][q_heads][head_dim]
 * and k [rows][k_heads][head_dim]; row t is at position + t. */
ctox_status ctox_hip_partial_rope_device(ctox_hip_backend *backend, float *d_q, float *d_k, size_t rows,
                                         size_t q_heads, size_t k_heads, size_t head_dim, size_t rotary_dim,
                                         uint64_t position, float theta, void *stream);

/* ---- paged mixed Q2/Q4 KV cache (device buffers) ----
 * Page layout of Q/src/kv_cache.rs:280-300: token-major [K heads, V heads]
 * canonical Q4_B64 / Q2_B64 blocks; a page is wholly Q2 or Q4 and lives at
 * pool + physical_slot * page_bytes in its pool. */
typedef struct {                /* CtoxPagedKvDescriptor, q2q4_fused_matvec_sm86.cu:1614-1619 */
    uint32_t precision;         /* 0 = Q2 pool, otherwise Q4 pool */
    uint32_t physical_slot;
    uint32_t tokens;
    uint32_t first_token;
} ctox_paged_kv_descriptor;

typedef struct {                /* CtoxPagedGqaParams, q2q4_fused_matvec_sm86.cu:1621-1634 */
    uint32_t query_heads;
    uint32_t key_value_heads;
    uint32_t head_dim;          /* 256 */
    uint32_t tokens;            /* cached tokens, the query rows included */
    uint32_t page_tokens;
    uint32_t page_count;
    uint32_t combined_values;   /* 2 * key_value_heads * head_dim */
    uint32_t q2_token_bytes;
    uint32_t q4_token_bytes;
    uint32_t q2_page_bytes;
    uint32_t q4_page_bytes;
    float scale;                /* 1 / sqrt(head_dim) in Q/src/reference.rs:420-499 */
} ctox_paged_gqa_params;

/* Quantize token_count K/V rows ([token][component_values] each) into
 * consecutive slots of one Q4 page starting at first_token_in_page,
 * bit-exact with QuantizedKvPage::push (Q/src/kv_cache.rs:200-206,
 * Q4Block64::quantize Q/src/quant.rs:144-168). Replaces
 * ctox_pack_paged_kv_q4_batch_f32_sm86 (q2q4_fused_matvec_sm86.cu:1734-1799). */
ctox_status ctox_hip_kv_pack_q4_device(ctox_hip_backend *backend, uint8_t *d_q4_pages, const float *d_keys,
                                       const float *d_values, size_t token_count, size_t component_values,
                                       uint32_t physical_slot, uint32_t first_token_in_page,
                                       uint32_t q4_page_bytes, void *stream);
/* An attention layer's K/V append for `rows` (<= 8) projected rows, fused:
 * per q head RMS norm with q_norm ((1 + w), Q/src/reference.rs:38-62) and
 * partial RoPE (:115-155) into d_q_out [rows][q_heads][head_dim]; per k head
 * the same with k_norm, then K and V (the v part of the row as it is)
 * quantized into Q4 page slot slots[t] at token positions_in_page[t], as
 * ctox_hip_kv_pack_q4_device does. d_proj rows: per q head [q, gate] (2 *
 * head_dim), then k [kv_heads * head_dim], then v. Replaces the q/k norm,
 * RoPE and KV-append steps of FullAttentionState::append
 * (Q/src/decoder.rs:687-800, Q/src/kv_cache.rs:200-206) and the CUDA
 * runtime's query-gate-norm-rope + pack pair (q2q4_fused_matvec_sm86.cu:1491-1546,
 * :1734-1799). head_dim 256. Up to 32 further words (words[word_count],
 * e.g. changed page descriptors) are stored to d_words_dst in the same
 * launch, as ctox_hip_write_words_device would. */
ctox_status ctox_hip_attn_prep_device(ctox_hip_backend *backend, const float *d_proj, size_t proj_stride,
                                      const float *d_q_norm, const float *d_k_norm, size_t rows, size_t q_heads,
                                      size_t kv_heads, size_t head_dim, size_t rotary_dim, uint64_t position,
                                      float theta, float eps, uint8_t *d_q4_pages, uint32_t q4_page_bytes,
                                      const uint32_t *slots, const uint32_t *positions_in_page, float *d_q_out,
                                      uint32_t *d_words_dst, const uint32_t *words, size_t word_count,
                                      void *stream);
/* Rewrite one Q4 page as Q2, byte-identical to QuantizedKvPage::requantize
 * (Q/src/kv_cache.rs:216-236). Replaces ctox_demote_paged_kv_q4_to_q2_sm86
 * (q2q4_fused_matvec_sm86.cu:1801-1834). */
ctox_status ctox_hip_kv_demote_device(ctox_hip_backend *backend, const uint8_t *d_q4_page, uint8_t *d_q2_page,
                                      size_t tokens, size_t blocks_per_token, void *stream);
/* Grouped-query attention of query_tokens rows (d_query [rows][query_heads][256],
 * the last rows cached tokens; row t sees tokens 0 ..= tokens - rows + t) over
 * the paged cache; d_out [rows][query_heads][256]. Q/src/reference.rs:420-499
 * over flattened pages (Q/src/kv_cache.rs:579-605). Replaces the split-KV pair
 * ctox_paged_q2q4_gqa_split_partial/_combine_f32_sm86
 * (q2q4_fused_matvec_sm86.cu:2296-2558) and the one-row decode kernel
 * (:2026-2100). Limits: head_dim 256, (query_heads / key_value_heads) * rows <= 32. */
ctox_status ctox_hip_paged_gqa_device(ctox_hip_backend *backend, const float *d_query, const uint8_t *d_q2_pages,
                                      const uint8_t *d_q4_pages, const ctox_paged_kv_descriptor *d_descriptors,
                                      const ctox_paged_gqa_params *params, size_t query_tokens, float *d_out,
                                      void *stream);

/* ---- decode engine helpers (device buffers) ---- */
/* Seeded synthetic tensors (counter-based, reproducible for any sub-range):
 * kind 0 Q4_B64 blocks and 1 Q2_B64 blocks (uniform codes, fp16 scale
 * |N(0, p1)|; count = blocks), 2 f32 N(p0, p1), 3 fp16 U(p0, p1), 4 f32
 * U(p0, p1). No counterpart in the crate, which loads real artifacts. */
ctox_status ctox_hip_fill_random_device(ctox_hip_backend *backend, void *d_ptr, uint64_t count, uint32_t kind,
                                        uint64_t seed, float p0, float p1, void *stream);
/* ArtifactDecoder::embedding (Q/src/decoder.rs:531-537) for `rows` token ids
 * held on the device: recovered_row (Q/src/backend/cpu.rs:474-476) of each. */
ctox_status ctox_hip_embedding_rows_device(ctox_hip_backend *backend, int32_t dtype, const uint8_t *d_weights,
                                           const uint16_t *d_s_in, const uint16_t *d_s_out, const uint32_t *d_tokens,
                                           size_t rows, size_t vocab, size_t cols, float *d_out, void *stream);
/* RMS norms of Q/src/reference.rs:38-93 over rows addressed with two-level
 * strides (row r at (r / inner) * x_outer + (r % inner) * x_inner floats),
 * optionally adding a residual delta first (x += delta, written back). */
typedef struct {
    float *x;
    const float *delta;  /* [rows][cols] or NULL */
    const float *gate;   /* mode 1 only, addressed like x with g_inner / g_outer */
    const float *w;
    float *out;          /* row r at r * out_stride */
    uint32_t rows, cols, mode, inner;  /* mode 0: (1 + w); 1: w * silu(gate) */
    float eps;
    uint32_t delta_parts;  /* 0 or 1: one delta; n: n partial sums delta_stride floats apart */
    uint64_t x_inner, x_outer, g_inner, g_outer, out_stride, delta_stride;
} ctox_norm_rows;
ctox_status ctox_hip_norm_rows_device(ctox_hip_backend *backend, const ctox_norm_rows *desc, void *stream);
/* values[t][h][d] *= sigmoid(gate): the gate half of each head's [q, gate]
 * in q_proj's output rows (Q/src/decoder.rs:727-737, :788). */
ctox_status ctox_hip_attention_gate_device(ctox_hip_backend *backend, float *d_values, const float *d_qg, size_t rows,
                                           size_t heads, size_t head_dim, size_t qg_stride, void *stream);
/* swiglu (Q/src/reference.rs:96-112) over token rows of a fused gate|up
 * projection: out[t][c] = silu(in[t][c]) * in[t][up_offset + c]. */
ctox_status ctox_hip_swiglu_rows_device(ctox_hip_backend *backend, const float *d_in, size_t in_stride,
                                        size_t up_offset, size_t rows, size_t cols, float *d_out, size_t out_stride,
                                        void *stream);
/* out[t][c] = in[t * in_stride + col_offset + c]. */
ctox_status ctox_hip_copy_rows_device(ctox_hip_backend *backend, const float *d_in, size_t in_stride,
                                      size_t col_offset, size_t rows, size_t cols, float *d_out, size_t out_stride,
                                      void *stream);

/* Writes `count` 32-bit words to device memory in stream order; the words
 * travel in kernel arguments, so the host array may be reused on return. */
ctox_status ctox_hip_write_words_device(ctox_hip_backend *backend, uint32_t *d_dst, const uint32_t *words,
                                        size_t count, void *stream);

/* A plain streaming read of `bytes` (a multiple of 16) with the tiled
 * matvec's access pattern (each wave 8 KiB, every 16-byte load issued before
 * the first wait, non-temporal); d_out receives ceil(bytes / 8192) words.
 * No counterpart in the reference: the HBM read floor the matvec kernels
 * are measured against (bench.py). */
ctox_status ctox_hip_stream_read_device(ctox_hip_backend *backend, const void *d_src, size_t bytes, uint32_t *d_out,
                                        void *stream);

/* ---- device-resident decode engine (engine.cpp) ----
 * The crate's model graph (Q/src/decoder.rs:427-1114) and MTP executor
 * (:1217-1458, CUDA MTP4 flow cuda_executor.rs:797-889) over the entry points
 * above, with synthetic seeded weights of the configured shapes (the crate
 * would hand its loaded tensors instead). Geometry as Qwen38Config
 * (Q/src/config.rs:35-73). */
typedef struct {
    uint32_t hidden_size, intermediate_size, num_hidden_layers, full_attention_interval;
    uint32_t num_attention_heads, num_key_value_heads, head_dim, rotary_dim;
    uint32_t linear_num_key_heads, linear_num_value_heads, linear_key_head_dim, linear_value_head_dim;
    uint32_t linear_conv_kernel_dim, vocab_size, max_tokens;
    uint32_t page_tokens, sink_tokens, recent_tokens;  /* paged KV policy, Q/src/kv_cache.rs:10-12 */
    uint32_t mtp_layers;      /* 0 or 1 */
    uint32_t draft_tokens;    /* k drafts per speculative step, 0..7 */
    float rms_norm_epsilon, rope_theta;
} ctox_engine_config;

typedef struct {
    void *data;               /* device pointer */
    size_t bytes;
    uint32_t rows, cols;
    int32_t dtype;            /* CTOX_DTYPE_* for quantized matrices, -1 for f32 vectors */
    uint32_t pad;
    const uint16_t *s_in, *s_out;  /* fp16 device vectors of quantized matrices */
} ctox_engine_tensor;

typedef struct ctox_hip_engine ctox_hip_engine;

ctox_status ctox_hip_engine_create(ctox_hip_backend *backend, const ctox_engine_config *config, uint64_t seed,
                                   ctox_hip_engine **out);

/* Loading a `.ctoxq` model artifact into the engine (CpuCorrectnessExecutor::load,
 * Q/src/decoder.rs:1149-1182, over the tensor contract of
 * Q/src/tensor_contract.rs:137-244). The engine's matrices are the crate's
 * fan-out groups concatenated by rows ("L<i>.in" = in_proj_qkv|z|a|b,
 * "L<i>.qkv" = q|k|v, "L<i>.gate_up" = gate|up), one packed dtype each:
 * create with the dtype plan of the artifact (names as ctox_hip_engine_tensor;
 * unnamed matrices keep the default plan: Q4_B64, down projections Q2_B64),
 * write every tensor, then finish. A mixed or mixed-member matrix is created
 * Q4_B64 and its Q2 rows are written widened (Q2 code c -> Q4 code 5c, the
 * same block scale: value-exact, Q/src/quant.rs codebooks). */
typedef struct {
    const char *name;
    int32_t dtype;            /* CTOX_DTYPE_Q2B64 or CTOX_DTYPE_Q4B64 */
} ctox_engine_matrix_dtype;
ctox_status ctox_hip_engine_create_with_dtypes(ctox_hip_backend *backend, const ctox_engine_config *config,
                                               uint64_t seed, const ctox_engine_matrix_dtype *plan, size_t plan_len,
                                               ctox_hip_engine **out);
/* Parts of a named tensor. */
#define CTOX_ENGINE_PART_DATA 0   /* packed rows of a matrix, or the f32 values of a vector */
#define CTOX_ENGINE_PART_S_IN 1   /* fp16 s_in of a matrix */
#define CTOX_ENGINE_PART_S_OUT 2  /* fp16 s_out of a matrix */
/* Copies `bytes` host bytes into part `part` of tensor `name` at byte offset
 * `offset` (an engine at position 0 with no draft vocabulary bound, else
 * CTOX_ERR_INVALID_STATE; out of range: CTOX_ERR_SHAPE). Steps are refused
 * until ctox_hip_engine_finish_load. */
ctox_status ctox_hip_engine_write(ctox_hip_engine *engine, const char *name, uint32_t part, size_t offset,
                                  const void *host, size_t bytes);
/* Rebuilds the tiled copies of every written matrix; steps are allowed again. */
ctox_status ctox_hip_engine_finish_load(ctox_hip_engine *engine);
void ctox_hip_engine_destroy(ctox_hip_engine *engine);
void *ctox_hip_engine_stream(ctox_hip_engine *engine);
/* Pcg32 state of the sampler (Q/src/sampler.rs:149-174). */
ctox_status ctox_hip_engine_set_rng(ctox_hip_engine *engine, uint64_t state);
/* One target step, decode_target_step (Q/src/decoder.rs:956-998) plus the MTP
 * cache advance of prefill (:1248-1261); *d_logits = the next-token logits. */
ctox_status ctox_hip_engine_decode(ctox_hip_engine *engine, uint32_t token, const float **d_logits);
/* One speculative step at `temperature`: out[0] next token, out[1] accepted
 * drafts n, out[2 .. 2 + n) the accepted drafts (out holds >= 2 + k words).
 * Temperature 0 is the crate's greedy MTP (Q/src/engine.rs:583-590, 915-963;
 * argmax drafts, Q/src/decoder.rs:1311-1329): the longest draft prefix equal
 * to the target argmax tokens is accepted, then the first differing target
 * token or the bonus row's argmax; temperature > 0 is rejection sampling
 * with the engine's Pcg32 stream. Non-finite logits: CTOX_ERR_INVALID_STATE,
 * nothing committed; a negative or non-finite temperature:
 * CTOX_ERR_INVALID_ARTIFACT.
 * The commit's device work (MTP cache replay, descriptor uploads) may still
 * run on the engine stream when the call returns; every later engine call
 * and every read of engine memory through that stream (or the legacy null
 * stream) is ordered after it. */
ctox_status ctox_hip_engine_mtp_step(ctox_hip_engine *engine, uint32_t token, float temperature, uint32_t *out);
/* Fill every paged cache with `tokens` random K/V rows (an empty engine only). */
ctox_status ctox_hip_engine_fill_context(ctox_hip_engine *engine, uint32_t tokens, uint64_t seed);
/* which: 0 logits [R][V], 1 final hiddens [R][H], 2 previous target hidden,
 * 3 GatedDeltaNet states (the blocked layout of
 * ctox_hip_gdn_fused_snap_device), 4 conv states, 5 draft logits [k][V]. */
ctox_status ctox_hip_engine_buffer(ctox_hip_engine *engine, uint32_t which, void **d_ptr, size_t *bytes);
uint32_t ctox_hip_engine_position(const ctox_hip_engine *engine);
/* Binds the release's MTP draft vocabulary (ModelExecutor::load's
 * mtp_draft_token_ids, Q/src/engine.rs:331 and Q/src/decoder.rs:1129-1182;
 * canonical: strictly increasing, inside the vocabulary, else
 * CTOX_ERR_INVALID_ARTIFACT). Set once; drafts then use the restricted LM
 * head (Q/src/decoder.rs:589-627) and the acceptance sees restricted draft
 * distributions. Without it drafts score the full vocabulary. */
ctox_status ctox_hip_engine_set_draft_vocab(ctox_hip_engine *engine, const uint32_t *ids, size_t n);
/* Weights by name ("embed", "lm_head", "final_norm", "L<i>.<part>", "mtp.<part>"). */
ctox_status ctox_hip_engine_tensor(ctox_hip_engine *engine, const char *name, ctox_engine_tensor *out);

typedef struct {                /* one paged cache of the engine (test view) */
    const ctox_paged_kv_descriptor *descriptors;  /* host copy, `pages` entries */
    uint32_t pages, tokens;
    const uint8_t *d_q4_pool, *d_q2_pool;         /* slot pools (device) */
    uint32_t q4_page_bytes, q2_page_bytes;
} ctox_engine_cache_view;
/* The paged K/V cache of full-attention layer `layer` (layer index of the
 * model; 0xffffffff: the MTP layer's cache), as PagedKvCache::page_views
 * exposes pages (Q/src/kv_cache.rs:558-575): valid until the next step. */
ctox_status ctox_hip_engine_cache(ctox_hip_engine *engine, uint32_t layer, ctox_engine_cache_view *out);

#ifdef __cplusplus
}
#endif
#endif /* CTOX_HIP_H */
