/*
 * ctox_oracle.h -- CPU restatement of CTOX-LLM's scalar correctness oracle for
 * the Qwen3.8-27B decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing under oracle/ is part of the product:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and only as the checker (or the timed CPU baseline). The HIP
 * product path never calls into this library.
 *
 * Every function cites the reference source it restates. Paths are relative
 * to the reference tree, with Q/ = models/qwen38_27b/.
 *
 * Numerics contract: compiled with -O2 -ffp-contract=off (Rust never fuses
 * a*b+c), glibc expf/log1pf/sqrtf, and round-to-nearest-even f32->f16
 * (the `half` 2.7.1 crate semantics). Summation order follows the Rust
 * iterators exactly (sequential left-to-right f32 accumulation).
 */
#ifndef CTOX_ORACLE_H
#define CTOX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: identical numbering to include/ctox_hip.h (EngineError). */
enum {
    ORC_OK = 0,
    ORC_ERR_INVALID_ARTIFACT = 3,
    ORC_ERR_UNSUPPORTED_DTYPE = 4,
    ORC_ERR_UNSUPPORTED_OPERATION = 5,
    ORC_ERR_SHAPE = 7,
    ORC_ERR_INVALID_STATE = 8,
};

/* TensorDType (Q/src/format.rs:26-33). */
enum { ORC_Q2B64 = 0, ORC_Q4B64 = 1, ORC_MIXED = 2, ORC_F16 = 3, ORC_F32 = 4 };
/* Scale slice kind (Q/src/backend/mod.rs:74-78); 0 = None. */
enum { ORC_SCALE_NONE = 0, ORC_SCALE_F32 = 1, ORC_SCALE_F16LE = 2 };
/* CPU profile (Q/src/backend/cpu.rs:15-19). */
enum { ORC_PROFILE_SCALAR = 0, ORC_PROFILE_AVX2 = 1 };

typedef struct {
    uint32_t group_index;
    uint64_t row_start, row_end;
    int32_t dtype;
    uint64_t offset, length;
} orc_segment;

typedef struct {
    int32_t kind;          /* ORC_SCALE_* */
    const void *data;      /* float* or little-endian f16 bytes */
    size_t len;            /* number of values (not bytes) */
} orc_scale;

/* FusedMatVec descriptor (Q/src/backend/mod.rs:115-128). */
typedef struct {
    int32_t dtype;
    const uint8_t *weights;
    size_t weights_len;
    const orc_segment *segments;
    size_t n_segments;
    size_t rows, columns;
    const float *input;
    size_t input_len;
    orc_scale s_in, s_out;
    const float *bias;     /* NULL = None */
    size_t bias_len;
    int32_t activation;    /* 0 identity, 1 SiLU */
} orc_matvec_op;

/* ---- f16 (half 2.7.1) ---- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);

/* ---- quant.rs ---- */
int orc_q2_quantize(const float *values64, uint8_t out18[18]);
int orc_q4_quantize(const float *values64, uint8_t out34[34]);
int orc_a8_quantize(const float *values64, float *scale, int8_t codes[64]);
int orc_q2_decode_check(const uint8_t block18[18]);
int orc_q4_decode_check(const uint8_t block34[34]);
float orc_q2_value(const uint8_t block18[18], size_t index);
float orc_q4_value(const uint8_t block34[34], size_t index);

/* ---- backend/cpu.rs ---- */
int orc_validate(const orc_matvec_op *op, size_t *blocks_per_row);
int orc_fused_matvec(int profile, const orc_matvec_op *op, float *output);
int orc_fused_matvec_fanout(int profile, const orc_matvec_op *ops, size_t n,
                            float *const *outputs);
int orc_recovered_row(int32_t dtype, const uint8_t *weights, size_t weights_len,
                      size_t columns, orc_scale s_in, float s_out, float *output);
int orc_recovered_row_matvec(int profile, int32_t dtype, const uint8_t *weights,
                             size_t weights_len, const float *corrected_input,
                             size_t len, float s_out, float *result);
float orc_packed_q2_dot(int profile, float scale, const uint8_t codes[16], const float x[64]);
float orc_packed_q4_dot(int profile, float scale, const uint8_t codes[32], const float x[64]);
int orc_avx2_available(void);
/* Row-parallel driver over `threads` POSIX threads (not crate behaviour;
 * used only for the optional multi-core CPU baseline). */
int orc_fused_matvec_threads(int profile, const orc_matvec_op *op, float *output, int threads);

/* ---- reference.rs ---- */
int orc_gated_delta_step(const float *q, const float *k, const float *v,
                         const float *log_decay, const float *beta, float *state,
                         size_t heads, size_t key_dim, size_t value_dim, float *out);
int orc_gated_delta_step_f16_state(const float *q, const float *k, const float *v,
                                   const float *log_decay, const float *beta, uint16_t *state,
                                   size_t heads, size_t key_dim, size_t value_dim, float *out);
int orc_gated_delta_sequence(const float *q, const float *k, const float *v,
                             const float *log_decay, const float *beta, float *state,
                             size_t tokens, size_t heads, size_t key_dim, size_t value_dim,
                             float *out);
int orc_rms_norm_1p_weight(const float *x, size_t rows, size_t cols, const float *w,
                           float eps, float *out);
int orc_rms_norm_gated(const float *x, const float *gate, size_t rows, size_t cols,
                       const float *w, float eps, float *out);
int orc_swiglu(const float *gate, const float *up, size_t n, float *out);
int orc_causal_conv_silu_update(const float *input, float *state, const float *weight,
                                size_t channels, size_t kernel, float *out);
int orc_apply_partial_rope(float *q, float *k, size_t qh, size_t kh, size_t head_dim,
                           size_t rotary_dim, uint64_t position, float theta);
int orc_grouped_query_attention(const float *q, const float *k, const float *v,
                                size_t qh, size_t kvh, size_t q_tokens, size_t kv_tokens,
                                size_t head_dim, size_t q_start, float *out);
int orc_sigmoid_gate(float *values, const float *gate, size_t n);

/* ---- decoder.rs glue ---- */
float orc_softplus(float x);
int orc_repeat_heads(const float *values, size_t heads, size_t dim, size_t repeats, float *out);
/* beta = sigmoid(b); log_decay = -exp(A_log) * softplus(a + dt_bias) */
void orc_gdn_gates(const float *a, const float *b, const float *a_log, const float *dt_bias,
                   size_t heads, float *log_decay, float *beta);

/* ---- sampler.rs / engine.rs ---- */
typedef struct { uint64_t state; } orc_pcg32;
void orc_pcg32_init(orc_pcg32 *g, uint64_t seed);
uint32_t orc_pcg32_next_u32(orc_pcg32 *g);
float orc_pcg32_next_f32(orc_pcg32 *g);
int orc_sample_with_draw(const float *logits, size_t n, float temperature, size_t top_k,
                         float top_p, float draw, size_t *token);
int orc_greedy_token(const float *logits, size_t n, uint32_t *token);
/* verify_greedy_mtp over full logits: draft[i], target[i] are vocab-length rows. */
int orc_verify_greedy_mtp(const float *draft_logits, const float *target_logits,
                          const float *bonus_logits, size_t drafts, size_t vocab,
                          uint32_t *next_token, uint32_t *verified, uint32_t *accepted,
                          uint32_t *n_accepted);
/* Speculative rejection-sampling acceptance at temperature T (no crate
 * counterpart: the crate's MTP is greedy-only; pinned by the closed forms of
 * rejection sampling, not by the crate). */
int orc_mtp_accept_sample(const float *draft_logits, const float *target_logits,
                          const float *bonus_logits, const uint32_t *draft_tokens,
                          size_t drafts, size_t vocab, float temperature, orc_pcg32 *rng,
                          uint32_t *next_token, uint32_t *n_accepted);
/* The same with restricted draft rows of draft_n scores over draft_ids. */
int orc_mtp_accept_sample_restricted(const float *draft_logits, const uint32_t *draft_ids, size_t draft_n,
                                     const float *target_logits, const float *bonus_logits,
                                     const uint32_t *draft_tokens, size_t drafts, size_t vocab,
                                     float temperature, orc_pcg32 *rng, uint32_t *next_token,
                                     uint32_t *n_accepted);

#ifdef __cplusplus
}
#endif
#endif
