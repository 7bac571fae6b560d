// Library-internal entry points shared by the shim (ctox_hip.cpp) and the
// decode engine (engine.cpp); not part of the C ABI in include/ctox_hip.h.
#pragma once

#include "ctox_hip.h"

// A residual-delta projection of 2..8 rows (the transform-matvec, on the
// staged small-M path) that also stages the input of the (1 + w) RMS-normed
// projection that follows it: h = x->res_h + output goes to next_h_out,
// h * (1 + next_norm_w) * next_s_in is staged in the backend's next-norm
// buffers for a matrix of next_dtype, and next_sq_out [batch][rows / 64]
// receives per-64-row sums of h^2. *staged reports whether the staging was
// made (otherwise the call is the plain transform-matvec and the caller
// stages the norm itself). input_staged: x's transform of this call was
// already staged (ctox_paged_gqa_stage_o_device), no staging launch is made;
// only valid where ctox_small_m_staged holds.
ctox_status ctox_delta_matvec_stage_next(ctox_hip_backend *b, const ctox_input_transform *x, int32_t dtype,
                                         const void *d_weights, const uint16_t *d_s_in, const uint16_t *d_s_out,
                                         float *d_output, uint32_t rows, uint32_t columns, uint32_t batch,
                                         const float *next_norm_w, const uint16_t *next_s_in, int32_t next_dtype,
                                         float *next_h_out, float *next_sq_out, bool *staged, void *stream,
                                         bool input_staged = false);

// The projection of what ctox_delta_matvec_stage_next staged: registered
// weights of next_dtype, the same batch, `sq` its per-block sums of h^2 and
// eps the norm's epsilon. max_parts / parts as for
// ctox_hip_norm_matvec_parts_device.
ctox_status ctox_norm_matvec_prestaged(ctox_hip_backend *b, int32_t dtype, const void *d_weights,
                                       const uint16_t *d_s_out, float *d_output, uint32_t rows, uint32_t columns,
                                       uint32_t batch, const float *sq, float eps, uint32_t max_parts, uint32_t *parts,
                                       void *stream);

// ctox_hip_greedy_tokens_device whose row argmax index i is written as
// d_ids[i] (a restricted draft row's index mapped to its token) when d_ids
// is not null.
ctox_status ctox_greedy_tokens_mapped(ctox_hip_backend *b, const float *d_logits, size_t rows, size_t vocab,
                                      const uint32_t *d_ids, uint32_t *d_tokens, void *stream);

// Writes n host word ranges (src[i], count[i] words) to device addresses
// dst[i] with as few launches as the argument block allows (one for the
// engine's per-step descriptor uploads).
ctox_status ctox_write_word_ranges_device(ctox_hip_backend *b, uint32_t *const *dst, const uint32_t *const *src,
                                          const size_t *count, size_t n, void *stream);

// Whether a 2..8-row projection of these registered weights runs the staged
// small-M kernels (its input staged by a separate pass), not the in-kernel build.
bool ctox_small_m_staged(ctox_hip_backend *b, const void *d_weights, uint32_t batch, uint32_t rows, uint32_t columns);

// ctox_hip_paged_gqa_device whose combine also stages the o projection's
// input (attention output times sigmoid of the gate half of d_gate's rows,
// gate_stride floats apart, times the o projection's f16 s_in) for a staged
// small-M launch of an o_dtype matrix; the transform-matvec then passes
// input_staged.
ctox_status ctox_paged_gqa_stage_o_device(ctox_hip_backend *b, const float *d_query, const uint8_t *d_q2_pages,
                                          const uint8_t *d_q4_pages, const ctox_paged_kv_descriptor *d_descriptors,
                                          const ctox_paged_gqa_params *p, size_t rows, float *d_out,
                                          const float *d_gate, uint32_t gate_stride, const uint16_t *d_o_s_in,
                                          int32_t o_dtype, void *stream);
