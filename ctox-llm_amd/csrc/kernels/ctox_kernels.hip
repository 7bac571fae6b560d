// Single code object for every gfx950 kernel of the backend.
#include "qmatvec.hip"
#include "qmatvec_slices.hip"
#include "gated_delta.hip"
#include "gated_delta_chunk.hip"
#include "decode_ops.hip"
#include "layer_ops.hip"
#include "paged_attention.hip"
#include "engine_ops.hip"
