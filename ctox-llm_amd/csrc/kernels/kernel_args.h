// Kernel argument blocks shared by the device code object and the host shim.
// Every kernel takes exactly one of these structs by value; the shim passes
// it through hipModuleLaunchKernel's kernelParams. Plain C layout only.
#pragma once
#include <stdint.h>

#define CTOX_BLOCK_LEN 64
#define CTOX_Q2_BLOCK_BYTES 18
#define CTOX_Q4_BLOCK_BYTES 34
// Matvec tiling: a workgroup is 4 waves sharing 16 rows; each wave covers a
// quarter of the K dimension.
#define CTOX_MV_WAVES 4
#define CTOX_MV_ROWS 16
#define CTOX_MAX_BATCH 8
// Activation fixed-point: |X| <= 2^22 per 64-column block, three signed
// 8-bit limbs (X = X0 + 2^8 X1 + 2^16 X2).
#define CTOX_XFRAC_BITS 22

// Scale pointer kinds inside kernels.
#define CTOX_KSCALE_NONE 0
#define CTOX_KSCALE_F32 1
#define CTOX_KSCALE_F16 2

// Converts a [batch][columns] f32 activation (times s_in) into the int8
// MFMA A-fragment rows consumed by ctox_q*_matvec_*: for every 64-column
// block b and token t, three limbs x four k-groups x 16 bytes (192 bytes).
// Per (block, token) it also writes the float4 epilogue constants
// {2q, 512q, 131072q, K*q} (q = quantum, K = -off * sum of the limbs).
struct PrepArgs {
    const float *input;     // [batch][columns]
    const void *s_in;       // NULL, f32[columns] or f16[columns]
    int8_t *xa;             // [blocks][batch][3 limbs][4 k-groups][16]
    float *xc;              // [blocks][batch][4]
    uint32_t columns;
    uint32_t batch;
    uint32_t dtype;         // 0 = Q2 layout, 1 = Q4 layout
    uint32_t s_in_kind;
    uint32_t tgroups;       // ceil(batch / 4)
    uint32_t pad;
};

// One workgroup per 16 output rows (grid = ceil(rows / 16)); its four waves
// split the K dimension.
struct MatvecArgs {
    const uint8_t *weights; // packed rows of this launch (pure Q2 or Q4)
    uint64_t weights_len;   // bytes readable from `weights`
    const int8_t *xa;       // prep output
    const float *xc;        // prep output
    const void *s_out;      // NULL, f32[rows] or f16[rows]
    const float *bias;      // NULL or f32[rows]
    float *output;          // [batch][out_stride], row r at output[m*out_stride + r]
    uint32_t rows;
    uint32_t columns;
    uint32_t batch;
    uint32_t out_stride;
    uint32_t s_out_kind;
    uint32_t activation;
};

// Batch-1 slice kernels (rows of whole 16-byte units): a workgroup of
// CTOX_SLICE_WAVES waves walks a 16-row tile in slices of 28 (Q4) / 56 (Q2)
// blocks, each slice one 1 KiB coalesced load per row.
constexpr uint32_t ctox_slice_blocks(uint32_t dtype) { return dtype ? 28u : 56u; }
#define CTOX_SLICE_WAVES 8

struct RecoveredRowArgs {
    const uint8_t *weights; // one packed row
    const void *s_in;       // f32 or f16 [columns]
    float *output;          // [columns]
    uint32_t columns;
    uint32_t dtype;
    uint32_t s_in_kind;
    float s_out;
};

struct RowDotArgs {
    const uint8_t *weights; // one packed row
    const float *x;         // corrected input [len]
    float *result;          // 1 float
    uint32_t len;
    uint32_t dtype;
    float s_out;
    uint32_t pad;
};

// Gated-delta recurrence. State [heads][key_dim][value_dim] f32.
struct GdnArgs {
    const float *q;         // [tokens][heads][key_dim]
    const float *k;
    const float *v;         // [tokens][heads][value_dim]
    const float *log_decay; // [tokens][heads]
    const float *beta;      // [tokens][heads]
    float *state;
    float *out;             // [tokens][heads][value_dim]
    float *norms;           // chunked prefill scratch: per (head, chunk) T, A, G, k_inv, q_inv
    uint32_t tokens;
    uint32_t heads;
    uint32_t key_dim;
    uint32_t value_dim;
    uint32_t chunk;
    uint32_t pad;
};
