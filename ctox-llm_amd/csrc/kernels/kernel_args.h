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
// Activation fixed-point: |X| <= 2^F per 64-column block, three signed
// 8-bit limbs (X = X0 + 2^8 X1 + 2^16 X2). F = 22, except for Q4 weights in
// the staged fragments (xa / xc, written by the prep kernels), where F = 21.
// With codes c <= 3 (Q2, F = 22) or c <= 15 (Q4, F = 21) a block's sum of
// c * X is below 2^30 or 64 * 15 * 2^21 < 2^31: the limb sums C0 + 2^8 C1 +
// 2^16 C2 combine exactly in int32 and take one conversion. Fragments built
// inside the matvec keep F = 22 for Q4 and combine the limbs in float.
#define CTOX_XFRAC_BITS 22
#define ctox_staged_xfrac_bits(dtype) ((dtype) ? 21 : 22)

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

// Residual add + RMS norm fused with the activation staging (qmatvec.hip).
struct NormPrepArgs {
    PrepArgs p;             // input unused; columns, batch, dtype, s_in as for the prep
    const float *x;         // [batch][columns]
    const float *delta;     // [delta_parts][batch][columns] partial sums (added in part order) or NULL
    float *x_out;           // x + delta when delta is set (must not alias x)
    uint32_t delta_parts;
    uint32_t delta_stride;  // floats between parts
    const float *w;         // [columns], (1 + w) weight
    float *out;             // normalized rows [batch][columns] or NULL
    float eps;
    uint32_t sq_n;          // sums of squares per row in sq_in (0: reduce the row here)
    const float *sq_in;     // [batch][sq_n]: per 16-column tile, sum of (x + delta)^2
};

// Activation staging of a transformed input (qmatvec.hip, ctox_prep_transform_gfx950).
struct PrepXArgs {
    PrepArgs p;             // input unused
    const float *a;
    const float *b;
    const float *w;
    uint32_t mode;          // 1 swiglu, 2 gated norm, 3 attention gate
    uint32_t a_stride;
    uint32_t b_stride;
    uint32_t off;
    uint32_t head_dim;
    float eps;
    uint32_t a_parts;       // mode 1: a is the sum of this many partials (0/1: one)
    uint32_t a_pstride;     // floats between partials
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
    uint32_t part_stride;   // split K (slice kernels, gridDim.y > 1): workgroup y takes
                            // slice y and writes its partial at output + y * part_stride
    uint32_t pad;
};

// Batch-1 slice kernels (rows of whole 16-byte units): a workgroup of
// CTOX_SLICE_WAVES waves walks a 16-row tile in slices of 28 (Q4) / 56 (Q2)
// blocks, each slice one 1 KiB coalesced load per row.
constexpr uint32_t ctox_slice_blocks(uint32_t dtype) { return dtype ? 28u : 56u; }
// Slices of the small-M (2..8 activation rows) slice kernels.
constexpr uint32_t ctox_slice_blocks_tok(uint32_t dtype) { return dtype ? 28u : 26u; }
#define CTOX_SLICE_WAVES 8

// Tiled weight layout (resident matrices): a unit is 16 rows x 16 blocks.
// Unit (c, t) = column chunk c (blocks 16c..16c+15), row tile t (rows
// 16t..16t+15) sits at byte ((c * tiles) + t) * unit_bytes. Inside a unit:
//   codes: 4 groups G, each Q2: [lane][16 B], Q4: [half][lane][16 B], where
//          lane (g, j) = 16 g + j holds the code bytes (Q4: bytes 16 half ..)
//          of block 16c + 4G + g of row 16t + j;
//   scales (after the codes): [lane][4 x fp16], scale of group G's block.
// Blocks and rows past the matrix are zero (zero scale).
#define CTOX_TILE_ROWS 16
#define CTOX_TILE_BLOCKS 16
constexpr uint32_t ctox_tile_code_bytes(uint32_t dtype) { return dtype ? 8192u : 4096u; }
constexpr uint32_t ctox_tile_unit_bytes(uint32_t dtype) { return ctox_tile_code_bytes(dtype) + 512u; }
// Row tiles one wave of the tiled matvec handles at most.
#define CTOX_TILE_MAXU 4

struct TileRepackArgs {
    const uint8_t *src;     // crate rows, [rows][blocks * block_bytes]
    uint8_t *dst;           // tiled units
    uint32_t rows;
    uint32_t blocks;
    uint32_t tiles;
    uint32_t chunks;
    uint32_t dtype;
    uint32_t pad;
};

// Tiled fused matvec. Wave v of the grid takes chunk c = v / segs and row
// tiles [s * tpw, min(tiles, s * tpw + tpw)) with s = v % segs. With more
// than one chunk the per-chunk row sums go to `partial` ([chunks][tiles *
// 16]) and the wave that brings a tile's arrival count to `chunks` adds them
// in chunk order, applies the epilogue and resets the count to zero.
struct TileMatvecArgs {
    const uint8_t *weights; // tiled units
    const int8_t *xa;       // activation fragments (prep output) or NULL (mode 1)
    const float *xc;        // epilogue constants (prep output)
    const float *input;     // mode 1: f32 activation [columns]
    const void *s_in;       // mode 1: NULL, f32 or f16 [columns]
    const void *s_out;      // NULL, f32[rows] or f16[rows]
    const float *bias;      // NULL or f32[rows]
    float *output;          // [rows]
    uint64_t *partial;      // [chunks - 1][tiles * 16] when chunks > 1: f32 bits | seq << 32
                            // ([chunks][tiles * 16] with arrive)
    uint32_t *arrive;       // batch 1: per row tile, chunks arrived (zero between launches); NULL: the
                            // last chunk combines
    uint32_t seq;           // this launch's tag in the partial slots (never 0)
    uint32_t sq_n;          // xmode 1: entries of sq_in (0: reduce the row itself)
    uint32_t parts_out;     // write each chunk's s_out-scaled sum to output[chunk * out_stride + row]
                            // (batch 1) or output[(chunk * batch + token) * out_stride + row] (small M)
    uint32_t a_parts;       // xmode 2: input holds a_parts partial rows a_pstride floats apart (summed in order)
    uint32_t a_pstride;
    uint32_t pad3;
    const float *res_h;     // res_sq set: the residual the output is added to [rows]
    float *res_sq;          // NULL or [tiles]: sum over the tile's rows of (res_h + out)^2
    const float *sq_in;     // xmode 1: per-tile sums of squares of the residual row, or NULL
    uint32_t rows;
    uint32_t blocks;
    uint32_t tiles;
    uint32_t chunks;
    uint32_t segs;          // waves per chunk
    uint32_t tpw;           // row tiles per wave (<= CTOX_TILE_MAXU)
    uint32_t s_out_kind;
    uint32_t activation;
    uint32_t s_in_kind;
    uint32_t pad;
    // In-kernel fragment build (the _x kernels): the activation is computed
    // from its producer's outputs (`input` is `a` below). xmode:
    //   0 plain:       x = a[c]
    //   1 residual norm (Q/src/reference.rs:38-62): h = a[c] + delta[c] (delta
    //                  may be NULL), x = h * rsqrt(mean(h^2) + eps) * (1 + w[c]);
    //                  h goes to x_out and x to norm_out (each when set) for
    //                  the columns of the chunk, by the workgroup of segment 0
    //   2 swiglu (Q/src/reference.rs:96-112): x = silu(a[c]) * a[off + c]
    //   3 gated norm per head (Q/src/reference.rs:66-93):
    //                  x = a[c] * rsqrt(mean_head(a^2) + eps) * w[c % head_dim] * silu(b[c])
    //   4 attention gate (Q/src/decoder.rs:727-737): x = a[c] * sigmoid(b[h * 2 hd + hd + d])
    // then x * s_in.
    const float *xb;
    const float *xw;
    const float *delta;
    float *x_out;
    float *norm_out;
    uint32_t xmode;
    uint32_t off;
    uint32_t head_dim;
    float eps;
    // Small-M kernels (ctox_q*_mv_tilem*): activation rows (2..8, staged in
    // xa/xc by a prep kernel, or built in the kernel by ctox_q*_mv_tilemx*)
    // and the output row stride.
    uint32_t batch;
    uint32_t out_stride;
    // tilemx: floats between rows of `input` and of xb / delta. Rows of
    // x_out / norm_out are `blocks * 64` apart, sq_in rows sq_n apart, and a
    // producer's res_h / res_sq rows `rows` / `tiles` apart.
    uint32_t a_stride;
    uint32_t b_stride;
    // Small-M producer of a residual delta that also stages the next (1 + w)
    // RMS-normed projection's input (nx_xa set; the last chunk combines, rows
    // a multiple of 64): per token row t and output row r, h = res_h + out goes
    // to nx_h[t][r], h * (1 + nx_w[r]) * nx_s_in[r] (f16 scale, or none) is
    // staged in nx_xa / nx_xc ([block][token], nx_dtype's fragment order)
    // without the row's 1 / rms, and nx_sq[t][block] receives the block's sum
    // of h^2. The consumer, a staged small-M launch with rms_sq set, scales
    // token row t's outputs by 1 / sqrt(sum(rms_sq[t][0 .. rms_n)) / (blocks * 64) + eps).
    const float *rms_sq;
    uint32_t rms_n;
    uint32_t rms_pad;
    int8_t *nx_xa;
    float *nx_xc;
    float *nx_h;
    const float *nx_w;
    const uint16_t *nx_s_in;
    float *nx_sq;
    uint32_t nx_dtype;
    uint32_t nx_pad;
};

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
    uint32_t rep;           // value heads per key head: q, k of head h are key head h / rep
    uint32_t qk_stride;     // floats between tokens of q and of k
    uint32_t v_stride;      // floats between tokens of v
    uint32_t pad;
};

// GatedDeltaNet token mixer core in one launch (gated_delta.hip,
// ctox_gdn_fused_gfx950): causal conv + SiLU of the q, k, v channels of the
// projected rows, the gates, and the recurrence. Projected rows are
// [tokens][proj_stride] holding [q (key_heads*key_dim) | k | v (heads*value_dim)]
// at 0, a at a_off and b at b_off. The conv window goes from conv_in to
// conv_out ([channels][kernel], channels = 2 key_heads key_dim + heads
// value_dim; the buffers must not alias).
struct GdnFusedArgs {
    const float *proj;
    const float *conv_w;     // [channels][kernel]
    const float *conv_in;
    float *conv_out;
    const float *a_log;      // [heads]
    const float *dt_bias;    // [heads]
    float *log_decay;        // [tokens][heads]: written, or read when gates_given
    float *beta;             // [tokens][heads]: likewise
    float *state;            // [heads][key_dim][value_dim] read at the start
    float *out;              // [tokens][heads][value_dim]
    // Where the state goes: state_out (may equal state: every workgroup has
    // read its slice before it writes it). snap_stride != 0: the state after
    // token t is written at state_out + t * snap_stride for every t, and the
    // conv windows after token t at conv_out + t * conv_snap_stride (the
    // speculative verify keeps every row's state; commit picks one).
    float *state_out;
    uint64_t snap_stride;    // floats; 0: only the final state
    uint64_t conv_snap_stride;
    uint32_t tokens;
    uint32_t heads;
    uint32_t key_heads;
    uint32_t key_dim;
    uint32_t value_dim;
    uint32_t kernel;
    uint32_t proj_stride;
    uint32_t a_off;
    uint32_t b_off;
    uint32_t gates_given;
    // 0: state [head][key i][value j] (the crate's layout); 1: the engine's
    // blocked layout, per head and 16-column slice the 256 threads' 8 rows
    // contiguous ([head][slice][ig * 16 + jj][r] for i = ig + 16 r,
    // j = 16 slice + jj; key_dim <= 128), so a wave moves 2 KiB per access.
    uint32_t state_blocked;
    uint32_t pad;
};

// Decode-step glue and token selection (decode_ops.hip).
struct GateArgs {
    const float *a;          // [tokens][heads]
    const float *b;          // [tokens][heads]
    const float *a_log;      // [heads]
    const float *dt_bias;    // [heads]
    float *log_decay;        // [tokens][heads]
    float *beta;             // [tokens][heads]
    uint32_t tokens;
    uint32_t heads;
    uint32_t in_stride;      // floats between tokens of a and of b
    uint32_t pad;
};

struct RepeatArgs {
    const float *in;         // [rows][heads][dim]
    float *out;              // [rows][heads * repeats][dim]
    uint32_t rows;
    uint32_t heads;
    uint32_t dim;
    uint32_t repeats;
};

// Per-(row, part) partial reductions over 2 * drafts + 1 logits rows:
// rows [0, drafts) from `draft`, [drafts, 2 drafts) from `target`, row
// 2 drafts is `bonus`. mode 0: {total-order key, index} of the maximum;
// mode 1: {max(x / T), sum exp(x / T - max)}.
struct PartialArgs {
    const float *draft;      // [drafts][draft_vocab]
    const float *target;
    const float *bonus;
    float *out;              // [rows][parts][2] (mode 0: key and index bit patterns)
    uint32_t drafts;
    uint32_t vocab;
    uint32_t parts;
    uint32_t mode;
    float temperature;
    uint32_t draft_vocab;    // length of a draft row (restricted drafts: the draft vocabulary)
};

// Token-selection decision state shared by the accept kernels.
struct PickState {
    float thr_draw;          // the draw u of the cumulative search
    float m_t, z_t;          // softmax stats of the weight row (target or bonus)
    float m_d, z_d;          // draft row stats (residual mode)
    uint32_t row;            // draft index of the rejection (residual) or drafts (bonus)
    uint32_t accepted;
    uint32_t mode;           // 0 residual max(0, p - q), 1 bonus softmax, 2 invalid token, 3 non-finite logits
};

// Top-k / top-p sampling with a host draw (decode_ops.hip).
#define CTOX_TOPK_PART 4096  // logits per part of the first stage
#define CTOX_TOPK_MAX 256    // largest top_k
#define CTOX_TOPK_CANDS 16384  // candidates the second stage sorts (parts * top_k)
struct TopkArgs {
    const float *logits;     // [vocab]
    uint64_t *cand;          // [parts][top_k] (stage 1 out, stage 2 in): (order key << 32) | token
    uint32_t *flags;         // [parts]: a non-finite logit or scaled logit in the part
    uint32_t *out;           // [4]: token, status, nucleus length, nucleus total (f32 bits)
    uint32_t vocab;
    uint32_t top_k;
    uint32_t parts;
    float inv_temperature;
    float top_p;
    float draw;
};

struct VerifyArgs {
    const float *partials;   // PartialArgs mode 0 output
    uint32_t *out;           // [3 + drafts]: next, verified, accepted count, accepted tokens
    uint32_t drafts;
    uint32_t parts;
    const uint32_t *ids;     // argmax_final: row index -> token map (restricted draft rows), or null
};

struct AcceptArgs {
    const float *draft;      // [drafts][vocab]
    const float *target;     // [drafts][vocab]
    const float *bonus;      // [vocab]
    const uint32_t *tokens;  // [drafts] proposed draft tokens
    const float *partials;   // PartialArgs mode 1 output
    float *sums;             // [parts2] per-part weight sums
    PickState *state;
    uint64_t *rng;           // Pcg32 state, advanced in place
    uint32_t *out;           // [2]: next token, accepted count
    // Restricted drafts (Q/src/engine.rs:151-200): draft rows hold
    // draft_vocab scores; draft_inv[t] is token t's index in them
    // (0xffffffff: outside the draft vocabulary, q = 0). NULL: full rows.
    const uint32_t *draft_inv;
    // Token of each bonus-row index (a restricted row sampled as the bonus
    // row); NULL: the index is the token.
    const uint32_t *bonus_ids;
    uint32_t drafts;
    uint32_t vocab;
    uint32_t parts;          // partials per row
    uint32_t parts2;         // parts of the cumulative search
    float temperature;
    uint32_t draft_vocab;
};

// Layer glue (layer_ops.hip).
struct NormArgs {
    const float *x;          // [rows][cols]
    const float *gate;       // [rows][cols] (mode 1) or NULL
    const float *w;          // [cols]
    float *out;              // [rows][cols]
    uint32_t cols;
    uint32_t mode;           // 0: x * inv * (1 + w); 1: x * inv * w * silu(gate)
    float eps;
    uint32_t pad;
};

struct EltArgs {
    const float *a;
    const float *b;
    float *out;
    uint64_t n;
};

struct ConvArgs {
    const float *input;      // [channels]
    float *state;            // [channels][kernel], updated in place
    const float *weight;     // [channels][kernel]
    float *out;              // [channels]
    uint32_t channels;
    uint32_t kernel;
    uint32_t rows;           // consecutive tokens, applied in order
    uint32_t in_stride;      // floats between tokens of input (out is dense)
};

struct RopeArgs {
    float *q;                // [rows][qh][hd], in place
    float *k;                // [rows][kh][hd], in place
    uint32_t qh;
    uint32_t kh;
    uint32_t hd;
    uint32_t rd;
    uint64_t position;       // position of row 0; row t is at position + t
    float theta;
    uint32_t pad;
};

// Paged KV cache and attention (paged_attention.hip).
struct PagedKvDesc {         // one logical page
    uint32_t precision;      // 0 = Q2 pool, otherwise Q4 pool
    uint32_t physical_slot;  // page index inside its pool
    uint32_t tokens;         // tokens held
    uint32_t first_token;    // logical index of the page's first token
};

struct KvPackArgs {
    uint8_t *q4_pages;
    const float *keys;       // [tokens][component_values]
    const float *values;     // [tokens][component_values]
    uint32_t physical_slot;
    uint32_t first_token_in_page;
    uint32_t component_values;
    uint32_t q4_token_bytes;
    uint64_t q4_page_bytes;
};

// Fused attention-layer prep (ctox_attn_prep_gfx950): per-head q/k RMS norm,
// partial RoPE and the Q4 page append of the new K/V rows.
#define CTOX_ATTN_PREP_ROWS 8
#define CTOX_ATTN_PREP_DESC_WORDS 32
struct AttnPrepArgs {
    const float *proj;       // [rows][proj_stride]: per q head [q, gate] (2 hd), then k [kh hd], v [kh hd]
    const float *q_norm;     // [hd]
    const float *k_norm;     // [hd]
    float *q_out;            // [rows][qh][hd]
    uint8_t *q4_pages;
    uint64_t q4_page_bytes;
    uint64_t position;       // rope position of row 0
    uint32_t proj_stride;
    uint32_t qh;
    uint32_t kh;
    uint32_t hd;             // 256
    uint32_t rd;             // rotary dims (even, <= hd)
    uint32_t q4_token_bytes;
    float eps;
    float theta;
    uint32_t slot[CTOX_ATTN_PREP_ROWS];  // Q4 page slot of row t
    uint32_t pos[CTOX_ATTN_PREP_ROWS];   // token index of row t inside that page
    uint32_t *desc_dst;                  // page descriptor words to store (NULL: none)
    uint32_t desc_words;                 // <= CTOX_ATTN_PREP_DESC_WORDS
    uint32_t desc[CTOX_ATTN_PREP_DESC_WORDS];
};

struct KvDemoteArgs {
    const uint8_t *q4_page;
    uint8_t *q2_page;
    uint64_t blocks;         // tokens * blocks per token
};

struct GqaArgs {
    const float *query;      // [rows][query_heads][256]
    const uint8_t *q2;
    const uint8_t *q4;
    const PagedKvDesc *desc; // [page_count]
    float *part_out;         // [kv heads][splits][queries][256]
    float *part_stats;       // [kv heads][splits][queries][2] = (max, denominator)
    float *out;              // [rows][query_heads][256]
    uint64_t q2_page_bytes;
    uint64_t q4_page_bytes;
    uint32_t query_heads;
    uint32_t group;          // query heads per kv head
    uint32_t tokens;         // cached tokens, the query rows included
    uint32_t rows;           // query rows (the last `rows` cached tokens)
    uint32_t queries;        // group * rows
    uint32_t page_tokens;
    uint32_t page_count;
    uint32_t component_values;
    uint32_t q2_token_bytes;
    uint32_t q4_token_bytes;
    uint32_t tiles;          // ceil(tokens / 16)
    uint32_t tiles_per_wave;
    uint32_t splits;
    float scale;
    uint32_t tile_pages;     // 1 when page_tokens % 16 == 0: a 16-token tile lies in one page
    uint32_t st_dtype;       // staging below: 0 = Q2, 1 = Q4 fragment order of the o projection
    // Optional (st_xa set): the combine also stages the o projection's input
    // x[t][c] = out[t][c] * sigmoid(gate[t * st_gate_stride + head * 512 + 256 + d])
    // (Q/src/decoder.rs:727-737), times st_s_in[c] (f16, or none), for
    // column c = head * 256 + d, as the prep kernel would: 64-column block b
    // of row t at st_xa + (b * rows + t) * 192, its constants at st_xc.
    int8_t *st_xa;
    float *st_xc;
    const float *st_gate;
    const uint16_t *st_s_in;
    uint32_t st_gate_stride;
    uint32_t st_pad;
};

// Decode engine helpers (engine_ops.hip).
struct FillArgs {
    void *ptr;
    uint64_t count;          // elements (kinds 2..4) or blocks (kinds 0, 1) of this launch
    uint64_t index_base;     // global index of element 0 (keeps chunked fills reproducible)
    uint64_t seed;
    uint32_t kind;           // 0 Q4 blocks, 1 Q2 blocks, 2 f32 normal, 3 f16 uniform, 4 f32 uniform
    float p0;                // mean (2) or low bound (3, 4)
    float p1;                // std (2), high bound (3, 4), scale sigma (0, 1)
    uint32_t pad;
};

struct EmbedArgs {
    const uint8_t *weights;  // [vocab][cols / 64] blocks
    const uint16_t *s_in;    // [cols] fp16 or NULL
    const uint16_t *s_out;   // [vocab] fp16 or NULL
    const uint32_t *tokens;  // [rows] on the device
    float *out;              // [rows][cols]
    uint32_t cols;
    uint32_t vocab;
    uint32_t dtype;          // 0 Q2, 1 Q4
    uint32_t pad;
};

struct NormRowsArgs {
    float *x;                // rows at (r / inner) * x_outer + (r % inner) * x_inner
    const float *delta;      // [rows][cols] added to x first (x updated) or NULL
    const float *gate;       // mode 1, same two-level addressing with g_*
    const float *w;          // [cols]
    float *out;              // rows at r * out_stride
    uint32_t cols;
    uint32_t mode;           // 0: (1 + w); 1: w * silu(gate)
    float eps;
    uint32_t inner;
    uint64_t x_inner, x_outer, g_inner, g_outer, out_stride;
    uint32_t delta_parts;    // partial sums in delta (>= 1)
    uint32_t delta_stride;   // floats between parts
};

struct AttnGateArgs {
    float *values;           // [rows][heads][head_dim]
    const float *qg;         // token rows of q_proj output: per head [q (head_dim), gate (head_dim)]
    uint32_t rows;
    uint32_t heads;
    uint32_t head_dim;
    uint32_t qg_stride;      // floats between tokens of qg
};

struct RowsArgs {
    const float *in;
    float *out;
    uint32_t rows;
    uint32_t cols;
    uint32_t in_stride;
    uint32_t out_stride;
    uint32_t offset;         // swiglu: offset of up within an input row; copy: offset of the copied columns
    uint32_t pad;
};

struct FiniteArgs {          // ctox_finite_check_gfx950
    const float *x;
    uint32_t *flags;         // [gridDim.x]: 1 if a value of the workgroup's range is not finite, else 0
    uint64_t n;
};

struct FlagStatusArgs {      // ctox_greedy_status_gfx950
    const uint32_t *flags;   // ctox_finite_check_gfx950 output
    uint32_t *out;           // the sampler's d_out: [1] status, [2] nucleus length, [3] total
    uint32_t parts;
};

struct StreamReadArgs {      // ctox_stream_read_gfx950
    const uint8_t *src;
    uint32_t *out;           // [ceil(bytes / 8 KiB)]: xor of each wave's 8 KiB
    uint64_t bytes;          // multiple of 16
};

struct GatherRowsArgs {      // ctox_gather_rows_gfx950: dst row r = src row ids[r] (bytes)
    const uint8_t *src;
    uint8_t *dst;
    const uint32_t *ids;
    uint64_t row_bytes;
    uint32_t rows;
    uint32_t pad;
};

// Several small host-to-device writes in one launch (the engine's descriptor
// uploads after a step): segment i writes words[off[i] .. off[i + 1]) to dst[i].
#define CTOX_SEG_MAX 24
#define CTOX_SEG_WORDS 512
struct SegWordsArgs {
    uint32_t *dst[CTOX_SEG_MAX];
    uint32_t off[CTOX_SEG_MAX + 1];
    uint32_t nseg;
    uint32_t pad;
    uint32_t words[CTOX_SEG_WORDS];
};

struct WordsArgs {           // small host-to-device writes carried in the kernel arguments
    uint32_t *dst;
    uint32_t count;          // <= 32
    uint32_t pad;
    uint32_t words[32];
};
