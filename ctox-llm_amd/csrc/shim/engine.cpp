// Device-resident Qwen3.8 decode engine over the ctox_hip C ABI.
//
// The crate's model graph (Q/src/decoder.rs) composed from the HIP entry
// points: every tensor and state lives in HBM, one process drives one GPU,
// and a step is a sequence of launches on one stream with a single
// device-to-host read (the speculative result) per MTP step.
//
//  * Target step over R rows (R = 1 decode, R = k + 1 MTP verification):
//    embedding (decoder.rs:531-537), per layer a GatedDeltaNet
//    (decoder.rs:806-938) or full-attention (:687-800) token mixer, the MLP
//    (:636-670), the final norm and the LM head (:940-951). Residual adds are
//    folded into the next RMS norm; projections that share an input are one
//    row-concatenated matrix (qkv|z|a|b, q|k|v, gate|up), which computes the
//    same rows as the crate's fan-out (cpu.rs:444-472) because rows are
//    independent and their s_in is shared.
//  * MTP draft (decoder.rs:1009-1046): embed, the two pre-fc norms, fc over
//    [embedding, hidden], one full-attention layer with its own paged cache,
//    the MLP, the MTP norm, the shared LM head; the token is sampled at the
//    requested temperature from the crate's Pcg32 stream.
//  * Speculative step: k chained drafts (each fed the previous draft's MTP
//    hidden), one batched target pass over [t0, d1..dk], rejection-sampling
//    acceptance (ctox_hip_mtp_accept_device), then commit: GatedDeltaNet and
//    conv states are restored from a checkpoint and replayed over the
//    committed tokens, paged caches are truncated, and the MTP cache is
//    replayed with target hiddens as commit_speculative does
//    (decoder.rs:1397-1458).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <cstdlib>
#include <vector>

#include "ctox_hip.h"
#include "shim_internal.h"

void ctox_set_last_error(const char *msg);  // ctox_hip.cpp

namespace {

struct Mat {
    int32_t dtype = CTOX_DTYPE_Q4B64;
    uint32_t rows = 0, cols = 0;
    uint8_t *w = nullptr;
    uint16_t *s_in = nullptr, *s_out = nullptr;
    size_t bytes() const { return (size_t)rows * (cols / 64) * (dtype == CTOX_DTYPE_Q4B64 ? 34 : 18); }
};

struct Mlp {
    float *norm = nullptr;  // post_attention_layernorm
    Mat gate_up, down;
};

struct GdnLayer {
    float *norm = nullptr;  // input_layernorm
    Mat in;                 // [qkv | z | a | b]
    float *conv_w = nullptr, *a_log = nullptr, *dt_bias = nullptr, *gnorm = nullptr;
    Mat out;
    size_t state_off = 0;    // offset of the layer's state in each state slot
    size_t conv_off = 0;     // offset of the layer's conv windows in each conv slot
};

// Host bookkeeping of one paged cache (Q/src/kv_cache.rs:303-478 policy).
struct Cache {
    uint8_t *q4 = nullptr, *q2 = nullptr;
    ctox_paged_kv_descriptor *d_desc = nullptr;
    std::vector<ctox_paged_kv_descriptor> desc;
    std::vector<uint32_t> free_q4, free_q2;
    uint32_t pages = 0, tokens = 0;
    uint32_t dirty = 0;  // lowest page whose descriptor changed since the last upload
    // Pages before `scan` are demoted or in the sink: demotion resumes there.
    // Truncation only removes rows after the last commit, which lie in pages
    // at or after it, so the cursor never passes a page that changes again.
    uint32_t scan = 0;
};

struct AttnLayer {
    float *norm = nullptr;
    Mat qkv;                // [q|gate per head, k, v]
    float *q_norm = nullptr, *k_norm = nullptr;
    Mat o;
    Cache cache;
};

struct Layer {
    bool full = false;
    GdnLayer g;
    AttnLayer f;
    Mlp mlp;
};

}  // namespace

struct ctox_hip_engine {
    ctox_hip_backend *b = nullptr;
    ctox_engine_config c{};
    hipStream_t s = nullptr;
    std::vector<void *> allocs;
    struct Tiled {
        const void *w;
        int32_t dtype;
        uint32_t rows, cols;
    };
    std::vector<Tiled> tiled;  // weights with a registered tiled copy
    bool loading = false;      // tensors written since the last finish_load
    std::vector<Layer> layers;
    Mat embed, lm_head;
    float *final_norm = nullptr;
    // Restricted MTP draft head (Q/src/decoder.rs:589-627): the LM-head rows
    // of the release-bound draft vocabulary, gathered once into a compact
    // matrix (s_in shared with the LM head); draft_inv maps a token to its
    // row (0xffffffff outside). draft_n = 0: drafts use the full head.
    Mat draft_head;
    uint32_t draft_n = 0;
    uint32_t *d_draft_ids = nullptr, *d_draft_inv = nullptr;
    // Fail-closed flags: non-finite logits (device words, read back through
    // pinned host memory with the step's one synchronization).
    uint32_t *d_flags = nullptr;
    // Host copy of the step result / flags. Ordinary (pageable) memory: the
    // runtime then copies these few words with a blit kernel on the stream,
    // which measured faster per step than a copy into pinned memory.
    uint32_t h_res[256] = {};
    // MTP
    bool mtp = false;
    float *mtp_norm_emb = nullptr, *mtp_norm_hid = nullptr, *mtp_norm = nullptr;
    Mat mtp_fc;
    AttnLayer mtp_attn;
    Mlp mtp_mlp;
    // geometry
    uint32_t H = 0, I = 0, Kw = 0, Vw = 0, C = 0, Rin = 0, Rq = 0, kvw = 0, V = 0, R = 0;
    uint32_t q4_token_bytes = 0, q2_token_bytes = 0, q4_page_bytes = 0, q2_page_bytes = 0;
    // Recurrent state and conv windows of every GatedDeltaNet layer, in two
    // banks of R slots each (one slot = all layers). The current state is
    // slot `sidx` of bank `bank`; a target pass over R rows reads it and
    // writes the state after each row t into slot t of the other bank, so a
    // speculative commit of n + 1 rows only selects slot n (no checkpoint
    // copy, no replay), and the conv windows are never updated in place.
    float *gdn_bank = nullptr, *conv_bank = nullptr;
    uint32_t bank = 0, sidx = 0;
    size_t gdn_floats = 0, conv_floats = 0;
    // activations (sized for R rows)
    float *hid = nullptr, *hid2 = nullptr, *proj = nullptr, *convo = nullptr, *core = nullptr, *coren = nullptr,
          *delta = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr, *gu = nullptr, *act = nullptr,
          *fin = nullptr, *logits = nullptr, *ld = nullptr, *beta = nullptr, *fcin = nullptr;
    float *draft_logits = nullptr, *mtp_hidden = nullptr, *prev_hidden = nullptr;
    // d_drafts = d_result + 16: the acceptance result and the step's tokens
    // come back to the host in one read.
    uint32_t *d_tokens = nullptr, *d_drafts = nullptr, *d_result = nullptr;
    uint64_t *d_rng = nullptr;
    uint32_t delta_parts = 1;  // partial sums held in delta (split-K producers)
    // Per-16-row sums of (hid + delta)^2 written by the last single-row
    // producer of `rsq_delta` against residual `rsq_hid` (the next norm's
    // sum of squares); valid until that norm consumes them.
    float *rsq = nullptr;
    const float *rsq_delta = nullptr, *rsq_hid = nullptr;
    // Next-norm staging on the small-M verify path: a residual producer
    // (delta_mv) told which norm-matvec follows it (nx_w, nx_m) stages that
    // projection's input itself; pre_* records the staging until the
    // matching norm_mv consumes it. blk_sq: its per-64-column sums of h^2.
    const float *nx_w = nullptr;
    const struct Mat *nx_m = nullptr;
    const float *pre_w = nullptr, *pre_delta = nullptr;
    const struct Mat *pre_m = nullptr;
    uint32_t pre_rows = 0;
    float *blk_sq = nullptr;
    bool next_norm = true;  // CTOX_NEXT_NORM=0 turns the next-norm staging off
    // Matrix dtypes by engine name (ctox_hip_engine_create_with_dtypes); the
    // default plan is Q4 projections and Q2 down projections.
    std::unordered_map<std::string, int32_t> dtype_plan;
    uint32_t position = 0;   // tokens processed by the target model
    uint32_t mtp_tokens = 0; // entries in the MTP cache
    bool have_prev = false;  // prev_hidden holds the last target final hidden
};

namespace {

ctox_status efail(ctox_status st, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    ctox_set_last_error(buf);
    return st;
}

#define TRY(x)                                  \
    do {                                        \
        ctox_status st_ = (x);                  \
        if (st_ != CTOX_OK) return st_;         \
    } while (0)

ctox_status dalloc(ctox_hip_engine *e, void **p, size_t bytes) {
    if (bytes == 0) bytes = 256;
    if (hipMalloc(p, bytes) != hipSuccess) return efail(CTOX_ERR_MEMORY_BUDGET, "device allocation of %zu bytes failed", bytes);
    e->allocs.push_back(*p);
    return CTOX_OK;
}

template <typename T>
ctox_status dalloc_t(ctox_hip_engine *e, T **p, size_t count) {
    return dalloc(e, (void **)p, count * sizeof(T));
}

ctox_status fill(ctox_hip_engine *e, void *p, uint64_t n, uint32_t kind, uint64_t seed, float p0, float p1) {
    return ctox_hip_fill_random_device(e->b, p, n, kind, seed, p0, p1, e->s);
}

// A quantized matrix with fp16 s_in / s_out in U(0.75, 1.25) and block scales |N(0, 0.02)|.
ctox_status make_mat(ctox_hip_engine *e, const std::string &name, Mat &m, int32_t dtype, uint32_t rows, uint32_t cols,
                     uint64_t &seed, uint16_t *shared_s_in = nullptr, bool projection = true) {
    auto planned = e->dtype_plan.find(name);
    if (planned != e->dtype_plan.end()) dtype = planned->second;
    m.dtype = dtype;
    m.rows = rows;
    m.cols = cols;
    TRY(dalloc(e, (void **)&m.w, m.bytes()));
    TRY(fill(e, m.w, (uint64_t)rows * (cols / 64), dtype == CTOX_DTYPE_Q4B64 ? 0 : 1, seed++, 0.0f, 0.02f));
    if (shared_s_in) {
        m.s_in = shared_s_in;
    } else {
        TRY(dalloc_t(e, &m.s_in, cols));
        TRY(fill(e, m.s_in, cols, 3, seed++, 0.75f, 1.25f));
    }
    TRY(dalloc_t(e, &m.s_out, rows));
    TRY(fill(e, m.s_out, rows, 3, seed++, 0.75f, 1.25f));
    if (projection) {
        // Batch-1 projections stream the tiled copy; the crate-layout rows stay
        // for the small-M verify kernels.
        TRY(ctox_hip_register_tiled_weights(e->b, dtype, m.w, rows, cols, e->s));
        e->tiled.push_back({m.w, dtype, rows, cols});
    }
    return CTOX_OK;
}

ctox_status make_vec(ctox_hip_engine *e, float **p, size_t n, uint64_t &seed, float mean, float std) {
    TRY(dalloc_t(e, p, n));
    return fill(e, *p, n, 2, seed++, mean, std);
}

ctox_status matvec(ctox_hip_engine *e, const Mat &m, const float *in, float *out, uint32_t rows) {
    return ctox_hip_launch_fused_matvec(e->b, m.dtype, m.w, in, m.s_in, m.s_out, nullptr, out, m.rows, m.cols, 0, rows,
                                        e->s);
}

// Rows whose residual producers hand the next norm its per-tile sums of
// squares (the projections build up to 5 rows in the kernel).
constexpr uint32_t kSumRows = 5;

// x += delta (when set), (1 + w) RMS norm, then the projection m of the
// normalized rows into out; the normalized rows also go to norm_out if set.
// The residual stream ping-pongs between e->hid and e->hid2: with a delta the
// sum goes to the other buffer, which becomes the stream.
ctox_status norm_mv(ctox_hip_engine *e, const float *delta, const float *w, uint32_t rows, const Mat &m, float *out,
                    float *norm_out = nullptr, uint32_t max_parts = 1, uint32_t *parts = nullptr) {
    const bool pre = e->pre_m == &m && e->pre_w == w && e->pre_delta == delta && delta && e->pre_rows == rows &&
                     !norm_out && e->rsq_hid == e->hid;
    e->pre_m = nullptr;
    if (pre) {
        // The producer already wrote hid + delta to hid2 and staged the
        // normed rows; this launch applies each row's 1 / rms.
        e->rsq_delta = e->rsq_hid = nullptr;
        TRY(ctox_norm_matvec_prestaged(e->b, m.dtype, m.w, m.s_out, out, m.rows, m.cols, rows, e->blk_sq,
                                       e->c.rms_norm_epsilon, max_parts, parts, e->s));
        std::swap(e->hid, e->hid2);
        return CTOX_OK;
    }
    const bool sums = delta && rows <= kSumRows && e->rsq_delta == delta && e->rsq_hid == e->hid && e->delta_parts == 1;
    e->rsq_delta = e->rsq_hid = nullptr;
    TRY(ctox_hip_norm_matvec_parts_device(e->b, e->hid, delta, e->delta_parts, (size_t)rows * e->H, delta ? e->hid2 : nullptr,
                                    w, e->c.rms_norm_epsilon, norm_out, m.dtype, m.w, m.s_in, m.s_out, out, m.rows,
                                    m.cols, rows, sums ? e->rsq : nullptr, sums ? (e->H + 15) / 16 : 0, max_parts, parts, e->s));
    if (delta) std::swap(e->hid, e->hid2);
    return CTOX_OK;
}

// A single-row producer of residual delta `out` also leaves the next norm's
// per-tile sums of squares (ctox_input_transform::res_sums).
// input_staged: x's staging was already written (the attention combine's),
// only with a next norm-matvec in view (the stage-next path).
ctox_status delta_mv(ctox_hip_engine *e, ctox_input_transform &x, const Mat &m, float *out, uint32_t R,
                     bool input_staged = false) {
    const float *nx_w = e->nx_w;
    const Mat *nx_m = e->nx_m;
    e->nx_w = nullptr;
    e->nx_m = nullptr;
    e->pre_m = nullptr;
    if (R <= kSumRows) {
        x.res_h = e->hid;
        x.res_sums = e->rsq;
    }
    e->rsq_delta = e->rsq_hid = nullptr;
    bool staged = false;
    if (nx_m && R >= 2 && R <= kSumRows && e->next_norm) {
        TRY(ctox_delta_matvec_stage_next(e->b, &x, m.dtype, m.w, m.s_in, m.s_out, out, m.rows, m.cols, R, nx_w,
                                         nx_m->s_in, nx_m->dtype, e->hid2, e->blk_sq, &staged, e->s, input_staged));
        e->delta_parts = 1;
        if (staged) {
            e->pre_w = nx_w;
            e->pre_m = nx_m;
            e->pre_delta = out;
            e->pre_rows = R;
        }
    } else {
        TRY(ctox_hip_transform_matvec_device(e->b, &x, m.dtype, m.w, m.s_in, m.s_out, out, m.rows, m.cols, R, 1,
                                             &e->delta_parts, e->s));
    }
    if (R <= kSumRows) {
        e->rsq_delta = out;
        e->rsq_hid = e->hid;
    }
    return CTOX_OK;
}

// Norm of `rows` dense rows of width cols; x += delta first when delta is set.
ctox_status norm(ctox_hip_engine *e, float *x, const float *delta, const float *w, uint32_t rows, uint32_t cols,
                 float *out, size_t out_stride) {
    ctox_norm_rows d{};
    d.x = x;
    d.delta = delta;
    d.w = w;
    d.out = out;
    d.rows = rows;
    d.cols = cols;
    d.mode = 0;
    d.inner = rows;
    d.eps = e->c.rms_norm_epsilon;
    d.x_inner = cols;
    d.x_outer = 0;
    d.out_stride = out_stride;
    d.delta_parts = delta ? e->delta_parts : 0;
    d.delta_stride = (uint64_t)rows * cols;
    return ctox_hip_norm_rows_device(e->b, &d, e->s);
}

// ---- paged cache bookkeeping ----
ctox_status cache_init(ctox_hip_engine *e, Cache &c) {
    const uint32_t pages = (e->c.max_tokens + e->c.page_tokens - 1) / e->c.page_tokens;
    const uint32_t q4_slots =
        std::min(pages, e->c.sink_tokens / e->c.page_tokens + (e->c.recent_tokens + e->c.page_tokens - 1) / e->c.page_tokens +
                            2 + (e->R + e->c.page_tokens - 1) / e->c.page_tokens);
    TRY(dalloc(e, (void **)&c.q4, (size_t)q4_slots * e->q4_page_bytes));
    TRY(dalloc(e, (void **)&c.q2, (size_t)pages * e->q2_page_bytes));
    TRY(dalloc_t(e, &c.d_desc, pages));
    c.desc.assign(pages, ctox_paged_kv_descriptor{0, 0, 0, 0});
    for (uint32_t i = q4_slots; i-- > 0;) c.free_q4.push_back(i);
    for (uint32_t i = pages; i-- > 0;) c.free_q2.push_back(i);
    return CTOX_OK;
}

// Descriptors [dirty, pages) to the device, in stream order (kernel-argument writes).
ctox_status cache_upload(ctox_hip_engine *e, Cache &c) {
    if (c.dirty < c.pages)
        TRY(ctox_hip_write_words_device(e->b, (uint32_t *)(c.d_desc + c.dirty), (const uint32_t *)(c.desc.data() + c.dirty),
                                        (size_t)(c.pages - c.dirty) * 4, e->s));
    c.dirty = c.pages;
    return CTOX_OK;
}

// Reserve Q4 page slots for `rows` new tokens: row t goes to slot slots[t] at
// token index pos[t] of that page (descriptors updated, device copy dirty).
ctox_status cache_reserve(ctox_hip_engine *e, Cache &c, uint32_t rows, uint32_t *slots, uint32_t *pos) {
    if (c.tokens + rows > e->c.max_tokens) return efail(CTOX_ERR_MEMORY_BUDGET, "paged KV cache is full");
    for (uint32_t t = 0; t < rows; t++) {
        if (c.pages == 0 || c.desc[c.pages - 1].tokens == e->c.page_tokens) {
            if (c.free_q4.empty()) return efail(CTOX_ERR_MEMORY_BUDGET, "no free Q4 page slot");
            c.desc[c.pages] = ctox_paged_kv_descriptor{1, c.free_q4.back(), 0, c.pages * e->c.page_tokens};
            c.free_q4.pop_back();
            c.pages++;
        }
        ctox_paged_kv_descriptor &d = c.desc[c.pages - 1];
        c.dirty = std::min(c.dirty, c.pages - 1);
        slots[t] = d.physical_slot;
        pos[t] = d.tokens;
        d.tokens++;
        c.tokens++;
    }
    return CTOX_OK;
}

// Append `rows` tokens (k, v: [rows][cv] dense) into Q4 pages, one pack per page run.
ctox_status cache_push(ctox_hip_engine *e, Cache &c, const float *k, const float *v, uint32_t rows) {
    std::vector<uint32_t> slots(rows), pos(rows);
    TRY(cache_reserve(e, c, rows, slots.data(), pos.data()));
    for (uint32_t t = 0; t < rows;) {
        uint32_t n = 1;
        while (t + n < rows && slots[t + n] == slots[t] && pos[t + n] == pos[t] + n) n++;
        TRY(ctox_hip_kv_pack_q4_device(e->b, c.q4, k + (size_t)t * e->kvw, v + (size_t)t * e->kvw, n, e->kvw, slots[t],
                                       pos[t], e->q4_page_bytes, e->s));
        t += n;
    }
    return CTOX_OK;
}

// Drop the last `n` tokens (speculative rollback; pages emptied go back to the pool).
void cache_truncate(Cache &c, uint32_t n) {
    while (n > 0 && c.pages > 0) {
        ctox_paged_kv_descriptor &d = c.desc[c.pages - 1];
        c.dirty = std::min(c.dirty, c.pages - 1);
        const uint32_t drop = std::min(n, d.tokens);
        d.tokens -= drop;
        c.tokens -= drop;
        n -= drop;
        if (d.tokens == 0) {
            (d.precision ? c.free_q4 : c.free_q2).push_back(d.physical_slot);
            c.pages--;
        }
    }
}

// Q/src/kv_cache.rs:463-478: pages past the sink and wholly older than the recent window become Q2.
ctox_status cache_demote(ctox_hip_engine *e, Cache &c) {
    const uint32_t recent_start = c.tokens > e->c.recent_tokens ? c.tokens - e->c.recent_tokens : 0;
    // Pages are in token order: the first one not wholly older than the
    // recent window ends the scan (host work per step independent of the context).
    for (uint32_t i = c.scan; i < c.pages; i++) {
        ctox_paged_kv_descriptor &d = c.desc[i];
        if (d.first_token + d.tokens > recent_start) break;
        c.scan = i + 1;
        if (d.precision && d.first_token >= e->c.sink_tokens) {
            if (c.free_q2.empty()) return efail(CTOX_ERR_MEMORY_BUDGET, "no free Q2 page slot");
            const uint32_t q2 = c.free_q2.back();
            c.free_q2.pop_back();
            TRY(ctox_hip_kv_demote_device(e->b, c.q4 + (size_t)d.physical_slot * e->q4_page_bytes,
                                          c.q2 + (size_t)q2 * e->q2_page_bytes, d.tokens, 2 * e->kvw / 64, e->s));
            c.free_q4.push_back(d.physical_slot);
            d.precision = 0;
            d.physical_slot = q2;
            c.dirty = std::min(c.dirty, i);
        }
    }
    return CTOX_OK;
}

ctox_paged_gqa_params gqa_params(ctox_hip_engine *e, const Cache &c) {
    ctox_paged_gqa_params p{};
    p.query_heads = e->c.num_attention_heads;
    p.key_value_heads = e->c.num_key_value_heads;
    p.head_dim = e->c.head_dim;
    p.tokens = c.tokens;
    p.page_tokens = e->c.page_tokens;
    p.page_count = std::max(1u, c.pages);
    p.combined_values = 2 * e->kvw;
    p.q2_token_bytes = e->q2_token_bytes;
    p.q4_token_bytes = e->q4_token_bytes;
    p.q2_page_bytes = e->q2_page_bytes;
    p.q4_page_bytes = e->q4_page_bytes;
    p.scale = 1.0f / std::sqrt((float)e->c.head_dim);
    return p;
}

// ---- layers ----
ctox_status make_attn(ctox_hip_engine *e, const std::string &prefix, AttnLayer &a, uint64_t &seed) {
    const uint32_t H = e->H, qh = e->c.num_attention_heads, hd = e->c.head_dim;
    TRY(make_vec(e, &a.norm, H, seed, 0.0f, 0.1f));
    TRY(make_mat(e, prefix + ".qkv", a.qkv, CTOX_DTYPE_Q4B64, e->Rq, H, seed));
    TRY(make_vec(e, &a.q_norm, hd, seed, 0.0f, 0.1f));
    TRY(make_vec(e, &a.k_norm, hd, seed, 0.0f, 0.1f));
    TRY(make_mat(e, prefix + ".o", a.o, CTOX_DTYPE_Q4B64, H, qh * hd, seed));
    return cache_init(e, a.cache);
}

ctox_status make_mlp(ctox_hip_engine *e, const std::string &prefix, Mlp &m, uint64_t &seed) {
    TRY(make_vec(e, &m.norm, e->H, seed, 0.0f, 0.1f));
    TRY(make_mat(e, prefix + ".gate_up", m.gate_up, CTOX_DTYPE_Q4B64, 2 * e->I, e->H, seed));
    return make_mat(e, prefix + ".down", m.down, CTOX_DTYPE_Q2B64, e->H, e->I, seed);
}

// Full-attention token mixer over R rows at rope positions rope0.. (the
// cache's last R tokens after the push); writes the residual delta. Unless
// `retain` (a speculative branch, kv_cache.rs:372-381), pages are demoted
// right after the push, before attention reads them, as
// FullAttentionState::append does (decoder.rs:774).
ctox_status attn_forward(ctox_hip_engine *e, AttnLayer &a, uint32_t R, uint32_t rope0, float *delta, bool retain) {
    const uint32_t qh = e->c.num_attention_heads, kvh = e->c.num_key_value_heads, hd = e->c.head_dim;
    // the q|k|v projection is already in e->proj (norm_mv): q/k norms, RoPE
    // and the K/V append in one launch
    uint32_t slots[8], pos[8];
    if (R > 8) return efail(CTOX_ERR_SHAPE, "attention rows exceed 8");
    TRY(cache_reserve(e, a.cache, R, slots, pos));
    Cache &c = a.cache;
    // The reserved pages' descriptors travel with the append's launch.
    const size_t words = (size_t)(c.pages - std::min(c.dirty, c.pages)) * 4;
    const bool carry = words > 0 && words <= 32;
    if (!carry) TRY(cache_upload(e, c));
    TRY(ctox_hip_attn_prep_device(e->b, e->proj, e->Rq, a.q_norm, a.k_norm, R, qh, kvh, hd, e->c.rotary_dim, rope0,
                                  e->c.rope_theta, e->c.rms_norm_epsilon, c.q4, e->q4_page_bytes, slots, pos, e->q,
                                  carry ? (uint32_t *)(c.d_desc + c.dirty) : nullptr,
                                  carry ? (const uint32_t *)(c.desc.data() + c.dirty) : nullptr, carry ? words : 0,
                                  e->s));
    if (carry) c.dirty = c.pages;
    // Pages are demoted after the rows are appended, before attention reads
    // them, as FullAttentionState::append pushes and then demotes
    // (Q/src/kv_cache.rs:394-429, 463-478; decoder.rs:774): with a recent
    // window shorter than the rows appended, a page holding new rows may go.
    if (!retain) {
        TRY(cache_demote(e, c));
        TRY(cache_upload(e, c));
    }
    const ctox_paged_gqa_params p = gqa_params(e, a.cache);
    // On the verify path the combine also stages o_proj's gated input (no
    // staging launch); o_proj then runs as a next-norm producer.
    const bool stage_o = e->next_norm && e->nx_m && R >= 2 && R <= kSumRows &&
                         ctox_small_m_staged(e->b, a.o.w, R, a.o.rows, a.o.cols);
    if (stage_o)
        TRY(ctox_paged_gqa_stage_o_device(e->b, e->q, a.cache.q2, a.cache.q4, a.cache.d_desc, &p, R, e->attn, e->proj,
                                          e->Rq, a.o.s_in, a.o.dtype, e->s));
    else
        TRY(ctox_hip_paged_gqa_device(e->b, e->q, a.cache.q2, a.cache.q4, a.cache.d_desc, &p, R, e->attn, e->s));
    ctox_input_transform x{e->attn, e->proj, nullptr, 3, qh * hd, e->Rq, 0, hd, 0.0f, nullptr, nullptr, 0, 0};
    return delta_mv(e, x, a.o, delta, R, stage_o);
}

float *state_cur(ctox_hip_engine *e) { return e->gdn_bank + ((size_t)e->bank * e->R + e->sidx) * e->gdn_floats; }
float *conv_cur(ctox_hip_engine *e) { return e->conv_bank + ((size_t)e->bank * e->R + e->sidx) * e->conv_floats; }

// Causal conv, gates and recurrence of one GatedDeltaNet layer over R
// projected rows (one launch): reads the current state slot and writes the
// state after row t into slot t of the other bank.
ctox_status gdn_core(ctox_hip_engine *e, GdnLayer &g, const float *proj, uint32_t R) {
    const uint32_t Hv = e->c.linear_num_value_heads, Hk = e->c.linear_num_key_heads;
    const size_t other = (size_t)(e->bank ^ 1u) * e->R;
    return ctox_hip_gdn_fused_snap_device(e->b, proj, e->Rin, e->C + e->Vw, e->C + e->Vw + Hv, g.conv_w,
                                          conv_cur(e) + g.conv_off, e->conv_bank + other * e->conv_floats + g.conv_off,
                                          e->conv_floats, e->c.linear_conv_kernel_dim, g.a_log, g.dt_bias, e->ld,
                                          e->beta, state_cur(e) + g.state_off,
                                          e->gdn_bank + other * e->gdn_floats + g.state_off, e->gdn_floats, 1, R, Hv, Hk,
                                          e->c.linear_key_head_dim, e->c.linear_value_head_dim, e->core, e->s);
}

ctox_status gdn_forward(ctox_hip_engine *e, GdnLayer &g, uint32_t R, float *delta) {
    const uint32_t dv = e->c.linear_value_head_dim;
    TRY(gdn_core(e, g, e->proj, R));  // the in-projection is already in e->proj (norm_mv)
    ctox_input_transform x{e->core, e->proj + e->C, g.gnorm, 2, e->Vw, e->Rin, 0, dv, e->c.rms_norm_epsilon, nullptr, nullptr, 0, 0};
    return delta_mv(e, x, g.out, delta, R);
}

// nx_w / nx_m: the norm-matvec that follows the MLP (the next layer's
// in-projection), whose input down may stage.
ctox_status mlp_forward(ctox_hip_engine *e, Mlp &m, uint32_t R, const float *delta_in, float *delta_out,
                        const float *nx_w = nullptr, const Mat *nx_m = nullptr) {
    // gate|up leaves its chunk partials and down's SwiGLU build or staging adds them.
    uint32_t parts = 1;
    TRY(norm_mv(e, delta_in, m.norm, R, m.gate_up, e->gu, nullptr, 6, &parts));
    ctox_input_transform x{e->gu, nullptr, nullptr, 1, 2 * e->I, 0, e->I, 0, 0.0f, nullptr, nullptr, parts, R * 2 * e->I};
    e->nx_w = nx_w;
    e->nx_m = nx_m;
    return delta_mv(e, x, m.down, delta_out, R);
}

// Target model over R rows (tokens in d_tok, positions position..position+R-1).
// Leaves logits [R][V] and final hiddens [R][H] (e->fin).
// `retain`: a speculative branch (Q4 pages are not demoted). The
// GatedDeltaNet states after each row land in the other bank; the caller
// selects the committed row (bank flip + slot).
ctox_status target_forward(ctox_hip_engine *e, const uint32_t *d_tok, uint32_t R, bool retain) {
    TRY(ctox_hip_embedding_rows_device(e->b, e->embed.dtype, e->embed.w, e->embed.s_in, e->embed.s_out, d_tok, R, e->V,
                                       e->H, e->hid, e->s));
    bool pending = false;
    for (size_t li = 0; li < e->layers.size(); li++) {
        Layer &L = e->layers[li];
        const float *dl = pending ? e->delta : nullptr;
        // The token mixer's output projection stages the MLP's normed input.
        if (L.full) {
            TRY(norm_mv(e, dl, L.f.norm, R, L.f.qkv, e->proj));
            e->nx_w = L.mlp.norm;
            e->nx_m = &L.mlp.gate_up;
            TRY(attn_forward(e, L.f, R, e->position, e->delta, retain));
        } else {
            TRY(norm_mv(e, dl, L.g.norm, R, L.g.in, e->proj));
            e->nx_w = L.mlp.norm;
            e->nx_m = &L.mlp.gate_up;
            TRY(gdn_forward(e, L.g, R, e->delta));
        }
        const float *nw = nullptr;
        const Mat *nm = nullptr;
        if (li + 1 < e->layers.size()) {
            const Layer &N = e->layers[li + 1];
            nw = N.full ? N.f.norm : N.g.norm;
            nm = N.full ? &N.f.qkv : &N.g.in;
        }
        TRY(mlp_forward(e, L.mlp, R, e->delta, e->delta, nw, nm));
        pending = true;
    }
    return norm_mv(e, e->delta, e->final_norm, R, e->lm_head, e->logits, e->fin);
}

// MTP over R rows: tokens d_tok, previous hiddens prev [R][H], rope positions rope0..;
// leaves the MTP final hidden in mtp_hidden and, when `logits` is set, its LM head rows there.
ctox_status mtp_forward(ctox_hip_engine *e, const uint32_t *d_tok, const float *prev, uint32_t R, uint32_t rope0,
                        float *logits, bool retain) {
    TRY(ctox_hip_embedding_rows_device(e->b, e->embed.dtype, e->embed.w, e->embed.s_in, e->embed.s_out, d_tok, R, e->V,
                                       e->H, e->hid, e->s));
    // [norm(embedding), norm(previous hidden)] (decoder.rs:1023-1033)
    TRY(norm(e, e->hid, nullptr, e->mtp_norm_emb, R, e->H, e->fcin, 2 * e->H));
    // (no delta: the norm only reads its rows)
    TRY(norm(e, const_cast<float *>(prev), nullptr, e->mtp_norm_hid, R, e->H, e->fcin + e->H, 2 * e->H));
    TRY(matvec(e, e->mtp_fc, e->fcin, e->hid, R));
    TRY(norm_mv(e, nullptr, e->mtp_attn.norm, R, e->mtp_attn.qkv, e->proj));
    TRY(attn_forward(e, e->mtp_attn, R, rope0, e->delta, retain));
    TRY(mlp_forward(e, e->mtp_mlp, R, e->delta, e->delta));
    if (logits) return norm_mv(e, e->delta, e->mtp_norm, R, e->draft_n ? e->draft_head : e->lm_head, logits,
                               e->mtp_hidden);
    return norm(e, e->hid, e->delta, e->mtp_norm, R, e->H, e->mtp_hidden, e->H);
}

// Demotes every cache's aged pages, then uploads all changed descriptors
// in one launch.
ctox_status demote_all(ctox_hip_engine *e) {
    std::vector<Cache *> caches;
    for (Layer &L : e->layers)
        if (L.full) caches.push_back(&L.f.cache);
    if (e->mtp) caches.push_back(&e->mtp_attn.cache);
    std::vector<uint32_t *> dst;
    std::vector<const uint32_t *> src;
    std::vector<size_t> count;
    for (Cache *c : caches) {
        TRY(cache_demote(e, *c));
        if (c->dirty < c->pages) {
            dst.push_back((uint32_t *)(c->d_desc + c->dirty));
            src.push_back((const uint32_t *)(c->desc.data() + c->dirty));
            count.push_back((size_t)(c->pages - c->dirty) * 4);
        }
        c->dirty = c->pages;
    }
    return ctox_write_word_ranges_device(e->b, dst.data(), src.data(), count.data(), dst.size(), e->s);
}

// Queues the finite check of `n` logits into flag words [0, kFlagParts).
constexpr uint32_t kFlagParts = 64;
ctox_status check_logits(ctox_hip_engine *e, const float *x, size_t n, uint32_t flag0 = 0) {
    return ctox_hip_check_finite_device(e->b, x, n, e->d_flags + flag0, kFlagParts, e->s);
}

// After the step's synchronization: fail closed on a flagged buffer
// (Q/src/backend/cuda_runtime.rs:10627-10632, Q/src/engine.rs:191-272).
ctox_status sync(ctox_hip_engine *e) {
    hipError_t err = hipStreamSynchronize(e->s);
    return err == hipSuccess ? CTOX_OK : efail(CTOX_ERR_INVALID_STATE, "engine stream failed: %s", hipGetErrorString(err));
}

// Reads count device words at src into e->h_res once the stream has run
// everything queued so far.
ctox_status read_result(ctox_hip_engine *e, const uint32_t *src, uint32_t count) {
    if (hipMemcpyAsync(e->h_res, src, count * sizeof(uint32_t), hipMemcpyDeviceToHost, e->s) != hipSuccess)
        return efail(CTOX_ERR_INVALID_STATE, "result read failed");
    return sync(e);
}

// Device copy of whole 32-bit words by a copy kernel (a runtime
// device-to-device copy costs several times the host time of a launch).
ctox_status copy_d2d(ctox_hip_engine *e, void *dst, const void *src, size_t bytes) {
    if (bytes % 4) return efail(CTOX_ERR_SHAPE, "engine copies move whole words");
    const size_t n = bytes / 4;
    return ctox_hip_copy_rows_device(e->b, (const float *)src, n, 0, 1, n, (float *)dst, n, e->s);
}

}  // namespace

extern "C" ctox_status ctox_hip_engine_create(ctox_hip_backend *b, const ctox_engine_config *cfg, uint64_t seed,
                                              ctox_hip_engine **out) {
    return ctox_hip_engine_create_with_dtypes(b, cfg, seed, nullptr, 0, out);
}

extern "C" ctox_status ctox_hip_engine_create_with_dtypes(ctox_hip_backend *b, const ctox_engine_config *cfg,
                                                          uint64_t seed, const ctox_engine_matrix_dtype *plan,
                                                          size_t plan_len, ctox_hip_engine **out) {
    if (!b || !cfg || !out || (!plan && plan_len)) return efail(CTOX_ERR_SHAPE, "null argument");
    for (size_t i = 0; i < plan_len; i++)
        if (!plan[i].name || (plan[i].dtype != CTOX_DTYPE_Q2B64 && plan[i].dtype != CTOX_DTYPE_Q4B64))
            return efail(CTOX_ERR_UNSUPPORTED_DTYPE, "an engine matrix is pure Q2_B64 or Q4_B64");
    *out = nullptr;
    const ctox_engine_config &c = *cfg;
    // Q/src/config.rs:35-73 geometry; the attention kernel needs head_dim 256.
    if (c.hidden_size == 0 || c.hidden_size % 64 || c.intermediate_size % 64 || c.num_hidden_layers == 0 ||
        c.full_attention_interval == 0 || c.num_key_value_heads == 0 ||
        c.num_attention_heads % c.num_key_value_heads || c.head_dim != 256 || c.linear_num_key_heads == 0 ||
        c.linear_num_value_heads % c.linear_num_key_heads || c.linear_key_head_dim > 128 ||
        c.linear_value_head_dim > 128 || c.linear_conv_kernel_dim == 0 || c.vocab_size == 0 || c.max_tokens == 0 ||
        c.page_tokens == 0 || c.sink_tokens % c.page_tokens || c.draft_tokens > 7 || c.recent_tokens > c.max_tokens ||
        (c.num_attention_heads * c.head_dim) % 64 || (c.linear_num_value_heads * c.linear_value_head_dim) % 64 ||
        !(c.rms_norm_epsilon > 0.0f) || !(c.rope_theta > 0.0f) || c.rotary_dim == 0 || c.rotary_dim % 2 ||
        c.rotary_dim > c.head_dim)
        return efail(CTOX_ERR_SHAPE, "engine configuration is invalid");
    // A zero recent window demotes the page being filled, after which the
    // crate appends Q2 rows to it (Q/src/kv_cache.rs:199-206); the device
    // appends Q4 rows only, so that configuration is refused.
    if (c.recent_tokens == 0)
        return efail(CTOX_ERR_UNSUPPORTED_OPERATION, "a zero recent KV window (Q2 appends) is not supported");
    ctox_hip_engine *e = new ctox_hip_engine();
    e->b = b;
    e->c = c;
    for (size_t i = 0; i < plan_len; i++) e->dtype_plan[plan[i].name] = plan[i].dtype;
    if (const char *v = std::getenv("CTOX_NEXT_NORM")) e->next_norm = std::atoi(v) != 0;
    e->mtp = c.mtp_layers > 0 && c.draft_tokens > 0;
    e->R = e->mtp ? c.draft_tokens + 1 : 1;
    e->H = c.hidden_size;
    e->I = c.intermediate_size;
    e->Kw = c.linear_num_key_heads * c.linear_key_head_dim;
    e->Vw = c.linear_num_value_heads * c.linear_value_head_dim;
    e->C = 2 * e->Kw + e->Vw;
    e->Rin = e->C + e->Vw + 2 * c.linear_num_value_heads;
    e->kvw = c.num_key_value_heads * c.head_dim;
    e->Rq = 2 * c.num_attention_heads * c.head_dim + 2 * e->kvw;
    e->V = c.vocab_size;
    e->q4_token_bytes = 2 * e->kvw / 64 * 34;
    e->q2_token_bytes = 2 * e->kvw / 64 * 18;
    e->q4_page_bytes = c.page_tokens * e->q4_token_bytes;
    e->q2_page_bytes = c.page_tokens * e->q2_token_bytes;
    auto cleanup = [&](ctox_status st) {
        ctox_hip_engine_destroy(e);
        return st;
    };
    if (hipStreamCreate(&e->s) != hipSuccess) return cleanup(efail(CTOX_ERR_INVALID_STATE, "stream creation failed"));
    ctox_status st;
    uint64_t sd = seed * 1000003ull + 17;
    if ((st = make_mat(e, "embed", e->embed, CTOX_DTYPE_Q4B64, e->V, e->H, sd, nullptr, false))) return cleanup(st);
    if ((st = make_mat(e, "lm_head", e->lm_head, CTOX_DTYPE_Q4B64, e->V, e->H, sd))) return cleanup(st);
    if ((st = make_vec(e, &e->final_norm, e->H, sd, 0.0f, 0.1f))) return cleanup(st);
    uint32_t n_gdn = 0;
    for (uint32_t l = 0; l < c.num_hidden_layers; l++) n_gdn += ((l + 1) % c.full_attention_interval) != 0;
    const uint32_t Hv = c.linear_num_value_heads;
    // States in the fused kernel's blocked layout: 128 x ceil16(value_dim) floats per head.
    const size_t head_floats = (size_t)(c.linear_value_head_dim + 15) / 16 * 2048;
    e->gdn_floats = (size_t)n_gdn * Hv * head_floats;
    e->conv_floats = (size_t)n_gdn * e->C * c.linear_conv_kernel_dim;
    if ((st = dalloc_t(e, &e->gdn_bank, 2 * (size_t)e->R * e->gdn_floats)) ||
        (st = dalloc_t(e, &e->conv_bank, 2 * (size_t)e->R * e->conv_floats)))
        return cleanup(st);
    // Only the current slot is read before it is written.
    if (hipMemsetAsync(e->gdn_bank, 0, e->gdn_floats * 4, e->s) != hipSuccess ||
        hipMemsetAsync(e->conv_bank, 0, e->conv_floats * 4, e->s) != hipSuccess)
        return cleanup(efail(CTOX_ERR_INVALID_STATE, "state clear failed"));
    e->layers.resize(c.num_hidden_layers);
    uint32_t gi = 0;
    for (uint32_t l = 0; l < c.num_hidden_layers; l++) {
        Layer &L = e->layers[l];
        L.full = ((l + 1) % c.full_attention_interval) == 0;  // config.rs:61-72
        if (L.full) {
            if ((st = make_attn(e, "L" + std::to_string(l), L.f, sd))) return cleanup(st);
        } else {
            GdnLayer &g = L.g;
            if ((st = make_vec(e, &g.norm, e->H, sd, 0.0f, 0.1f))) return cleanup(st);
            if ((st = make_mat(e, "L" + std::to_string(l) + ".in", g.in, CTOX_DTYPE_Q4B64, e->Rin, e->H, sd)))
                return cleanup(st);
            if ((st = make_vec(e, &g.conv_w, (size_t)e->C * c.linear_conv_kernel_dim, sd, 0.0f, 0.5f))) return cleanup(st);
            if ((st = dalloc_t(e, &g.a_log, Hv)) || (st = fill(e, g.a_log, Hv, 4, sd++, -2.0f, 1.0f))) return cleanup(st);
            if ((st = dalloc_t(e, &g.dt_bias, Hv)) || (st = fill(e, g.dt_bias, Hv, 4, sd++, -1.0f, 1.0f))) return cleanup(st);
            if ((st = make_vec(e, &g.gnorm, c.linear_value_head_dim, sd, 1.0f, 0.1f))) return cleanup(st);
            if ((st = make_mat(e, "L" + std::to_string(l) + ".out", g.out, CTOX_DTYPE_Q4B64, e->H, e->Vw, sd)))
                return cleanup(st);
            g.state_off = (size_t)gi * Hv * head_floats;
            g.conv_off = (size_t)gi * e->C * c.linear_conv_kernel_dim;
            gi++;
        }
        if ((st = make_mlp(e, "L" + std::to_string(l), L.mlp, sd))) return cleanup(st);
    }
    if (e->mtp) {
        if ((st = make_vec(e, &e->mtp_norm_emb, e->H, sd, 0.0f, 0.1f)) ||
            (st = make_vec(e, &e->mtp_norm_hid, e->H, sd, 0.0f, 0.1f)) ||
            (st = make_vec(e, &e->mtp_norm, e->H, sd, 0.0f, 0.1f)) ||
            (st = make_mat(e, "mtp.fc", e->mtp_fc, CTOX_DTYPE_Q4B64, e->H, 2 * e->H, sd)) ||
            (st = make_attn(e, "mtp", e->mtp_attn, sd)) || (st = make_mlp(e, "mtp", e->mtp_mlp, sd)))
            return cleanup(st);
    }
    const size_t R = e->R, qh = c.num_attention_heads, hd = c.head_dim;
    const size_t widest = std::max<size_t>({e->Rin, e->Rq, 2 * (size_t)e->I, e->H});
    if ((st = dalloc_t(e, &e->hid, R * e->H)) || (st = dalloc_t(e, &e->hid2, R * e->H)) ||
        (st = dalloc_t(e, &e->proj, R * widest)) || (st = dalloc_t(e, &e->convo, R * e->C)) ||
        (st = dalloc_t(e, &e->core, R * e->Vw)) || (st = dalloc_t(e, &e->coren, R * e->Vw)) ||
        (st = dalloc_t(e, &e->delta, 16 * R * e->H)) || (st = dalloc_t(e, &e->q, R * qh * hd)) ||
        (st = dalloc_t(e, &e->k, R * e->kvw)) || (st = dalloc_t(e, &e->v, R * e->kvw)) ||
        (st = dalloc_t(e, &e->attn, R * qh * hd)) || (st = dalloc_t(e, &e->gu, (size_t)R * 6 * 2 * e->I)) ||
        (st = dalloc_t(e, &e->act, R * e->I)) || (st = dalloc_t(e, &e->fin, R * e->H)) ||
        (st = dalloc_t(e, &e->logits, R * e->V)) || (st = dalloc_t(e, &e->ld, R * Hv)) ||
        (st = dalloc_t(e, &e->beta, R * Hv)) || (st = dalloc_t(e, &e->fcin, R * 2 * e->H)) ||
        (st = dalloc_t(e, &e->draft_logits, (size_t)std::max(1u, c.draft_tokens) * e->V)) ||
        (st = dalloc_t(e, &e->mtp_hidden, R * e->H)) || (st = dalloc_t(e, &e->prev_hidden, R * e->H)) ||
        (st = dalloc_t(e, &e->d_tokens, 16)) || (st = dalloc_t(e, &e->d_result, 32)) || (st = dalloc_t(e, &e->d_rng, 1)) ||
        (st = dalloc_t(e, &e->rsq, 8 * 512)) || (st = dalloc_t(e, &e->blk_sq, 8 * 128)) || (st = dalloc_t(e, &e->d_flags, 2 * kFlagParts + 32)))
        return cleanup(st);
    e->d_drafts = e->d_result + 16;
    if ((st = sync(e))) return cleanup(st);
    *out = e;
    return CTOX_OK;
}

extern "C" void ctox_hip_engine_destroy(ctox_hip_engine *e) {
    if (!e) return;
    if (e->s) hipStreamSynchronize(e->s);
    for (const auto &t : e->tiled) ctox_hip_unregister_tiled_weights(e->b, t.w);
    for (void *p : e->allocs) hipFree(p);
    if (e->s) hipStreamDestroy(e->s);
    delete e;
}

extern "C" void *ctox_hip_engine_stream(ctox_hip_engine *e) { return e ? (void *)e->s : nullptr; }

extern "C" ctox_status ctox_hip_engine_set_rng(ctox_hip_engine *e, uint64_t state) {
    if (!e) return efail(CTOX_ERR_SHAPE, "null argument");
    if (hipMemcpyAsync(e->d_rng, &state, 8, hipMemcpyHostToDevice, e->s) != hipSuccess)
        return efail(CTOX_ERR_INVALID_STATE, "rng upload failed");
    return sync(e);
}

// One target step (CpuCorrectnessExecutor::decode without MTP, decoder.rs:956-998):
// logits of the next position in the engine's logits buffer; *d_logits points there.
extern "C" ctox_status ctox_hip_engine_decode(ctox_hip_engine *e, uint32_t token, const float **d_logits) {
    if (!e) return efail(CTOX_ERR_SHAPE, "null argument");
    if (e->loading) return efail(CTOX_ERR_INVALID_STATE, "weights written without ctox_hip_engine_finish_load");
    if (token >= e->V) return efail(CTOX_ERR_SHAPE, "token outside the vocabulary");
    if (e->position >= e->c.max_tokens) return efail(CTOX_ERR_MEMORY_BUDGET, "context is full");
    TRY(ctox_hip_write_words_device(e->b, e->d_tokens, &token, 1, e->s));
    // MTP prefill semantics (decoder.rs:1248-1261): the MTP cache advances with
    // (token, previous target hidden) for every position after the first.
    if (e->mtp && e->have_prev) {
        TRY(mtp_forward(e, e->d_tokens, e->prev_hidden, 1, e->position, nullptr, false));
        e->mtp_tokens++;
    }
    TRY(target_forward(e, e->d_tokens, 1, false));
    e->bank ^= 1u;  // the state after the row is slot 0 of the other bank
    e->sidx = 0;
    TRY(copy_d2d(e, e->prev_hidden, e->fin, (size_t)e->H * 4));
    e->have_prev = true;
    e->position++;
    TRY(demote_all(e));
    TRY(check_logits(e, e->logits, e->V));
    if (d_logits) *d_logits = e->logits;
    TRY(read_result(e, e->d_flags, kFlagParts));
    for (uint32_t i = 0; i < kFlagParts; i++)
        if (e->h_res[i]) return efail(CTOX_ERR_INVALID_STATE, "non-finite logits in the decode step");
    return CTOX_OK;
}

// One speculative step: k drafts sampled at `temperature`, one batched target
// pass over [token, d1..dk], acceptance and commit. out[0] = next token,
// out[1] = accepted drafts n, out[2..2+n) = the accepted drafts.
// Temperature 0 is the crate's greedy MTP (Q/src/engine.rs:583-590,
// 915-963): drafts are argmax tokens (over the draft vocabulary when one is
// bound), the verification accepts the longest prefix equal to the target
// argmax tokens, and the next token is the first differing target argmax or,
// with every draft accepted, the bonus row's argmax.
extern "C" ctox_status ctox_hip_engine_mtp_step(ctox_hip_engine *e, uint32_t token, float temperature,
                                                uint32_t *out) {
    if (!e || !out) return efail(CTOX_ERR_SHAPE, "null argument");
    if (!std::isfinite(temperature) || temperature < 0.0f)
        return efail(CTOX_ERR_INVALID_ARTIFACT, "sampling temperature must be finite and non-negative");
    const bool greedy = temperature == 0.0f;
    if (!e->mtp) return efail(CTOX_ERR_UNSUPPORTED_OPERATION, "engine was created without an MTP head");
    if (e->loading) return efail(CTOX_ERR_INVALID_STATE, "weights written without ctox_hip_engine_finish_load");
    if (!e->have_prev) return efail(CTOX_ERR_INVALID_STATE, "MTP step needs a previous target step");
    if (token >= e->V) return efail(CTOX_ERR_SHAPE, "token outside the vocabulary");
    const uint32_t k = e->c.draft_tokens, R = k + 1, p = e->position;
    if (p + R > e->c.max_tokens) return efail(CTOX_ERR_MEMORY_BUDGET, "context is full");
    TRY(ctox_hip_write_words_device(e->b, e->d_tokens, &token, 1, e->s));
    // Drafts: d_{i+1} ~ softmax(MTP(x_i, g_i) / T) with x_0 = token, g_0 = the last
    // target hidden, then x_i = d_i, g_i = the MTP hidden of step i.
    TRY(copy_d2d(e, e->d_drafts, e->d_tokens, 4));
    // Draft rows: the full head, or the restricted one (draft_n scores).
    const uint32_t dn = e->draft_n ? e->draft_n : e->V;
    for (uint32_t i = 0; i < k; i++) {
        TRY(mtp_forward(e, e->d_drafts + i, i == 0 ? e->prev_hidden : e->mtp_hidden, 1, p + i,
                        e->draft_logits + (size_t)i * dn, true));
        if (greedy) {
            // The draft row's argmax (DraftDistribution::greedy_token: the
            // later index wins ties; a restricted index maps to its token).
            TRY(ctox_greedy_tokens_mapped(e->b, e->draft_logits + (size_t)i * dn, 1, dn,
                                          e->draft_n ? e->d_draft_ids : nullptr, e->d_drafts + i + 1, e->s));
            continue;
        }
        // drafts = 0 samples the bonus row: the draft token from its own
        // softmax (a restricted row's index mapped to its token).
        TRY(ctox_hip_mtp_accept_restricted_device(e->b, nullptr, dn, nullptr, nullptr, e->draft_logits + (size_t)i * dn,
                                                  e->draft_n ? e->d_draft_ids : nullptr, e->d_drafts, 0, dn,
                                                  temperature, e->d_rng, e->d_drafts + i + 1, e->s));
    }
    // Verify [token, d1..dk] in one pass; every row's GatedDeltaNet state is kept.
    TRY(target_forward(e, e->d_drafts, R, true));
    uint32_t next = 0, n = 0;
    const uint32_t *host = e->h_res;
    if (greedy) {
        // One read brings back the finite flags of the target and draft
        // logits (words [0, 2 * kFlagParts)), the target argmax of every row
        // (16 words from 2 * kFlagParts) and [token, d1..dk] (the 16 after).
        uint32_t *d_tail = e->d_flags + 2 * kFlagParts;
        TRY(check_logits(e, e->logits, (size_t)R * e->V));
        TRY(check_logits(e, e->draft_logits, (size_t)k * dn, kFlagParts));
        TRY(ctox_hip_greedy_tokens_device(e->b, e->logits, R, e->V, d_tail, e->s));
        TRY(copy_d2d(e, d_tail + 16, e->d_drafts, (size_t)R * 4));
        TRY(read_result(e, e->d_flags, 2 * kFlagParts + 16 + R));
        uint32_t flagged = 0;
        for (uint32_t i = 0; i < 2 * kFlagParts; i++) flagged |= host[i];
        if (flagged) return efail(CTOX_ERR_INVALID_STATE, "non-finite logits in the speculative step");
        const uint32_t *targets = host + 2 * kFlagParts, *drafts = targets + 16;
        next = targets[k];
        n = k;
        for (uint32_t i = 0; i < k; i++)
            if (drafts[1 + i] != targets[i]) {
                next = targets[i];
                n = i;
                break;
            }
        // The commit below reads the accepted drafts at host[17 + i].
        std::memmove(e->h_res + 16, drafts, (size_t)R * sizeof(uint32_t));
    } else {
        TRY(ctox_hip_mtp_accept_restricted_device(e->b, e->draft_logits, dn, e->draft_n ? e->d_draft_inv : nullptr,
                                                  e->logits, e->logits + (size_t)k * e->V, nullptr, e->d_drafts + 1, k,
                                                  e->V, temperature, e->d_rng, e->d_result, e->s));
        TRY(read_result(e, e->d_result, 16 + R));
        // The acceptance reports non-finite draft or target logits as 0xfffffffe;
        // nothing is committed from such a step.
        if (host[0] == 0xfffffffeu) return efail(CTOX_ERR_INVALID_STATE, "non-finite logits in the speculative step");
        next = host[0];
        n = host[1];
    }
    if (n > k || next >= e->V) return efail(CTOX_ERR_INVALID_STATE, "acceptance produced an invalid result");
    // Commit n + 1 target tokens: the state after row n, the caches truncated.
    e->bank ^= 1u;
    e->sidx = n;
    for (Layer &L : e->layers)
        if (L.full) cache_truncate(L.f.cache, k - n);
    // MTP cache: keep the first draft's entry (token, previous hidden), replay
    // d1..dn with the target final hiddens h_p..h_{p+n-1} (commit_speculative),
    // rows 0..n-1 of fin (the MTP layer does not write fin).
    cache_truncate(e->mtp_attn.cache, k - 1);
    if (n > 0) TRY(mtp_forward(e, e->d_drafts + 1, e->fin, n, p + 1, nullptr, true));
    e->mtp_tokens = e->mtp_attn.cache.tokens;
    TRY(copy_d2d(e, e->prev_hidden, e->fin + (size_t)n * e->H, (size_t)e->H * 4));
    e->position = p + n + 1;
    TRY(demote_all(e));  // uploads every changed descriptor
    out[0] = next;
    out[1] = n;
    for (uint32_t i = 0; i < n; i++) out[2 + i] = host[17 + i];
    // The commit's launches stay queued on the engine stream: every later
    // call and read is ordered after them, and the host returns without
    // waiting (the result above came back with the acceptance).
    return CTOX_OK;
}

// Context of `tokens` random K/V rows in every paged cache (and the MTP cache),
// position = tokens; recurrent states stay as they are. Config 5's "context
// filled with random K/V".
extern "C" ctox_status ctox_hip_engine_fill_context(ctox_hip_engine *e, uint32_t tokens, uint64_t seed) {
    if (!e) return efail(CTOX_ERR_SHAPE, "null argument");
    if (e->loading) return efail(CTOX_ERR_INVALID_STATE, "weights written without ctox_hip_engine_finish_load");
    if (e->position != 0 || tokens == 0 || tokens + e->R > e->c.max_tokens)
        return efail(CTOX_ERR_SHAPE, "context fill needs an empty engine and room for a step");
    const uint32_t chunk = 1024;
    float *kbuf = nullptr, *vbuf = nullptr;
    TRY(dalloc_t(e, &kbuf, (size_t)chunk * e->kvw));
    TRY(dalloc_t(e, &vbuf, (size_t)chunk * e->kvw));
    auto fill_cache = [&](Cache &c, uint64_t sd) -> ctox_status {
        for (uint32_t t = 0; t < tokens; t += chunk) {
            const uint32_t n = std::min(chunk, tokens - t);
            TRY(fill(e, kbuf, (uint64_t)n * e->kvw, 2, sd + 2 * t, 0.0f, 1.0f));
            TRY(fill(e, vbuf, (uint64_t)n * e->kvw, 2, sd + 2 * t + 1, 0.0f, 1.0f));
            for (uint32_t o = 0; o < n; o += e->c.page_tokens) {  // demote as the pages fill
                const uint32_t m = std::min(e->c.page_tokens, n - o);
                TRY(cache_push(e, c, kbuf + (size_t)o * e->kvw, vbuf + (size_t)o * e->kvw, m));
                TRY(cache_demote(e, c));
            }
            TRY(cache_upload(e, c));
        }
        return CTOX_OK;
    };
    uint64_t sd = seed * 7919 + 3;
    for (Layer &L : e->layers)
        if (L.full) TRY(fill_cache(L.f.cache, sd += 1000003));
    if (e->mtp) TRY(fill_cache(e->mtp_attn.cache, sd += 1000003));
    // A previous target hidden so that the first MTP step has its input.
    TRY(fill(e, e->prev_hidden, e->H, 2, sd + 11, 0.0f, 1.0f));
    e->have_prev = true;
    e->position = tokens;
    e->mtp_tokens = e->mtp ? tokens : 0;
    if (e->mtp) {
        // the MTP cache holds position - 1 entries (decoder.rs:1018-1021)
        cache_truncate(e->mtp_attn.cache, 1);
        TRY(cache_upload(e, e->mtp_attn.cache));
        e->mtp_tokens = tokens - 1;
    }
    return sync(e);
}

// Device views for tests and tools. which: 0 logits [R][V], 1 final hidden
// [R][H], 2 previous target hidden [H], 3 GatedDeltaNet states (blocked layout of ctox_hip_gdn_fused_snap_device), 4 conv states,
// 5 draft logits [k][V].
extern "C" ctox_status ctox_hip_engine_buffer(ctox_hip_engine *e, uint32_t which, void **ptr, size_t *bytes) {
    if (!e || !ptr || !bytes) return efail(CTOX_ERR_SHAPE, "null argument");
    switch (which) {
    case 0: *ptr = e->logits; *bytes = (size_t)e->R * e->V * 4; break;
    case 1: *ptr = e->fin; *bytes = (size_t)e->R * e->H * 4; break;
    case 2: *ptr = e->prev_hidden; *bytes = (size_t)e->H * 4; break;
    case 3: *ptr = state_cur(e); *bytes = e->gdn_floats * 4; break;
    case 4: *ptr = conv_cur(e); *bytes = e->conv_floats * 4; break;
    case 5:
        *ptr = e->draft_logits;
        *bytes = (size_t)std::max(1u, e->c.draft_tokens) * (e->draft_n ? e->draft_n : e->V) * 4;
        break;
    default: return efail(CTOX_ERR_SHAPE, "unknown engine buffer");
    }
    return CTOX_OK;
}

extern "C" uint32_t ctox_hip_engine_position(const ctox_hip_engine *e) { return e ? e->position : 0; }

// Binds the release's MTP draft vocabulary (CpuCorrectnessExecutor::load,
// Q/src/decoder.rs:1129-1182; ReleaseManifest::load_mtp_draft_token_ids,
// Q/src/release.rs:414-431): strictly increasing token IDs inside the
// vocabulary, set once. Drafts then score only those LM-head rows.
extern "C" ctox_status ctox_hip_engine_set_draft_vocab(ctox_hip_engine *e, const uint32_t *ids, size_t n) {
    if (!e || (!ids && n)) return efail(CTOX_ERR_SHAPE, "null argument");
    if (!e->mtp) return efail(CTOX_ERR_UNSUPPORTED_OPERATION, "engine was created without an MTP head");
    if (e->draft_n) return efail(CTOX_ERR_INVALID_STATE, "the draft vocabulary is already bound");
    bool canonical = n > 0 && n <= e->V;
    for (size_t i = 0; canonical && i < n; i++) canonical = ids[i] < e->V && (i == 0 || ids[i - 1] < ids[i]);
    if (!canonical) return efail(CTOX_ERR_INVALID_ARTIFACT, "noncanonical MTP draft vocabulary");
    Mat &m = e->draft_head;
    m.dtype = e->lm_head.dtype;
    m.rows = (uint32_t)n;
    m.cols = e->lm_head.cols;
    m.s_in = e->lm_head.s_in;
    const size_t rb = (size_t)m.cols / 64 * (m.dtype == CTOX_DTYPE_Q4B64 ? 34 : 18);
    TRY(dalloc(e, (void **)&m.w, m.bytes()));
    TRY(dalloc_t(e, &m.s_out, n));
    TRY(ctox_hip_gather_rows_device(e->b, e->lm_head.w, e->lm_head.rows, rb, ids, n, m.w, e->s));
    TRY(ctox_hip_gather_rows_device(e->b, e->lm_head.s_out, e->lm_head.rows, 2, ids, n, m.s_out, e->s));
    TRY(ctox_hip_register_tiled_weights(e->b, m.dtype, m.w, m.rows, m.cols, e->s));
    e->tiled.push_back({m.w, m.dtype, m.rows, m.cols});
    std::vector<uint32_t> inv(e->V, 0xffffffffu);
    for (size_t i = 0; i < n; i++) inv[ids[i]] = (uint32_t)i;
    TRY(dalloc_t(e, &e->d_draft_ids, n));
    TRY(dalloc_t(e, &e->d_draft_inv, e->V));
    if (hipMemcpyAsync(e->d_draft_ids, ids, n * 4, hipMemcpyHostToDevice, e->s) != hipSuccess ||
        hipMemcpyAsync(e->d_draft_inv, inv.data(), (size_t)e->V * 4, hipMemcpyHostToDevice, e->s) != hipSuccess)
        return efail(CTOX_ERR_INVALID_STATE, "draft vocabulary upload failed");
    TRY(sync(e));
    e->draft_n = (uint32_t)n;
    return CTOX_OK;
}

// Weights by name, as the crate's tensor names (Q/src/tensor_contract.rs) with
// the fused matrices named by their first member: "embed", "lm_head",
// "final_norm", "L<i>.<part>" with part in {norm, in (qkv|z|a|b), conv_w,
// a_log, dt_bias, gnorm, out, qkv (q|gate, k, v), q_norm, k_norm, o,
// mlp_norm, gate_up, down} and the MTP parts "mtp.<part>" with part in
// {norm_emb, norm_hid, norm, fc, attn_norm, qkv, q_norm, k_norm, o, mlp_norm,
// gate_up, down}.
extern "C" ctox_status ctox_hip_engine_tensor(ctox_hip_engine *e, const char *name, ctox_engine_tensor *t) {
    if (!e || !name || !t) return efail(CTOX_ERR_SHAPE, "null argument");
    std::memset(t, 0, sizeof *t);
    auto mat = [&](const Mat &m) {
        t->data = m.w;
        t->bytes = m.bytes();
        t->rows = m.rows;
        t->cols = m.cols;
        t->dtype = m.dtype;
        t->s_in = m.s_in;
        t->s_out = m.s_out;
        return CTOX_OK;
    };
    auto vec = [&](const float *p, size_t n) {
        t->data = (void *)p;
        t->bytes = n * 4;
        t->rows = 1;
        t->cols = (uint32_t)n;
        t->dtype = -1;
        return CTOX_OK;
    };
    const std::string s(name);
    if (s == "embed") return mat(e->embed);
    if (s == "lm_head") return mat(e->lm_head);
    if (s == "final_norm") return vec(e->final_norm, e->H);
    auto attn_part = [&](const AttnLayer &a, const std::string &part) -> ctox_status {
        if (part == "attn_norm" || part == "norm") return vec(a.norm, e->H);
        if (part == "qkv") return mat(a.qkv);
        if (part == "q_norm") return vec(a.q_norm, e->c.head_dim);
        if (part == "k_norm") return vec(a.k_norm, e->c.head_dim);
        if (part == "o") return mat(a.o);
        return efail(CTOX_ERR_SHAPE, "unknown tensor %s", name);
    };
    auto mlp_part = [&](const Mlp &m, const std::string &part, bool *hit) -> ctox_status {
        *hit = true;
        if (part == "mlp_norm") return vec(m.norm, e->H);
        if (part == "gate_up") return mat(m.gate_up);
        if (part == "down") return mat(m.down);
        *hit = false;
        return CTOX_OK;
    };
    if (s.rfind("mtp.", 0) == 0) {
        if (!e->mtp) return efail(CTOX_ERR_SHAPE, "engine has no MTP head");
        const std::string part = s.substr(4);
        if (part == "norm_emb") return vec(e->mtp_norm_emb, e->H);
        if (part == "norm_hid") return vec(e->mtp_norm_hid, e->H);
        if (part == "norm") return vec(e->mtp_norm, e->H);
        if (part == "fc") return mat(e->mtp_fc);
        bool hit;
        ctox_status st = mlp_part(e->mtp_mlp, part, &hit);
        if (hit) return st;
        return attn_part(e->mtp_attn, part == "attn_norm" ? "norm" : part);
    }
    if (s.size() > 1 && s[0] == 'L') {
        const size_t dot = s.find('.');
        if (dot == std::string::npos) return efail(CTOX_ERR_SHAPE, "unknown tensor %s", name);
        const uint32_t l = (uint32_t)std::strtoul(s.substr(1, dot - 1).c_str(), nullptr, 10);
        if (l >= e->layers.size()) return efail(CTOX_ERR_SHAPE, "layer out of range");
        const std::string part = s.substr(dot + 1);
        const Layer &L = e->layers[l];
        bool hit;
        ctox_status st = mlp_part(L.mlp, part, &hit);
        if (hit) return st;
        if (L.full) return attn_part(L.f, part);
        const GdnLayer &g = L.g;
        if (part == "norm") return vec(g.norm, e->H);
        if (part == "in") return mat(g.in);
        if (part == "conv_w") return vec(g.conv_w, (size_t)e->C * e->c.linear_conv_kernel_dim);
        if (part == "a_log") return vec(g.a_log, e->c.linear_num_value_heads);
        if (part == "dt_bias") return vec(g.dt_bias, e->c.linear_num_value_heads);
        if (part == "gnorm") return vec(g.gnorm, e->c.linear_value_head_dim);
        if (part == "out") return mat(g.out);
    }
    return efail(CTOX_ERR_SHAPE, "unknown tensor %s", name);
}

extern "C" ctox_status ctox_hip_engine_cache(ctox_hip_engine *e, uint32_t layer, ctox_engine_cache_view *v) {
    if (!e || !v) return efail(CTOX_ERR_SHAPE, "null argument");
    const Cache *c = nullptr;
    if (layer == 0xffffffffu) {
        if (!e->mtp) return efail(CTOX_ERR_SHAPE, "engine has no MTP head");
        c = &e->mtp_attn.cache;
    } else {
        if (layer >= e->layers.size() || !e->layers[layer].full)
            return efail(CTOX_ERR_SHAPE, "layer %u is not a full-attention layer", layer);
        c = &e->layers[layer].f.cache;
    }
    v->descriptors = c->desc.data();
    v->pages = c->pages;
    v->tokens = c->tokens;
    v->d_q4_pool = c->q4;
    v->d_q2_pool = c->q2;
    v->q4_page_bytes = e->q4_page_bytes;
    v->q2_page_bytes = e->q2_page_bytes;
    return CTOX_OK;
}

extern "C" ctox_status ctox_hip_engine_write(ctox_hip_engine *e, const char *name, uint32_t part, size_t offset,
                                             const void *host, size_t bytes) {
    if (!e || !name || (!host && bytes)) return efail(CTOX_ERR_SHAPE, "null argument");
    if (e->position || e->draft_n || e->have_prev)
        return efail(CTOX_ERR_INVALID_STATE, "weights are written into a fresh engine, before the draft vocabulary");
    ctox_engine_tensor t;
    TRY(ctox_hip_engine_tensor(e, name, &t));
    void *dst = nullptr;
    size_t cap = 0;
    if (part == CTOX_ENGINE_PART_DATA) {
        dst = t.data;
        cap = t.bytes;
    } else if (t.dtype < 0) {
        return efail(CTOX_ERR_SHAPE, "tensor %s is a vector without scales", name);
    } else if (part == CTOX_ENGINE_PART_S_IN) {
        dst = (void *)t.s_in;
        cap = (size_t)t.cols * 2;
    } else if (part == CTOX_ENGINE_PART_S_OUT) {
        dst = (void *)t.s_out;
        cap = (size_t)t.rows * 2;
    } else {
        return efail(CTOX_ERR_SHAPE, "unknown tensor part %u", part);
    }
    if (offset > cap || bytes > cap - offset)
        return efail(CTOX_ERR_SHAPE, "write of %zu bytes at %zu exceeds %s (%zu bytes)", bytes, offset, name, cap);
    e->loading = true;
    if (bytes && hipMemcpyAsync((uint8_t *)dst + offset, host, bytes, hipMemcpyHostToDevice, e->s) != hipSuccess)
        return efail(CTOX_ERR_INVALID_STATE, "weight upload failed");
    return sync(e);
}

extern "C" ctox_status ctox_hip_engine_finish_load(ctox_hip_engine *e) {
    if (!e) return efail(CTOX_ERR_SHAPE, "null argument");
    for (const auto &t : e->tiled) TRY(ctox_hip_register_tiled_weights(e->b, t.dtype, t.w, t.rows, t.cols, e->s));
    TRY(sync(e));
    e->loading = false;
    return CTOX_OK;
}
