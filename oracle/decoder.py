"""CPU restatement of the crate's decoder graph and MTP executor, the oracle
of the device engine (ctox_hip_engine_*).

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker; the product
path (ctox-llm_amd/) never imports it.

Follows Q/src/decoder.rs (Q = models/qwen38_27b):
  * decode_target_step (:956-998): embedding (:531-537), per layer
    linear_attention_residual (:806-938) or full_attention_residual_at
    (:687-800), decoder_mlp_residual (:636-670), final norm, LM head;
  * mtp_final_hidden (:1009-1046) and the prefill-time MTP advance
    (:1248-1261);
  * restricted_logits_from_final_hidden (:589-627): the draft head over the
    release-bound draft token IDs, one recovered_row_matvec per ID;
  * the speculative step the engine runs (the crate's executor is greedy
    only, so this is the build's specification, stated once here): k drafts
    where draft i + 1 is sampled at temperature T from MTP(x_i, g_i) (over
    the draft vocabulary when one is bound, as the CUDA MTP4 flow drafts,
    Q/src/backend/cuda_graph.rs:4501-4509) with
    x_0 = token, g_0 = the previous target hidden, x_i = d_i and g_i the MTP
    hidden of step i; one target pass over [token, d1..dk] with KV pushes
    that retain Q4 pages (push_retaining_q4, kv_cache.rs:372-381); the
    rejection-sampling acceptance (oracle.mtp_accept_sample); commit of the
    n + 1 accepted target tokens, and the MTP cache rebuilt as
    commit_speculative does (:1397-1458): the first draft's entry kept, the
    accepted drafts replayed with target hiddens; then page demotion.

Every operator is the oracle restatement of Q/src/reference.rs,
Q/src/backend/cpu.rs and Q/src/kv_cache.rs; weights are the engine's own
(downloaded), with the same row-concatenated fused matrices, which compute
the same rows as the crate's fan-out.
"""
from __future__ import annotations

import copy
import math
import os

import numpy as np

from . import oracle as orc
from . import paged_kv as pk


def check_draft_ids(ids, vocab: int) -> np.ndarray:
    """The canonical draft vocabulary: non-empty, strictly increasing, inside
    the vocabulary (Q/src/decoder.rs:597-608, Q/src/release.rs:414-431)."""
    ids = np.asarray(ids, dtype=np.int64).reshape(-1)
    if ids.size == 0 or np.any(ids[1:] <= ids[:-1]) or ids[0] < 0 or ids[-1] >= vocab:
        raise orc.OracleError(1)
    return ids.astype(np.uint32)


def verify_greedy_tokens(drafts, targets):
    """verify_greedy_mtp's compact branch (Q/src/engine.rs:928-943): drafts
    d_1..d_k against the target argmax tokens t_0..t_k; returns (next token,
    accepted count): the first i with d_{i+1} != t_i gives (t_i, i), no
    mismatch gives the bonus token (t_k, k)."""
    for i, d in enumerate(drafts):
        if d != targets[i]:
            return targets[i], i
    return targets[len(drafts)], len(drafts)


class OracleDecoder:
    def __init__(self, cfg: dict, tensor, draft_ids=None):
        """cfg: EngineConfig.as_dict(); tensor(name) -> the engine tensor dict;
        draft_ids: the release-bound MTP draft vocabulary (None: full head)."""
        self.c = cfg
        self.draft_ids = None if draft_ids is None else check_draft_ids(draft_ids, cfg["vocab_size"])
        self.t = {}
        self.fetch = tensor
        c = cfg
        self.H, self.I = c["hidden_size"], c["intermediate_size"]
        self.qh, self.kvh, self.hd = c["num_attention_heads"], c["num_key_value_heads"], c["head_dim"]
        self.hk, self.hv = c["linear_num_key_heads"], c["linear_num_value_heads"]
        self.dk, self.dv = c["linear_key_head_dim"], c["linear_value_head_dim"]
        self.Kw, self.Vw = self.hk * self.dk, self.hv * self.dv
        self.C = 2 * self.Kw + self.Vw
        self.K = c["linear_conv_kernel_dim"]
        self.eps = c["rms_norm_epsilon"]
        self.full = [((l + 1) % c["full_attention_interval"]) == 0 for l in range(c["num_hidden_layers"])]
        self.gdn_state = {l: np.zeros(self.hv * self.dk * self.dv, np.float32)
                          for l in range(len(self.full)) if not self.full[l]}
        self.conv_state = {l: np.zeros(self.C * self.K, np.float32) for l in self.gdn_state}
        self.caches = {l: self._cache() for l in range(len(self.full)) if self.full[l]}
        self.mtp_cache = self._cache() if c["mtp_layers"] else None
        self.position = 0
        self.prev_hidden = None
        # Row-parallel oracle matvecs: rows are independent, so the result
        # equals the single-threaded one.
        self.threads = max(1, min(16, os.cpu_count() or 1))

    def _cache(self):
        c = self.c
        if (self.kvh * self.hd) % orc.BLOCK_LEN:  # FullAttentionState::new (decoder.rs:171-195)
            return pk.DenseKvCache(c["max_tokens"], self.kvh * self.hd)
        return pk.PagedKvCache(c["max_tokens"], self.kvh * self.hd, c["page_tokens"], c["sink_tokens"],
                               c["recent_tokens"])

    # -- weights --------------------------------------------------------------
    def w(self, name):
        if name not in self.t:
            self.t[name] = self.fetch(name)
        return self.t[name]

    def matvec(self, name, x):
        m = self.w(name)
        return orc.MatVec(m["dtype"], m["data"], m["rows"], m["cols"], x, s_in=("f16le", m["s_in"]),
                          s_out=("f16le", m["s_out"]), segments=m.get("segments", ())).run(threads=self.threads)

    @staticmethod
    def _row(m, r):
        """(dtype, packed bytes) of row r; a mixed matrix resolves the row's
        segment (loader.rs:54-127)."""
        dtype, base, local = m["dtype"], 0, r
        for g, start, end, d, off, _ in m.get("segments", ()):
            if start <= r < end:
                dtype, base, local = d, off, r - start
                break
        rb = m["cols"] // 64 * (34 if dtype == orc.Q4B64 else 18)
        return dtype, bytes(m["data"][base + local * rb:base + (local + 1) * rb])

    def load_context(self, pages_of, position, prev_hidden):
        """Starts from a filled context: every full-attention cache (and the
        MTP cache, which holds position - 1 entries) takes the given pages,
        pages_of(layer) with layer -1 for the MTP cache."""
        for l, c in self.caches.items():
            c.load_pages(pages_of(l))
            if c.tokens() != position:
                raise orc.OracleError(7)
        if self.mtp_cache is not None:
            self.mtp_cache.load_pages(pages_of(-1))
            if self.mtp_cache.tokens() != position - 1:
                raise orc.OracleError(7)
        self.position = position
        self.prev_hidden = np.asarray(prev_hidden, np.float32).copy()

    def norm(self, x, name, rows=1):
        x = np.asarray(x, np.float32).reshape(-1)
        return orc.rms_norm_1p_weight(x, rows, x.size // rows, self.w(name)["data"], self.eps)

    def embedding(self, token):
        m = self.w("embed")
        if not 0 <= token < m["rows"]:
            raise orc.OracleError(1)
        s_out = float(np.frombuffer(m["s_out"].tobytes(), np.float16)[token])
        dtype, row = self._row(m, token)
        return orc.recovered_row(dtype, row, m["cols"], ("f16le", m["s_in"]), s_out)

    # -- mixers ---------------------------------------------------------------
    def attention(self, prefix, x, rope_pos, cache, retain):
        """full_attention_residual_at (Q/src/decoder.rs:687-800) minus the residual."""
        qh, kvh, hd = self.qh, self.kvh, self.hd
        out = self.matvec(f"{prefix}.qkv", x)
        qg = out[:2 * qh * hd].reshape(qh, 2 * hd)
        q = self.norm(qg[:, :hd].reshape(-1), f"{prefix}.q_norm", qh)
        gate = qg[:, hd:].reshape(-1).copy()
        k = self.norm(out[2 * qh * hd:2 * qh * hd + kvh * hd], f"{prefix}.k_norm", kvh)
        v = out[2 * qh * hd + kvh * hd:].copy()
        orc.apply_partial_rope(q, k, qh, kvh, hd, self.c["rotary_dim"], rope_pos, self.c["rope_theta"])
        cache.push(k, v, demote=not retain)
        att = pk.paged_attention(cache, q.reshape(1, qh, hd), 1, qh, kvh, hd)
        orc.sigmoid_gate(att, gate)
        return self.matvec(f"{prefix}.o", att)

    def gdn(self, l, x):
        """linear_attention_residual (Q/src/decoder.rs:806-938) minus the residual."""
        return self.matvec(f"L{l}.out", self.gdn_core(l, x))

    def gdn_core(self, l, x):
        """The GatedDeltaNet mixer up to out_proj's input (decoder.rs:822-927):
        in-projection split [qkv | z | a | b], conv + SiLU, key-head repeat,
        gates, one delta step, gated RMS norm."""
        p = f"L{l}"
        out = self.matvec(f"{p}.in", x)
        mixed, z = out[:self.C], out[self.C:self.C + self.Vw]
        a = out[self.C + self.Vw:self.C + self.Vw + self.hv]
        b = out[self.C + self.Vw + self.hv:]
        conv = orc.causal_conv_silu_update(mixed, self.conv_state[l], self.w(f"{p}.conv_w")["data"], self.C, self.K)
        rep = self.hv // self.hk
        q = orc.repeat_heads(conv[:self.Kw], self.hk, self.dk, rep)
        k = orc.repeat_heads(conv[self.Kw:2 * self.Kw], self.hk, self.dk, rep)
        ld, beta = orc.gdn_gates(a, b, self.w(f"{p}.a_log")["data"], self.w(f"{p}.dt_bias")["data"])
        core = orc.gated_delta_step(q, k, conv[2 * self.Kw:], ld, beta, self.gdn_state[l], self.hv, self.dk, self.dv)
        return orc.rms_norm_gated(core, z, self.hv, self.dv, self.w(f"{p}.gnorm")["data"], self.eps)

    def mlp(self, prefix, h):
        """decoder_mlp_residual (Q/src/decoder.rs:636-670)."""
        x = self.norm(h, f"{prefix}.mlp_norm")
        gu = self.matvec(f"{prefix}.gate_up", x)
        act = orc.swiglu(gu[:self.I], gu[self.I:])
        return h + self.matvec(f"{prefix}.down", act)

    # -- steps ----------------------------------------------------------------
    def target_step(self, token, retain=False):
        """decode_target_step (Q/src/decoder.rs:956-998): (logits, final hidden)."""
        h = self.embedding(token)
        for l, full in enumerate(self.full):
            x = self.norm(h, f"L{l}.norm")
            d = self.attention(f"L{l}", x, self.position, self.caches[l], retain) if full else self.gdn(l, x)
            h = self.mlp(f"L{l}", h + d)
        fin = self.norm(h, "final_norm")
        self.position += 1
        return self.matvec("lm_head", fin), fin

    def restricted_logits(self, fin, ids):
        """restricted_logits_from_final_hidden (Q/src/decoder.rs:589-627):
        x' = fin * s_in once, then one recovered_row_matvec per token ID."""
        m = self.w("lm_head")
        ids = check_draft_ids(ids, m["rows"])
        s_in = np.frombuffer(m["s_in"].tobytes(), np.float16).astype(np.float32)
        s_out = np.frombuffer(m["s_out"].tobytes(), np.float16).astype(np.float32)
        x = (np.asarray(fin, np.float32) * s_in).astype(np.float32)
        return np.array([orc.recovered_row_matvec(*self._row(m, int(t)), x, float(s_out[t])) for t in ids],
                        np.float32)

    def attention_residual(self, prefix, h, position, cache):
        """full_attention_residual (Q/src/decoder.rs:676-800): the position
        must be the cache's next token."""
        if position != cache.tokens():
            raise orc.OracleError(1)
        return h + self.attention(prefix, self.norm(h, f"{prefix}.norm"), position, cache, False)

    def mtp_fc(self, token, prev):
        """The MTP head's input projection (Q/src/decoder.rs:1027-1036): fc over
        [norm_emb(embedding(token)), norm_hid(prev)], in that order."""
        e = self.norm(self.embedding(token), "mtp.norm_emb")
        hn = self.norm(prev, "mtp.norm_hid")
        return self.matvec("mtp.fc", np.concatenate([e, hn]))

    def mtp(self, token, prev, rope_pos, retain, logits=True):
        """mtp_final_hidden (Q/src/decoder.rs:1009-1046) (+ the shared LM head,
        restricted to the draft vocabulary when one is bound)."""
        if rope_pos != self.mtp_cache.tokens() + 1:  # decoder.rs:1017-1024
            raise orc.OracleError(1)
        h = self.mtp_fc(token, prev)
        x = self.norm(h, "mtp.attn_norm")
        h = self.mlp("mtp", h + self.attention("mtp", x, rope_pos, self.mtp_cache, retain))
        fin = self.norm(h, "mtp.norm")
        if not logits:
            return fin, None
        if self.draft_ids is not None:
            return fin, self.restricted_logits(fin, self.draft_ids)
        return fin, self.matvec("lm_head", fin)

    def decode(self, token):
        """One target step with the prefill-time MTP advance (:1248-1261)."""
        if self.mtp_cache is not None and self.prev_hidden is not None:
            self.mtp(token, self.prev_hidden, self.position, retain=False, logits=False)
        logits, fin = self.target_step(token)
        self.prev_hidden = fin
        return logits

    def _demote_all(self):
        for c in list(self.caches.values()) + ([self.mtp_cache] if self.mtp_cache is not None else []):
            c.demote_old_pages()

    def mtp_step(self, token, temperature, rng: orc.Pcg32, drafts: int):
        """The speculative step described in the module docstring:
        returns (next token, accepted drafts). Temperature 0 is the crate's
        greedy MTP (Q/src/engine.rs:583-590, 915-963): each draft is the
        argmax of its draft row (a restricted row's index mapped to its
        token, decoder.rs:1311-1329), and verify_greedy_mtp accepts the
        longest prefix equal to the target argmax tokens."""
        greedy = temperature == 0.0
        p = self.position
        xs, g = [token], self.prev_hidden
        draft_logits = []
        mtp_after_first = None
        for i in range(drafts):
            g, lg = self.mtp(xs[-1], g, p + i, retain=True)
            if i == 0:
                mtp_after_first = copy.deepcopy(self.mtp_cache)
            draft_logits.append(lg)
            if not np.all(np.isfinite(lg)):
                raise orc.OracleError(8)  # InvalidState, fail closed (cuda_runtime.rs:10627-10632)
            if greedy:
                d = orc.greedy_token(lg)
            else:
                empty = np.zeros((0, lg.size), np.float32)
                d, _ = orc.mtp_accept_sample(empty, empty, lg, np.zeros(0, np.uint32), temperature, rng)
            xs.append(int(self.draft_ids[d]) if self.draft_ids is not None else d)
        saved = (copy.deepcopy(self.gdn_state), copy.deepcopy(self.conv_state), copy.deepcopy(self.caches),
                 self.position)
        target, hiddens = [], []
        for x in xs:
            lg, fin = self.target_step(x, retain=True)
            target.append(lg)
            hiddens.append(fin)
        if greedy:
            if not all(np.all(np.isfinite(t)) for t in target):
                raise orc.OracleError(8)
            # verify_greedy_mtp (engine.rs:915-963) on draft tokens: the
            # compact branch (:928-943), since a restricted draft row has no
            # full-vocabulary argmax of its own.
            nxt, n = verify_greedy_tokens(xs[1:], [orc.greedy_token(t) for t in target])
        else:
            nxt, n = orc.mtp_accept_sample(np.stack(draft_logits), np.stack(target[:drafts]), target[drafts],
                                           np.array(xs[1:], np.uint32), temperature, rng,
                                           draft_ids=self.draft_ids)
        # commit n + 1 target tokens
        self.gdn_state, self.conv_state, self.caches, self.position = saved
        for x in xs[:n + 1]:
            self.target_step(x, retain=True)
        self.mtp_cache = mtp_after_first
        for i in range(1, n + 1):
            self.mtp(xs[i], hiddens[i - 1], p + i, retain=True, logits=False)
        self.prev_hidden = hiddens[n]
        self._demote_all()
        return nxt, xs[1:n + 1], {"draft_logits": draft_logits, "target_logits": target, "drafts": xs[1:]}


# ---------------------------------------------------------------- artifacts
class ArtifactTensors:
    """Tensor provider of OracleDecoder over a `.ctoxq` file written with the
    crate's tensor names (Q/src/tensor_contract.rs:137-244).

    Reads the file independently of the product's loader: the 64-byte header
    (Q/src/format.rs:394-450), the JSON manifest, tensor payloads at
    data_offset + offset. An engine name resolves to the crate tensors the
    crate's decoder reads for it (decoder.rs:687-725 q/k/v fan-out, 806-860
    in_proj_qkv/z/a/b, 636-655 gate/up, 1009-1046 the MTP head), rows
    concatenated in that order; members of any dtype keep their own rows, so
    a fused matrix of several dtypes is a mixed matrix with one segment per
    member run (the crate's fan-out computes the same rows member by member)."""

    DT = {"q2_b64": orc.Q2B64, "q4_b64": orc.Q4B64, "mixed_q2_q4_b64": orc.MIXED, "f16": 3, "f32": 4}

    def __init__(self, path, cfg):
        import json
        import struct
        with open(path, "rb") as f:
            self.raw = f.read()
        if self.raw[:8] != b"CTOXQ2Q4":
            raise orc.OracleError(3)
        _, _, mlen, self.data_offset, _, _ = struct.unpack_from("<IIQQII", self.raw, 8)
        man = json.loads(self.raw[64:64 + mlen])
        self.entries = {t["name"]: t for t in man["tensors"]}
        self.c = cfg

    def _payload(self, e):
        start = self.data_offset + e["offset"]
        return self.raw[start:start + e["length"]]

    def _runs(self, name):
        e = self.entries[name]
        d = self.DT[e["dtype"]]
        if d != orc.MIXED:
            return [(d, e["shape"][0], self._payload(e))]
        p = self._payload(e)
        return [(self.DT[s["dtype"]], s["row_end"] - s["row_start"], p[s["offset"]:s["offset"] + s["length"]])
                for s in e["segments"]]

    def _f32(self, name):
        e = self.entries[name]
        dt = np.float16 if e["dtype"] == "f16" else np.float32
        return np.frombuffer(self._payload(e), dt).astype(np.float32)

    def members(self, name):
        c = self.c
        if name == "embed":
            return ["model.language_model.embed_tokens.weight"]
        if name == "lm_head":
            return ["lm_head.weight"]
        if name == "final_norm":
            return ["model.language_model.norm.weight"]
        if name.startswith("mtp."):
            part, layer, top = name[4:], "mtp.layers.0", {"fc": "mtp.fc.weight", "norm": "mtp.norm.weight",
                                                         "norm_emb": "mtp.pre_fc_norm_embedding.weight",
                                                         "norm_hid": "mtp.pre_fc_norm_hidden.weight"}
            if part in top:
                return [top[part]]
            if part == "attn_norm":
                part = "norm"
        else:
            l, part = name[1:].split(".", 1)
            layer = f"model.language_model.layers.{int(l)}"
        a, g, m = f"{layer}.self_attn", f"{layer}.linear_attn", f"{layer}.mlp"
        return {"norm": [f"{layer}.input_layernorm.weight"], "mlp_norm": [f"{layer}.post_attention_layernorm.weight"],
                "gate_up": [f"{m}.gate_proj.weight", f"{m}.up_proj.weight"], "down": [f"{m}.down_proj.weight"],
                "qkv": [f"{a}.q_proj.weight", f"{a}.k_proj.weight", f"{a}.v_proj.weight"],
                "o": [f"{a}.o_proj.weight"], "q_norm": [f"{a}.q_norm.weight"], "k_norm": [f"{a}.k_norm.weight"],
                "in": [f"{g}.in_proj_qkv.weight", f"{g}.in_proj_z.weight", f"{g}.in_proj_a.weight",
                       f"{g}.in_proj_b.weight"],
                "out": [f"{g}.out_proj.weight"], "conv_w": [f"{g}.conv1d.weight"], "a_log": [f"{g}.A_log"],
                "dt_bias": [f"{g}.dt_bias"], "gnorm": [f"{g}.norm.weight"]}[part]

    def __call__(self, name):
        members = self.members(name)
        first = self.entries[members[0]]
        if first["dtype"] in ("f16", "f32"):
            return {"kind": "f32", "data": self._f32(members[0])}
        runs = [r for m in members for r in self._runs(m)]
        cols = first["shape"][1]
        data, segs, row, off = [], [], 0, 0
        for i, (d, rows, p) in enumerate(runs):
            segs.append((i, row, row + rows, d, off, len(p)))
            data.append(p)
            row, off = row + rows, off + len(p)
        s_in = np.frombuffer(self._payload(self.entries[members[0] + ".s_in"]), np.uint8)
        if any(self._payload(self.entries[m + ".s_in"]) != s_in.tobytes() for m in members[1:]):
            raise orc.OracleError(3)  # fan-out members share one s_in (fanout.rs:77-120)
        s_out = np.frombuffer(b"".join(self._payload(self.entries[m + ".s_out"]) for m in members), np.uint8)
        t = {"kind": "quant", "rows": row, "cols": cols, "data": b"".join(data), "s_in": s_in, "s_out": s_out}
        if len({d for d, _, _ in runs}) == 1:
            t["dtype"] = runs[0][0]
        else:
            t["dtype"], t["segments"] = orc.MIXED, segs
        return t
