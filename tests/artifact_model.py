"""Writes a synthetic `.ctoxq` model artifact under the crate's tensor names
(models/qwen38_27b/src/tensor_contract.rs:137-244) for a given engine
configuration: random packed Q2/Q4 blocks, FP16 s_in / s_out in
U(0.75, 1.25) with one s_in per fan-out group (fanout.rs:31-70), FP16 norm
and conv weights, F32 A_log / dt_bias.

`dtypes` picks the packed dtype per crate matrix name: "q2", "q4" or "mixed"
(alternating Q4 / Q2 row segments); the default is Q4 for projections and
Q2 for down projections.
"""
from __future__ import annotations

import numpy as np


def _blocks(rng, rows, cols, dtype):
    nb = rows * (cols // 64)
    width = 34 if dtype == "q4" else 18
    out = np.empty((nb, width), np.uint8)
    out[:, :2] = np.abs(rng.normal(0.0, 0.02, nb)).astype(np.float16).view(np.uint8).reshape(nb, 2)
    out[:, 2:] = rng.integers(0, 256, (nb, width - 2), dtype=np.uint8)
    return out.tobytes()


def contract(c):
    """[(name, kind, shape, group)] with kind "quant" | "f16" | "f32"; group
    names the fan-out group whose s_in the matrix shares."""
    H, I = c.hidden_size, c.intermediate_size
    q, kv = c.num_attention_heads * c.head_dim, c.num_key_value_heads * c.head_dim
    kw = c.linear_num_key_heads * c.linear_key_head_dim
    vw = c.linear_num_value_heads * c.linear_value_head_dim
    conv = 2 * kw + vw
    out = [("model.language_model.embed_tokens.weight", "quant", (c.vocab_size, H), None),
           ("lm_head.weight", "quant", (c.vocab_size, H), None)]

    def attention(a):
        return [(f"{a}.q_proj.weight", "quant", (2 * q, H), f"{a}.qkv"),
                (f"{a}.k_proj.weight", "quant", (kv, H), f"{a}.qkv"),
                (f"{a}.v_proj.weight", "quant", (kv, H), f"{a}.qkv"),
                (f"{a}.o_proj.weight", "quant", (H, q), None),
                (f"{a}.q_norm.weight", "f16", (c.head_dim,), None),
                (f"{a}.k_norm.weight", "f16", (c.head_dim,), None)]

    def mlp(m):
        return [(f"{m}.gate_proj.weight", "quant", (I, H), f"{m}.gu"),
                (f"{m}.up_proj.weight", "quant", (I, H), f"{m}.gu"),
                (f"{m}.down_proj.weight", "quant", (H, I), None)]

    def norms(p):
        return [(f"{p}.input_layernorm.weight", "f16", (H,), None),
                (f"{p}.post_attention_layernorm.weight", "f16", (H,), None)]

    for l in range(c.num_hidden_layers):
        p = f"model.language_model.layers.{l}"
        out += norms(p) + mlp(f"{p}.mlp")
        if (l + 1) % c.full_attention_interval == 0:
            out += attention(f"{p}.self_attn")
        else:
            g = f"{p}.linear_attn"
            out += [(f"{g}.in_proj_qkv.weight", "quant", (conv, H), f"{g}.in"),
                    (f"{g}.in_proj_z.weight", "quant", (vw, H), f"{g}.in"),
                    (f"{g}.in_proj_a.weight", "quant", (c.linear_num_value_heads, H), f"{g}.in"),
                    (f"{g}.in_proj_b.weight", "quant", (c.linear_num_value_heads, H), f"{g}.in"),
                    (f"{g}.out_proj.weight", "quant", (H, vw), None),
                    (f"{g}.conv1d.weight", "f16", (conv, 1, c.linear_conv_kernel_dim), None),
                    (f"{g}.A_log", "f32", (c.linear_num_value_heads,), None),
                    (f"{g}.dt_bias", "f32", (c.linear_num_value_heads,), None),
                    (f"{g}.norm.weight", "f16", (c.linear_value_head_dim,), None)]
    out.append(("model.language_model.norm.weight", "f16", (H,), None))
    if c.mtp_layers:
        out.append(("mtp.fc.weight", "quant", (H, 2 * H), None))
        out += norms("mtp.layers.0") + mlp("mtp.layers.0.mlp") + attention("mtp.layers.0.self_attn")
        out += [(n, "f16", (H,), None) for n in ("mtp.norm.weight", "mtp.pre_fc_norm_embedding.weight",
                                                 "mtp.pre_fc_norm_hidden.weight")]
    return out


def write_artifact(path, c, dtypes=None, seed=0):
    from ctox_hip import QuantSegment, TensorDType
    from ctox_hip.artifact import ArtifactBuilder, PackedTensor
    dtypes = dtypes or {}
    rng = np.random.default_rng(seed)
    group_s_in = {}
    tensors = []
    for name, kind, shape, group in contract(c):
        if kind == "f16":
            tensors.append(PackedTensor(name, TensorDType.F16, shape,
                                        rng.normal(0.0, 0.1, int(np.prod(shape))).astype(np.float16).tobytes()))
            continue
        if kind == "f32":
            lo, hi = (-1.0, 0.5) if name.endswith("A_log") else (-0.5, 0.5)
            tensors.append(PackedTensor(name, TensorDType.F32, shape,
                                        rng.uniform(lo, hi, shape[0]).astype(np.float32).tobytes()))
            continue
        rows, cols = shape
        d = dtypes.get(name, "q2" if "down_proj" in name else "q4")
        if d == "mixed":
            cuts = sorted({0, rows} | {int(x) for x in np.linspace(0, rows, 4)[1:-1]})
            payload, segs, off = [], [], 0
            for i, (a, b) in enumerate(zip(cuts, cuts[1:])):
                sd = "q4" if i % 2 == 0 else "q2"
                p = _blocks(rng, b - a, cols, sd)
                segs.append(QuantSegment(i, a, b, TensorDType.Q4B64 if sd == "q4" else TensorDType.Q2B64,
                                         off, len(p)))
                payload.append(p)
                off += len(p)
            tensors.append(PackedTensor(name, TensorDType.MixedQ2Q4B64, shape, b"".join(payload), segs))
        else:
            tensors.append(PackedTensor(name, TensorDType.Q4B64 if d == "q4" else TensorDType.Q2B64, shape,
                                        _blocks(rng, rows, cols, d)))
        if group is None or group not in group_s_in:
            s_in = rng.uniform(0.75, 1.25, cols).astype(np.float16).tobytes()
            if group is not None:
                group_s_in[group] = s_in
        else:
            s_in = group_s_in[group]
        tensors.append(PackedTensor(f"{name}.s_in", TensorDType.F16, (cols,), s_in))
        tensors.append(PackedTensor(f"{name}.s_out", TensorDType.F16, (rows,),
                                    rng.uniform(0.75, 1.25, rows).astype(np.float16).tobytes()))
    ArtifactBuilder("Qwen/Qwen3.6-27B", "synthetic", "logical", tensors=tensors).write_new(path)
