"""Loading a `.ctoxq` artifact into the device engine.

Host side of CpuCorrectnessExecutor::load (models/qwen38_27b/src/decoder.rs:
1149-1182) for the device engine: every tensor of the crate's tensor contract
(tensor_contract.rs:137-244) goes to the engine tensor that holds it.

The engine fuses each fan-out group of the crate (fanout.rs:31-70; the
projections that share one FP16 s_in) into one row-concatenated matrix, so a
fused matrix computes exactly the rows the crate's projection_fanout computes
(decoder.rs:700-725, 840-860, 645-655):

* ``L<i>.in``      = linear_attn.in_proj_qkv | in_proj_z | in_proj_a | in_proj_b
* ``L<i>.qkv``     = self_attn.q_proj | k_proj | v_proj (q_proj rows: query and
  gate per head, as the crate splits them)
* ``L<i>.gate_up`` = mlp.gate_proj | up_proj

Each engine matrix holds one packed dtype. A group whose members are all
Q2_B64 stays Q2_B64; otherwise it is Q4_B64 and Q2 rows are widened on the
host, code c -> 5c under the same block scale: the Q2 codebook
{-1, -1/3, 1/3, 1} (quant.rs:151-156) is the Q4 codebook (code - 7.5) / 7.5
(quant.rs:171-175) at codes {0, 5, 10, 15}, so the dequantized values are the
same floats. Norm weights and conv weights (F16) are converted to float32,
which is exact; A_log / dt_bias are F32 already.
"""
from __future__ import annotations

import ctypes
from typing import Dict, Iterable, List, Optional, Sequence, Tuple

import numpy as np

from . import (BLOCK_LEN, Q2_BLOCK_BYTES, Q4_BLOCK_BYTES, HipBackend, InvalidArtifact, ShapeError, TensorDType,
               _check, load_library)
from .artifact import ModelArtifact
from .engine import Engine, EngineConfig

PART_DATA, PART_S_IN, PART_S_OUT = 0, 1, 2


class EngineDtypePlan(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_int32)]


def engine_tensor_sources(config: EngineConfig) -> Dict[str, Tuple[str, List[str]]]:
    """Engine tensor name -> ("matrix" | "vector", crate tensor names in row order)."""
    c = config
    out: Dict[str, Tuple[str, List[str]]] = {
        "embed": ("matrix", ["model.language_model.embed_tokens.weight"]),
        "lm_head": ("matrix", ["lm_head.weight"]),
        "final_norm": ("vector", ["model.language_model.norm.weight"]),
    }

    def attention(engine: str, layer: str) -> None:
        a = f"{layer}.self_attn"
        out[f"{engine}.qkv"] = ("matrix", [f"{a}.q_proj.weight", f"{a}.k_proj.weight", f"{a}.v_proj.weight"])
        out[f"{engine}.o"] = ("matrix", [f"{a}.o_proj.weight"])
        out[f"{engine}.q_norm"] = ("vector", [f"{a}.q_norm.weight"])
        out[f"{engine}.k_norm"] = ("vector", [f"{a}.k_norm.weight"])

    def mlp(engine: str, layer: str) -> None:
        m = f"{layer}.mlp"
        out[f"{engine}.gate_up"] = ("matrix", [f"{m}.gate_proj.weight", f"{m}.up_proj.weight"])
        out[f"{engine}.down"] = ("matrix", [f"{m}.down_proj.weight"])
        out[f"{engine}.mlp_norm"] = ("vector", [f"{layer}.post_attention_layernorm.weight"])

    for l in range(c.num_hidden_layers):
        layer = f"model.language_model.layers.{l}"
        e = f"L{l}"
        out[f"{e}.norm"] = ("vector", [f"{layer}.input_layernorm.weight"])
        mlp(e, layer)
        if (l + 1) % c.full_attention_interval == 0:  # config.rs:62-73
            attention(e, layer)
        else:
            g = f"{layer}.linear_attn"
            out[f"{e}.in"] = ("matrix", [f"{g}.in_proj_qkv.weight", f"{g}.in_proj_z.weight",
                                         f"{g}.in_proj_a.weight", f"{g}.in_proj_b.weight"])
            out[f"{e}.out"] = ("matrix", [f"{g}.out_proj.weight"])
            out[f"{e}.conv_w"] = ("vector", [f"{g}.conv1d.weight"])
            out[f"{e}.a_log"] = ("vector", [f"{g}.A_log"])
            out[f"{e}.dt_bias"] = ("vector", [f"{g}.dt_bias"])
            out[f"{e}.gnorm"] = ("vector", [f"{g}.norm.weight"])
    if c.mtp_layers:
        out["mtp.fc"] = ("matrix", ["mtp.fc.weight"])
        out["mtp.norm"] = ("vector", ["mtp.norm.weight"])
        out["mtp.norm_emb"] = ("vector", ["mtp.pre_fc_norm_embedding.weight"])
        out["mtp.norm_hid"] = ("vector", ["mtp.pre_fc_norm_hidden.weight"])
        out["mtp.attn_norm"] = ("vector", ["mtp.layers.0.input_layernorm.weight"])
        attention("mtp", "mtp.layers.0")
        mlp("mtp", "mtp.layers.0")
    return out


def _row_groups(artifact: ModelArtifact, name: str):
    """(dtype, rows, payload) runs of one crate matrix in row order."""
    m = artifact.quantized_matrix(name)
    if m.dtype in (TensorDType.Q2B64, TensorDType.Q4B64):
        return [(TensorDType(m.dtype), m.rows, m.weights)]
    return [(TensorDType(s.dtype), s.row_end - s.row_start, m.weights[s.offset:s.offset + s.length])
            for s in m.segments]


def widen_q2_rows(payload) -> bytes:
    """Q2_B64 blocks -> Q4_B64 blocks with the same values (code c -> 5c)."""
    b = np.frombuffer(payload, np.uint8).reshape(-1, Q2_BLOCK_BYTES)
    codes = (b[:, 2:, None] >> np.array([0, 2, 4, 6], np.uint8)) & 3
    q4 = (codes.reshape(-1, BLOCK_LEN) * 5).astype(np.uint8)
    out = np.empty((b.shape[0], Q4_BLOCK_BYTES), np.uint8)
    out[:, :2] = b[:, :2]
    out[:, 2:] = q4[:, 0::2] | (q4[:, 1::2] << 4)
    return out.tobytes()


def matrix_dtype(artifact: ModelArtifact, members: Sequence[str]) -> TensorDType:
    dtypes = {d for n in members for d, _, _ in _row_groups(artifact, n)}
    return TensorDType.Q2B64 if dtypes == {TensorDType.Q2B64} else TensorDType.Q4B64


def plan_artifact(artifact: ModelArtifact, config: EngineConfig) -> Dict[str, TensorDType]:
    """Engine matrix name -> packed dtype, after checking that every tensor
    the engine reads is present and each fan-out group shares its s_in bytes
    (verify_recovery_fanout, fanout.rs:77-120); InvalidArtifact otherwise.
    Touches no device."""
    plan = {}
    for name, (kind, members) in engine_tensor_sources(config).items():
        for m in members:
            artifact.tensor(m)
        if kind == "vector":
            continue
        s_in = [bytes(artifact.tensor(f"{m}.s_in").bytes) for m in members]
        if any(s != s_in[0] for s in s_in[1:]):
            raise InvalidArtifact(f"fan-out group {name} has differing s_in scales")
        for m in members:
            for suffix in (".s_in", ".s_out"):
                if artifact.tensor(m + suffix).entry.dtype != TensorDType.F16:
                    raise InvalidArtifact(f"{m}{suffix} is not F16")
        plan[name] = matrix_dtype(artifact, members)
    return plan


def _vector_f32(artifact: ModelArtifact, name: str) -> np.ndarray:
    return np.ascontiguousarray(artifact.float_tensor(name).to_f32_vec(), np.float32)


def load_engine(backend: HipBackend, artifact, config: EngineConfig, draft_ids: Optional[Iterable[int]] = None,
                seed: int = 1) -> Engine:
    """An engine holding the artifact's weights (path or open ModelArtifact).

    Shapes are checked against the engine's tensors; the members of a fan-out
    group must carry identical s_in bytes (verify_recovery_fanout,
    fanout.rs:77-120), else InvalidArtifact. draft_ids binds the release's
    MTP draft vocabulary after the weights."""
    own = not isinstance(artifact, ModelArtifact)
    art = ModelArtifact.open(artifact) if own else artifact
    lib = load_library()
    eng = None
    try:
        sources = engine_tensor_sources(config)
        plan = list(plan_artifact(art, config).items())
        keep = [n.encode() for n, _ in plan]
        arr = (EngineDtypePlan * len(plan))(*[EngineDtypePlan(k, int(d)) for k, (_, d) in zip(keep, plan)])
        h = ctypes.c_void_p()
        _check(lib.ctox_hip_engine_create_with_dtypes(backend.handle, ctypes.byref(config), seed, arr, len(plan),
                                                      ctypes.byref(h)))
        eng = Engine.__new__(Engine)
        eng.backend, eng.config, eng.handle = backend, config, h.value
        dtypes = dict(plan)

        write = eng.write
        for name, (kind, members) in sources.items():
            view = eng.tensor_info(name)
            if kind == "vector":
                v = _vector_f32(art, members[0])
                if v.size != view["cols"]:
                    raise ShapeError(f"{members[0]} has {v.size} values, the engine's {name} holds {view['cols']}")
                write(name, PART_DATA, 0, v)
                continue
            dtype = dtypes[name]
            rows = sum(art.quantized_matrix(m).rows for m in members)
            for m in members:
                if art.quantized_matrix(m).columns != view["cols"]:
                    raise ShapeError(f"{m} has {art.quantized_matrix(m).columns} columns, "
                                     f"the engine's {name} {view['cols']}")
            if rows != view["rows"] or int(dtype) != view["dtype"]:
                raise ShapeError(f"{name}: members give {rows} rows, the engine holds {view['rows']}")
            write(name, PART_S_IN, 0, bytes(art.tensor(f"{members[0]}.s_in").bytes))
            offset, s_out_offset = 0, 0
            for m in members:
                s_out = art.tensor(f"{m}.s_out")
                write(name, PART_S_OUT, s_out_offset, bytes(s_out.bytes))
                s_out_offset += len(s_out.bytes)
                for d, _, payload in _row_groups(art, m):
                    data = widen_q2_rows(payload) if d == TensorDType.Q2B64 and dtype == TensorDType.Q4B64 \
                        else bytes(payload)
                    write(name, PART_DATA, offset, data)
                    offset += len(data)
        eng.finish_load()
        if draft_ids is not None:
            eng.set_draft_vocab(list(draft_ids))
        return eng
    except BaseException:
        if eng is not None:
            eng.close()
        raise
    finally:
        if own:
            art.close()
