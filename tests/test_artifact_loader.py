"""Host side of loading a `.ctoxq` artifact into the engine (ctox_hip.loader)
and the oracle's own artifact reader (oracle.decoder.ArtifactTensors).

* The tensor map covers the crate's tensor contract exactly: every tensor
  the contract names (tensor_contract.rs:137-244, written by
  tests/artifact_model.py) is read by one engine tensor, none twice.
* Widening Q2 rows to Q4 keeps every dequantized value (oracle q2_value vs
  q4_value on all codes and random scales).
* A fused engine matrix computes the crate's fan-out: the oracle's fused
  matvec equals the concatenation of per-member matvecs, each member read
  through the product's ModelArtifact with its own dtype / segments.
* Fan-out members with differing s_in, and a missing tensor, are refused
  before any device work.
"""
import numpy as np
import pytest

from artifact_model import contract, write_artifact


def small_config(**kw):
    from ctox_hip.engine import EngineConfig
    c = EngineConfig(256, 512, 4, 4, 2, 1, 256, 64, 2, 4, 64, 64, 4, 512, 512, 16, 16, 32, 1, 4, 1e-6, 1e7)
    for k, v in kw.items():
        setattr(c, k, v)
    return c


MIXED = {
    "model.language_model.layers.0.linear_attn.in_proj_qkv.weight": "q4",
    "model.language_model.layers.0.linear_attn.in_proj_z.weight": "q2",
    "model.language_model.layers.0.linear_attn.in_proj_a.weight": "mixed",
    "model.language_model.layers.1.mlp.gate_proj.weight": "q2",
    "model.language_model.layers.1.mlp.up_proj.weight": "q2",
    "model.language_model.layers.2.mlp.down_proj.weight": "q4",
    "model.language_model.layers.3.self_attn.q_proj.weight": "q2",
    "model.language_model.layers.3.self_attn.k_proj.weight": "q2",
    "model.language_model.layers.3.self_attn.v_proj.weight": "q2",
    "model.language_model.layers.3.mlp.down_proj.weight": "mixed",
    "model.language_model.embed_tokens.weight": "q2",
    "lm_head.weight": "mixed",
    "mtp.fc.weight": "mixed",
    "mtp.layers.0.mlp.gate_proj.weight": "mixed",
}


def test_tensor_map_covers_contract():
    from ctox_hip.loader import engine_tensor_sources
    for c in (small_config(), small_config(mtp_layers=0), small_config(num_hidden_layers=8)):
        read = [m for _, members in engine_tensor_sources(c).values() for m in members]
        assert len(read) == len(set(read))
        quant = {n for n, k, _, _ in contract(c) if k == "quant"}
        assert set(read) == {n for n, _, _, _ in contract(c)}
        assert quant <= set(read)


def test_widen_q2_rows_keeps_values(orc):
    from ctox_hip.loader import widen_q2_rows
    rng = np.random.default_rng(4)
    blocks = bytearray(rng.integers(0, 256, 18 * 8, dtype=np.uint8).tobytes())
    for b in range(8):  # finite scales, one of them negative
        blocks[18 * b:18 * b + 2] = np.float16(rng.normal(0, 0.05) * (-1 if b == 3 else 1)).tobytes()
    blocks[2:18] = bytes(range(0, 256, 16))  # every code in block 0
    wide = widen_q2_rows(bytes(blocks))
    assert len(wide) == 34 * 8
    for b in range(8):
        q2, q4 = bytes(blocks[18 * b:18 * (b + 1)]), wide[34 * b:34 * (b + 1)]
        for i in range(64):
            assert orc.q2_value(q2, i) == orc.q4_value(q4, i)


def test_oracle_fused_matrices_equal_member_fanout(orc, tmp_path):
    from ctox_hip.artifact import ModelArtifact
    from oracle.decoder import ArtifactTensors, OracleDecoder
    c = small_config()
    path = tmp_path / "m.ctoxq"
    write_artifact(path, c, MIXED, seed=1)
    dec = OracleDecoder(c.as_dict(), ArtifactTensors(path, c.as_dict()))
    art = ModelArtifact.open(path)
    rng = np.random.default_rng(2)
    try:
        pre = "model.language_model.layers"
        cases = {"L0.in": [f"{pre}.0.linear_attn.in_proj_{p}.weight" for p in ("qkv", "z", "a", "b")],
                 "L3.qkv": [f"{pre}.3.self_attn.{p}_proj.weight" for p in "qkv"],
                 "L1.gate_up": [f"{pre}.1.mlp.{p}_proj.weight" for p in ("gate", "up")],
                 "L3.down": [f"{pre}.3.mlp.down_proj.weight"],
                 "lm_head": ["lm_head.weight"], "mtp.fc": ["mtp.fc.weight"],
                 "mtp.gate_up": [f"mtp.layers.0.mlp.{p}_proj.weight" for p in ("gate", "up")]}
        for name, members in cases.items():
            m = art.quantized_matrix(members[0])
            x = rng.normal(0, 1, m.columns).astype(np.float32)
            want = []
            for n in members:
                q = art.quantized_matrix(n)
                segs = [(s.group_index, s.row_start, s.row_end, int(s.dtype), s.offset, s.length)
                        for s in q.segments]
                want.append(orc.MatVec(int(q.dtype), bytes(q.weights), q.rows, q.columns, x,
                                       s_in=("f16le", np.frombuffer(bytes(art.tensor(n + ".s_in").bytes), np.uint8)),
                                       s_out=("f16le", np.frombuffer(bytes(art.tensor(n + ".s_out").bytes), np.uint8)),
                                       segments=segs).run())
            np.testing.assert_array_equal(dec.matvec(name, x), np.concatenate(want))
        # embedding rows of a Q2 matrix and restricted-head rows of a mixed one
        e = dec.embedding(7)
        assert e.shape == (c.hidden_size,) and np.all(np.isfinite(e))
        fin = rng.normal(0, 1, c.hidden_size).astype(np.float32)
        full = dec.matvec("lm_head", fin)
        ids = [0, 5, 200, 511]
        np.testing.assert_allclose(dec.restricted_logits(fin, ids), full[ids], rtol=1e-5, atol=1e-5)
        # vectors: F16 norm weights and the [C, 1, K] conv weight, as float32
        conv = dec.w("L0.conv_w")["data"]
        assert conv.dtype == np.float32 and conv.size == (2 * 2 * 64 + 4 * 64) * 4
    finally:
        art.close()


def test_plan_and_refusals(tmp_path):
    from ctox_hip import InvalidArtifact, TensorDType
    from ctox_hip.artifact import ArtifactBuilder, ModelArtifact, PackedTensor
    from ctox_hip.loader import plan_artifact
    c = small_config()
    path = tmp_path / "m.ctoxq"
    write_artifact(path, c, MIXED, seed=1)
    art = ModelArtifact.open(path)
    try:
        plan = plan_artifact(art, c)
        Q2, Q4 = TensorDType.Q2B64, TensorDType.Q4B64
        assert plan["L0.in"] == Q4 and plan["L1.gate_up"] == Q2 and plan["L3.qkv"] == Q2
        assert plan["L2.down"] == Q4 and plan["L0.down"] == Q2 and plan["L3.down"] == Q4
        assert plan["embed"] == Q2 and plan["lm_head"] == Q4 and plan["mtp.fc"] == Q4
        tensors = [PackedTensor(t.name, t.dtype, t.shape, bytes(art.tensor(t.name).bytes), t.segments)
                   for t in art.manifest.tensors]
    finally:
        art.close()
    # a fan-out member with its own s_in
    bad = []
    for t in tensors:
        if t.name == "model.language_model.layers.1.mlp.up_proj.weight.s_in":
            t = PackedTensor(t.name, t.dtype, t.shape, np.full(t.shape[0], 1.0, np.float16).tobytes())
        bad.append(t)
    p2 = tmp_path / "bad_s_in.ctoxq"
    ArtifactBuilder("Qwen/Qwen3.6-27B", "synthetic", "logical", tensors=bad).write_new(p2)
    with _closing(ModelArtifact.open(p2)) as a2:
        with pytest.raises(InvalidArtifact, match="s_in"):
            plan_artifact(a2, c)
    # a missing tensor
    p3 = tmp_path / "missing.ctoxq"
    ArtifactBuilder("Qwen/Qwen3.6-27B", "synthetic", "logical",
                    tensors=[t for t in tensors if t.name != "mtp.pre_fc_norm_hidden.weight"]).write_new(p3)
    with _closing(ModelArtifact.open(p3)) as a3:
        with pytest.raises(InvalidArtifact, match="no tensor named"):
            plan_artifact(a3, c)


class _closing:
    def __init__(self, a):
        self.a = a

    def __enter__(self):
        return self.a

    def __exit__(self, *exc):
        self.a.close()
