"""The C-ABI library loads and exports every symbol include/ctox_hip.h
declares; the Python binding's signature table covers exactly those."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "ctox_hip.h")).read()
    return set(re.findall(r"\b(ctox_hip_\w+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    import ctox_hip
    lib = ctox_hip.load_library()
    syms = declared_symbols()
    assert len(syms) >= 20
    for s in sorted(syms):
        assert hasattr(lib, s), s
    assert syms == set(ctox_hip.SIGNATURES)


def test_library_embeds_a_gfx950_code_object():
    import ctox_hip
    blob = open(ctox_hip.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
    for k in ("ctox_q4_matvec_b1_gfx950", "ctox_q2_matvec_b1_gfx950", "ctox_q4_matvec_sl_gfx950", "ctox_q2_matvec_sl3_gfx950", "ctox_q4_matvec_b4_gfx950", "ctox_q2_matvec_b8_gfx950", "ctox_prep_activation_gfx950",
              "ctox_gdn_scan_gfx950"):
        assert k.encode() in blob


def test_backend_creation_fails_closed_without_a_gpu():
    import torch
    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is present")
    import ctox_hip
    with pytest.raises(ctox_hip.UnsupportedOperation):
        ctox_hip.HipBackend(0)


def test_oracle_is_not_reachable_from_the_product():
    pkg = os.path.join(ROOT, "ctox-llm_amd")
    for dp, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h")):
                text = open(os.path.join(dp, f)).read()
                assert "libctox_oracle" not in text and "import oracle" not in text and "from oracle" not in text, f
