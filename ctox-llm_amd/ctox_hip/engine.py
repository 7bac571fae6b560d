"""Python handle of the device-resident decode engine (include/ctox_hip.h,
ctox_hip_engine_*): the crate's model graph (Q/src/decoder.rs) and MTP
executor on one GPU, driven from the host one step at a time."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, fields
from typing import List, Optional, Tuple

import numpy as np

from . import HipBackend, _check, load_library

_P, _SZ, _U32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32


class EngineConfig(ctypes.Structure):
    """ctox_engine_config; defaults are Qwen38Config (Q/src/config.rs:35-59)
    with BASELINE's vocabulary, page size and a 4-draft MTP head."""
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "hidden_size", "intermediate_size", "num_hidden_layers", "full_attention_interval",
        "num_attention_heads", "num_key_value_heads", "head_dim", "rotary_dim",
        "linear_num_key_heads", "linear_num_value_heads", "linear_key_head_dim", "linear_value_head_dim",
        "linear_conv_kernel_dim", "vocab_size", "max_tokens", "page_tokens", "sink_tokens", "recent_tokens",
        "mtp_layers", "draft_tokens")] + [("rms_norm_epsilon", ctypes.c_float), ("rope_theta", ctypes.c_float)]

    @classmethod
    def qwen38_27b(cls, max_tokens: int = 33024, vocab: int = 151936, page_tokens: int = 16, drafts: int = 4):
        return cls(5120, 17408, 64, 4, 24, 4, 256, 64, 16, 48, 128, 128, 4, vocab, max_tokens, page_tokens, 128,
                   256, 1 if drafts else 0, drafts, 1e-6, 1e7)

    def as_dict(self):
        return {f[0]: getattr(self, f[0]) for f in self._fields_}


class EngineTensor(ctypes.Structure):
    _fields_ = [("data", _P), ("bytes", _SZ), ("rows", _U32), ("cols", _U32), ("dtype", ctypes.c_int32),
                ("pad", _U32), ("s_in", _P), ("s_out", _P)]


class EngineCacheView(ctypes.Structure):
    _fields_ = [("descriptors", _P), ("pages", _U32), ("tokens", _U32), ("d_q4_pool", _P), ("d_q2_pool", _P),
                ("q4_page_bytes", _U32), ("q2_page_bytes", _U32)]


_hiprt = None


def _d2h(ptr: int, nbytes: int) -> np.ndarray:
    """Device-to-host copy through the HIP runtime the library already uses."""
    global _hiprt
    if _hiprt is None:
        _hiprt = ctypes.CDLL("libamdhip64.so")
        _hiprt.hipMemcpy.argtypes = [_P, _P, _SZ, ctypes.c_int]
        _hiprt.hipDeviceSynchronize.argtypes = []
    out = np.empty(nbytes, dtype=np.uint8)
    if _hiprt.hipMemcpy(out.ctypes.data, ptr, nbytes, 2) != 0:
        raise RuntimeError("hipMemcpy device-to-host failed")
    return out


def _lib():
    return load_library()


class Engine:
    def __init__(self, backend: HipBackend, config: EngineConfig, seed: int = 1):
        self.backend, self.config = backend, config
        h = _P()
        _check(_lib().ctox_hip_engine_create(backend.handle, ctypes.byref(config), seed, ctypes.byref(h)))
        self.handle = h.value

    def close(self) -> None:
        if self.handle:
            _lib().ctox_hip_engine_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- steps ---------------------------------------------------------------
    def set_rng(self, state: int) -> None:
        _check(_lib().ctox_hip_engine_set_rng(self.handle, state))

    def decode(self, token: int) -> None:
        p = _P()
        _check(_lib().ctox_hip_engine_decode(self.handle, token, ctypes.byref(p)))

    def mtp_step(self, token: int, temperature: float) -> Tuple[int, List[int]]:
        out = (_U32 * 16)()
        _check(_lib().ctox_hip_engine_mtp_step(self.handle, token, temperature, out))
        n = out[1]
        return out[0], [out[2 + i] for i in range(n)]

    def set_draft_vocab(self, ids) -> None:
        """Binds the MTP draft vocabulary (strictly increasing token IDs)."""
        a = np.ascontiguousarray(ids, dtype=np.uint32)
        _check(_lib().ctox_hip_engine_set_draft_vocab(self.handle, a.ctypes.data, a.size))
        self.draft_n = int(a.size)

    def fill_context(self, tokens: int, seed: int = 7) -> None:
        _check(_lib().ctox_hip_engine_fill_context(self.handle, tokens, seed))

    @property
    def position(self) -> int:
        return _lib().ctox_hip_engine_position(self.handle)

    @property
    def stream(self) -> int:
        return _lib().ctox_hip_engine_stream(self.handle)

    # -- views ---------------------------------------------------------------
    def buffer(self, which: int) -> Tuple[int, int]:
        p, n = _P(), _SZ()
        _check(_lib().ctox_hip_engine_buffer(self.handle, which, ctypes.byref(p), ctypes.byref(n)))
        return p.value, n.value

    def read(self, which: int, count: Optional[int] = None) -> np.ndarray:
        ptr, n = self.buffer(which)
        nbytes = n if count is None else count * 4
        return _d2h(ptr, nbytes).view(np.float32)

    def logits(self, rows: int = 1) -> np.ndarray:
        return self.read(0, rows * self.config.vocab_size).reshape(rows, -1)

    def cache_pages(self, layer: int):
        """Pages of a full-attention layer's cache (layer -1: the MTP cache):
        [(precision, tokens, first_token, bytes)] in page order; bytes hold
        `tokens` token rows of the page's precision."""
        v = EngineCacheView()
        _check(_lib().ctox_hip_engine_cache(self.handle, 0xffffffff if layer < 0 else layer, ctypes.byref(v)))
        desc = np.ctypeslib.as_array((_U32 * (4 * v.pages)).from_address(v.descriptors)).reshape(-1, 4).copy() \
            if v.pages else np.zeros((0, 4), np.uint32)
        kvw = 2 * self.config.num_key_value_heads * self.config.head_dim
        out = []
        for prec, slot, tokens, first in desc:
            tb = kvw // 64 * (34 if prec else 18)
            pool, pb = (v.d_q4_pool, v.q4_page_bytes) if prec else (v.d_q2_pool, v.q2_page_bytes)
            out.append((int(prec), int(tokens), int(first), _d2h(pool + int(slot) * pb, int(tokens) * tb).tobytes()))
        return out

    def write(self, name: str, part: int, offset: int, data) -> None:
        """Copies host bytes into part `part` (0 data, 1 s_in, 2 s_out) of a
        named tensor at byte `offset`; steps wait for finish_load."""
        buf = np.ascontiguousarray(data if isinstance(data, np.ndarray) else np.frombuffer(data, np.uint8))
        _check(_lib().ctox_hip_engine_write(self.handle, name.encode(), part, offset, buf.ctypes.data, buf.nbytes))

    def finish_load(self) -> None:
        _check(_lib().ctox_hip_engine_finish_load(self.handle))

    def tensor_info(self, name: str) -> dict:
        """Geometry of one weight without copying it: rows, cols, dtype (-1: f32 vector)."""
        t = EngineTensor()
        _check(_lib().ctox_hip_engine_tensor(self.handle, name.encode(), ctypes.byref(t)))
        return {"rows": t.rows, "cols": t.cols, "dtype": t.dtype, "bytes": t.bytes}

    def tensor(self, name: str) -> dict:
        """Host copy of one weight: quantized matrices as raw blocks plus fp16
        s_in / s_out bytes, vectors as float32."""
        t = EngineTensor()
        _check(_lib().ctox_hip_engine_tensor(self.handle, name.encode(), ctypes.byref(t)))
        raw = _d2h(t.data, t.bytes)
        if t.dtype < 0:
            return {"kind": "f32", "data": raw.view(np.float32).copy()}
        return {"kind": "quant", "dtype": t.dtype, "rows": t.rows, "cols": t.cols, "data": raw.tobytes(),
                "s_in": _d2h(t.s_in, 2 * t.cols), "s_out": _d2h(t.s_out, 2 * t.rows)}
