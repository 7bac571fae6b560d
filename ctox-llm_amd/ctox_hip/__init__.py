"""Python binding of the MI355X HIP backend (include/ctox_hip.h).

Mirrors the crate's backend API (Q/src/backend/mod.rs:54-169 in the
reference tree, Q/ = models/qwen38_27b/): `FusedMatVec`, `ScaleSlice`,
`Activation`, `TensorDType`, `QuantSegment`, `RecoveredRow`,
`RecoveredRowMatVec` and a `HipBackend` with `fused_matvec`,
`fused_matvec_fanout`, `recovered_row` and `recovered_row_matvec`, plus the
gated-delta entry points of Q/src/reference.rs:230-415. Errors raise the
`EngineError` subclass matching Q/src/error.rs.

The binding only loads `lib/libctox_hip.so`; it never computes anything
itself and has no CPU fallback. A missing library raises ImportError-free
`EngineError`s only when a backend is created, so the module can be imported
(and its symbols inspected) on machines without a GPU.
"""
from __future__ import annotations

import ctypes
import enum
import os
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "lib", "libctox_hip.so")


# ---------------------------------------------------------------- errors
class EngineError(Exception):
    """Base of the error kinds of Q/src/error.rs."""

    code = -1


class IoError(EngineError):
    code = 1


class JsonError(EngineError):
    code = 2


class InvalidArtifact(EngineError):
    code = 3


class UnsupportedDType(EngineError):
    code = 4


class UnsupportedOperation(EngineError):
    code = 5


class MemoryBudget(EngineError):
    code = 6


class ShapeError(EngineError):
    code = 7


class InvalidState(EngineError):
    code = 8


class Cancelled(EngineError):
    code = 9


_ERRORS = {c.code: c for c in (IoError, JsonError, InvalidArtifact, UnsupportedDType,
                               UnsupportedOperation, MemoryBudget, ShapeError, InvalidState,
                               Cancelled)}


# ---------------------------------------------------------------- enums
class TensorDType(enum.IntEnum):
    Q2B64 = 0
    Q4B64 = 1
    MixedQ2Q4B64 = 2
    F16 = 3
    F32 = 4


class Activation(enum.IntEnum):
    Identity = 0
    Silu = 1


BLOCK_LEN = 64
Q2_BLOCK_BYTES = 18
Q4_BLOCK_BYTES = 34
MAX_BATCH = 8


@dataclass(frozen=True)
class ScaleSlice:
    """Option<ScaleSlice>: `F32(values)` or `F16Le(bytes)` (Q/src/backend/mod.rs:74-112)."""

    kind: str  # "f32" | "f16le"
    data: np.ndarray

    @staticmethod
    def F32(values) -> "ScaleSlice":
        return ScaleSlice("f32", np.ascontiguousarray(values, dtype=np.float32))

    @staticmethod
    def F16Le(raw) -> "ScaleSlice":
        arr = np.frombuffer(bytes(raw), dtype=np.uint8) if not isinstance(raw, np.ndarray) \
            else np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
        return ScaleSlice("f16le", arr)

    def __len__(self) -> int:
        return len(self.data) if self.kind == "f32" else len(self.data) // 2


@dataclass(frozen=True)
class QuantSegment:
    group_index: int
    row_start: int
    row_end: int
    dtype: TensorDType
    offset: int
    length: int


@dataclass
class FusedMatVec:
    """Q/src/backend/mod.rs:115-128."""

    dtype: TensorDType
    weights: np.ndarray
    rows: int
    columns: int
    input: Optional[np.ndarray] = None
    segments: Sequence[QuantSegment] = field(default_factory=tuple)
    s_in: Optional[ScaleSlice] = None
    s_out: Optional[ScaleSlice] = None
    bias: Optional[np.ndarray] = None
    activation: Activation = Activation.Identity


@dataclass
class RecoveredRow:
    dtype: TensorDType
    weights: np.ndarray
    columns: int
    s_in: ScaleSlice
    s_out: float


@dataclass
class RecoveredRowMatVec:
    dtype: TensorDType
    weights: np.ndarray
    corrected_input: np.ndarray
    s_out: float


# ---------------------------------------------------------------- C structs
class _Scale(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("data", ctypes.c_void_p), ("len", ctypes.c_size_t)]


class _Segment(ctypes.Structure):
    _fields_ = [("group_index", ctypes.c_uint32), ("row_start", ctypes.c_uint64),
                ("row_end", ctypes.c_uint64), ("dtype", ctypes.c_int32),
                ("offset", ctypes.c_uint64), ("length", ctypes.c_uint64)]


class _FusedMatVec(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int32), ("weights", ctypes.c_void_p),
                ("weights_len", ctypes.c_size_t), ("segments", ctypes.POINTER(_Segment)),
                ("n_segments", ctypes.c_size_t), ("rows", ctypes.c_size_t),
                ("columns", ctypes.c_size_t), ("input", ctypes.c_void_p),
                ("input_len", ctypes.c_size_t), ("s_in", _Scale), ("s_out", _Scale),
                ("bias", ctypes.c_void_p), ("bias_len", ctypes.c_size_t),
                ("activation", ctypes.c_int32)]


class _RecoveredRow(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int32), ("weights", ctypes.c_void_p),
                ("weights_len", ctypes.c_size_t), ("columns", ctypes.c_size_t),
                ("s_in", _Scale), ("s_out", ctypes.c_float)]


class _RecoveredRowMatVec(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int32), ("weights", ctypes.c_void_p),
                ("weights_len", ctypes.c_size_t), ("corrected_input", ctypes.c_void_p),
                ("len", ctypes.c_size_t), ("s_out", ctypes.c_float)]


class PagedGqaParams(ctypes.Structure):
    """ctox_paged_gqa_params (CtoxPagedGqaParams, q2q4_fused_matvec_sm86.cu:1621-1634)."""
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "query_heads", "key_value_heads", "head_dim", "tokens", "page_tokens", "page_count", "combined_values",
        "q2_token_bytes", "q4_token_bytes", "q2_page_bytes", "q4_page_bytes")] + [("scale", ctypes.c_float)]


# Every symbol include/ctox_hip.h declares: name -> (restype, argtypes).
_P = ctypes.c_void_p
_SZ = ctypes.c_size_t
_U32 = ctypes.c_uint32
_I32 = ctypes.c_int32
SIGNATURES = {
    "ctox_hip_backend_create": (_I32, [ctypes.c_int, ctypes.POINTER(_P)]),
    "ctox_hip_backend_destroy": (None, [_P]),
    "ctox_hip_backend_kind": (ctypes.c_char_p, [_P]),
    "ctox_hip_backend_promotion_state": (ctypes.c_char_p, [_P]),
    "ctox_hip_backend_profile": (ctypes.c_char_p, [_P]),
    "ctox_hip_last_error": (ctypes.c_char_p, []),
    "ctox_hip_synchronize": (_I32, [_P]),
    "ctox_hip_fused_matvec": (_I32, [_P, ctypes.POINTER(_FusedMatVec), _P, _SZ]),
    "ctox_hip_fused_matvec_fanout": (_I32, [_P, ctypes.POINTER(_FusedMatVec), _SZ, ctypes.POINTER(_P)]),
    "ctox_hip_recovered_row": (_I32, [_P, ctypes.POINTER(_RecoveredRow), _P, _SZ]),
    "ctox_hip_recovered_row_matvec": (_I32, [_P, ctypes.POINTER(_RecoveredRowMatVec), _P]),
    "ctox_hip_matrix_prepare": (_I32, [_P, ctypes.POINTER(_FusedMatVec), ctypes.POINTER(_P)]),
    "ctox_hip_matrix_destroy": (None, [_P]),
    "ctox_hip_matrix_rows": (_SZ, [_P]),
    "ctox_hip_matrix_columns": (_SZ, [_P]),
    "ctox_hip_matrix_device_weights": (_P, [_P]),
    "ctox_hip_matrix_dispatch": (_I32, [_P, _P, _P, _SZ, _P, _P]),
    "ctox_hip_matrix_dispatch_fanout": (_I32, [_P, ctypes.POINTER(_P), _SZ, _P, _SZ, ctypes.POINTER(_P), _P]),
    "ctox_hip_launch_fused_matvec": (_I32, [_P, _I32, _P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _P]),
    "ctox_hip_register_tiled_weights": (_I32, [_P, _I32, _P, _U32, _U32, _P]),
    "ctox_hip_launch_fused_matvec_noalloc": (_I32, [_P, _I32, _P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _P]),
    "ctox_hip_gdn_fused_device": (_I32, [_P, _P, _SZ, _SZ, _SZ, _P, _P, _P, _SZ, _P, _P, _P, _P, ctypes.c_int, _P,
                                         _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P]),
    "ctox_hip_unregister_tiled_weights": (None, [_P, _P]),
    "ctox_hip_gated_delta_step": (_I32, [_P, _P, _P, _P, _P, _P, _P, _SZ, _SZ, _SZ, _P]),
    "ctox_hip_gated_delta_sequence": (_I32, [_P, _P, _P, _P, _P, _P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _P]),
    "ctox_hip_gated_delta_step_device": (_I32, [_P, _P, _P, _P, _P, _P, _P, _SZ, _SZ, _SZ, _P, _P]),
    "ctox_hip_gated_delta_sequence_device": (_I32, [_P, _P, _P, _P, _P, _P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P]),
    "ctox_hip_gdn_gates_device": (_I32, [_P, _P, _P, _P, _P, _SZ, _SZ, _P, _P, _P]),
    "ctox_hip_repeat_heads_device": (_I32, [_P, _P, _SZ, _SZ, _SZ, _SZ, _P, _P]),
    "ctox_hip_greedy_tokens_device": (_I32, [_P, _P, _SZ, _SZ, _P, _P]),
    "ctox_hip_verify_greedy_mtp_device": (_I32, [_P, _P, _P, _P, _SZ, _SZ, _P, _P]),
    "ctox_hip_mtp_accept_device": (_I32, [_P, _P, _P, _P, _P, _SZ, _SZ, ctypes.c_float, _P, _P, _P]),
    "ctox_hip_mtp_accept_restricted_device": (_I32, [_P, _P, _SZ, _P, _P, _P, _P, _P, _SZ, _SZ, ctypes.c_float, _P,
                                                     _P, _P]),
    "ctox_hip_check_finite_device": (_I32, [_P, _P, _SZ, _P, _SZ, _P]),
    "ctox_hip_sample_topk_topp_device": (_I32, [_P, _P, _SZ, ctypes.c_float, _U32, ctypes.c_float, ctypes.c_float, _P,
                                                _P]),
    "ctox_hip_gather_rows_device": (_I32, [_P, _P, _SZ, _SZ, _P, _SZ, _P, _P]),
    "ctox_hip_gdn_fused_snap_device": (_I32, [_P, _P, _SZ, _SZ, _SZ, _P, _P, _P, _SZ, _SZ, _P, _P, _P, _P, _P, _P,
                                              _SZ, ctypes.c_int, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P]),
    "ctox_hip_rms_norm_device": (_I32, [_P, _P, _SZ, _SZ, _P, ctypes.c_float, _P, _P]),
    "ctox_hip_rms_norm_gated_device": (_I32, [_P, _P, _P, _SZ, _SZ, _P, ctypes.c_float, _P, _P]),
    "ctox_hip_swiglu_device": (_I32, [_P, _P, _P, _SZ, _P, _P]),
    "ctox_hip_sigmoid_gate_device": (_I32, [_P, _P, _P, _SZ, _P]),
    "ctox_hip_causal_conv_update_device": (_I32, [_P, _P, _P, _P, _SZ, _SZ, _P, _P]),
    "ctox_hip_partial_rope_device": (_I32, [_P, _P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_uint64, ctypes.c_float, _P]),
    "ctox_hip_gated_delta_strided_device": (_I32, [_P, _P, _P, _P, _SZ, _SZ, _P, _P, _P, _SZ, _SZ, _SZ, _SZ, _SZ,
                                                    _SZ, _P, _P]),
    "ctox_hip_gdn_gates_strided_device": (_I32, [_P, _P, _P, _SZ, _P, _P, _SZ, _SZ, _P, _P, _P]),
    "ctox_hip_causal_conv_rows_device": (_I32, [_P, _P, _SZ, _P, _P, _SZ, _SZ, _SZ, _P, _P]),
    "ctox_hip_kv_pack_q4_device": (_I32, [_P, _P, _P, _P, _SZ, _SZ, _U32, _U32, _U32, _P]),
    "ctox_hip_attn_prep_device": (_I32, [_P, _P, _SZ, _P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_uint64, ctypes.c_float,
                                         ctypes.c_float, _P, _U32, _P, _P, _P, _P, _P, _SZ, _P]),
    "ctox_hip_kv_demote_device": (_I32, [_P, _P, _P, _SZ, _SZ, _P]),
    "ctox_hip_paged_gqa_device": (_I32, [_P, _P, _P, _P, _P, ctypes.POINTER(PagedGqaParams), _SZ, _P, _P]),
    "ctox_hip_fill_random_device": (_I32, [_P, _P, ctypes.c_uint64, _U32, ctypes.c_uint64, ctypes.c_float,
                                           ctypes.c_float, _P]),
    "ctox_hip_embedding_rows_device": (_I32, [_P, _I32, _P, _P, _P, _P, _SZ, _SZ, _SZ, _P, _P]),
    "ctox_hip_norm_rows_device": (_I32, [_P, _P, _P]),
    "ctox_hip_attention_gate_device": (_I32, [_P, _P, _P, _SZ, _SZ, _SZ, _SZ, _P]),
    "ctox_hip_swiglu_rows_device": (_I32, [_P, _P, _SZ, _SZ, _SZ, _SZ, _P, _SZ, _P]),
    "ctox_hip_copy_rows_device": (_I32, [_P, _P, _SZ, _SZ, _SZ, _SZ, _P, _SZ, _P]),
    "ctox_hip_write_words_device": (_I32, [_P, _P, _P, _SZ, _P]),
    "ctox_hip_norm_matvec_device": (_I32, [_P, _P, _P, _U32, _SZ, _P, _P, ctypes.c_float, _P, _I32, _P, _P, _P, _P,
                                           _U32, _U32, _U32, _P]),
    "ctox_hip_transform_matvec_device": (_I32, [_P, _P, _I32, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _P, _P]),
    "ctox_hip_norm_matvec_sums_device": (_I32, [_P, _P, _P, _U32, _SZ, _P, _P, ctypes.c_float, _P, _I32, _P, _P, _P, _P,
                                                _U32, _U32, _U32, _P, _U32, _P]),
    "ctox_hip_norm_matvec_parts_device": (_I32, [_P, _P, _P, _U32, _SZ, _P, _P, ctypes.c_float, _P, _I32, _P, _P, _P,
                                                 _P, _U32, _U32, _U32, _P, _U32, _U32, _P, _P]),
    # decode engine (struct arguments passed by reference)
    "ctox_hip_engine_create": (_I32, [_P, _P, ctypes.c_uint64, ctypes.POINTER(_P)]),
    "ctox_hip_engine_destroy": (None, [_P]),
    "ctox_hip_engine_stream": (_P, [_P]),
    "ctox_hip_engine_set_rng": (_I32, [_P, ctypes.c_uint64]),
    "ctox_hip_engine_decode": (_I32, [_P, _U32, ctypes.POINTER(_P)]),
    "ctox_hip_engine_mtp_step": (_I32, [_P, _U32, ctypes.c_float, ctypes.POINTER(_U32)]),
    "ctox_hip_engine_fill_context": (_I32, [_P, _U32, ctypes.c_uint64]),
    "ctox_hip_engine_buffer": (_I32, [_P, _U32, ctypes.POINTER(_P), ctypes.POINTER(_SZ)]),
    "ctox_hip_engine_position": (_U32, [_P]),
    "ctox_hip_engine_set_draft_vocab": (_I32, [_P, _P, _SZ]),
    "ctox_hip_engine_cache": (_I32, [_P, _U32, _P]),
    "ctox_hip_engine_tensor": (_I32, [_P, ctypes.c_char_p, _P]),
    "ctox_hip_engine_create_with_dtypes": (_I32, [_P, _P, ctypes.c_uint64, _P, _SZ, ctypes.POINTER(_P)]),
    "ctox_hip_engine_write": (_I32, [_P, ctypes.c_char_p, _U32, _SZ, _P, _SZ]),
    "ctox_hip_engine_finish_load": (_I32, [_P]),
    "ctox_hip_stream_read_device": (_I32, [_P, _P, _SZ, _P, _P]),
}

_lib: Optional[ctypes.CDLL] = None


def load_library() -> ctypes.CDLL:
    """Loads lib/libctox_hip.so (raises OSError if it was not built)."""
    global _lib
    if _lib is None:
        # A process holds one HIP runtime. When PyTorch is installed its
        # bundled libamdhip64.so.7 is loaded first, and this library (same
        # SONAME) binds to it instead of loading /opt/rocm's copy beside it.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise OSError(f"{LIB_PATH} is missing: run `python ctox-llm_amd/build.py`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def _check(status: int) -> None:
    if status != 0:
        msg = load_library().ctox_hip_last_error().decode(errors="replace")
        raise _ERRORS.get(status, EngineError)(msg)


def _ptr(a: Optional[np.ndarray]) -> Optional[int]:
    return None if a is None else a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a) -> np.ndarray:
    if isinstance(a, (bytes, bytearray)):
        return np.frombuffer(bytes(a), dtype=np.uint8)
    return np.ascontiguousarray(a).view(np.uint8).reshape(-1)


def _scale(s: Optional[ScaleSlice]) -> _Scale:
    if s is None:
        return _Scale(0, None, 0)
    return _Scale(1 if s.kind == "f32" else 2, s.data.ctypes.data, len(s))


class _Op:
    """Keeps the numpy buffers behind a C descriptor alive."""

    def __init__(self, op: FusedMatVec):
        self.w = _u8(op.weights)
        self.x = None if op.input is None else _f32(op.input)
        self.bias = None if op.bias is None else _f32(op.bias)
        self.s_in, self.s_out = op.s_in, op.s_out
        segs = list(op.segments)
        self.segs = (_Segment * max(1, len(segs)))(
            *[_Segment(s.group_index, s.row_start, s.row_end, int(s.dtype), s.offset, s.length) for s in segs])
        self.c = _FusedMatVec(
            int(op.dtype), self.w.ctypes.data, self.w.size, self.segs if segs else None, len(segs),
            op.rows, op.columns, _ptr(self.x), 0 if self.x is None else self.x.size,
            _scale(op.s_in), _scale(op.s_out), _ptr(self.bias),
            0 if self.bias is None else self.bias.size, int(op.activation))


class HipMatrix:
    """A packed matrix resident in HBM (ctox_hip_matrix_prepare)."""

    def __init__(self, backend: "HipBackend", op: FusedMatVec):
        self.backend = backend
        self._op = _Op(op)
        h = ctypes.c_void_p()
        _check(load_library().ctox_hip_matrix_prepare(backend.handle, ctypes.byref(self._op.c), ctypes.byref(h)))
        self.handle = h
        self.rows, self.columns = op.rows, op.columns

    @property
    def device_weights(self) -> int:
        return load_library().ctox_hip_matrix_device_weights(self.handle)

    def dispatch(self, d_input: int, batch: int, d_output: int, stream: Optional[int] = None) -> None:
        """Device pointers: d_input [batch, columns] f32, d_output [batch, rows] f32."""
        _check(load_library().ctox_hip_matrix_dispatch(self.backend.handle, self.handle, d_input, batch,
                                                       d_output, stream))

    def close(self) -> None:
        if self.handle:
            load_library().ctox_hip_matrix_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipBackend:
    """`impl Backend for HipBackend` (Q/src/backend/mod.rs:153-169)."""

    def __init__(self, device: int = 0):
        lib = load_library()
        h = ctypes.c_void_p()
        _check(lib.ctox_hip_backend_create(device, ctypes.byref(h)))
        self.handle = h

    # -- Backend::{kind, promotion_state, profile}
    def kind(self) -> str:
        return load_library().ctox_hip_backend_kind(self.handle).decode()

    def promotion_state(self) -> str:
        return load_library().ctox_hip_backend_promotion_state(self.handle).decode()

    def profile(self) -> str:
        return load_library().ctox_hip_backend_profile(self.handle).decode()

    # -- Backend::fused_matvec
    def fused_matvec(self, op: FusedMatVec) -> np.ndarray:
        c = _Op(op)
        out = np.empty(op.rows, dtype=np.float32)
        _check(load_library().ctox_hip_fused_matvec(self.handle, ctypes.byref(c.c), out.ctypes.data, out.size))
        return out

    # -- Backend::fused_matvec_fanout
    def fused_matvec_fanout(self, ops: Sequence[FusedMatVec]) -> list[np.ndarray]:
        cs = [_Op(o) for o in ops]
        arr = (_FusedMatVec * max(1, len(cs)))(*[c.c for c in cs])
        outs = [np.empty(o.rows, dtype=np.float32) for o in ops]
        ptrs = (ctypes.c_void_p * max(1, len(outs)))(*[o.ctypes.data for o in outs])
        _check(load_library().ctox_hip_fused_matvec_fanout(self.handle, arr, len(cs), ptrs))
        return outs

    # -- Backend::recovered_row
    def recovered_row(self, op: RecoveredRow) -> np.ndarray:
        w = _u8(op.weights)
        c = _RecoveredRow(int(op.dtype), w.ctypes.data, w.size, op.columns, _scale(op.s_in), op.s_out)
        out = np.empty(op.columns, dtype=np.float32)
        _check(load_library().ctox_hip_recovered_row(self.handle, ctypes.byref(c), out.ctypes.data, out.size))
        return out

    # -- Backend::recovered_row_matvec
    def recovered_row_matvec(self, op: RecoveredRowMatVec) -> float:
        w = _u8(op.weights)
        x = _f32(op.corrected_input)
        c = _RecoveredRowMatVec(int(op.dtype), w.ctypes.data, w.size, x.ctypes.data, x.size, op.s_out)
        r = ctypes.c_float()
        _check(load_library().ctox_hip_recovered_row_matvec(self.handle, ctypes.byref(c), ctypes.byref(r)))
        return float(r.value)

    # -- resident matrices / raw launch
    def prepare(self, op: FusedMatVec) -> HipMatrix:
        return HipMatrix(self, op)

    def dispatch_fanout(self, matrices: Sequence[HipMatrix], d_input: int, batch: int,
                        d_outputs: Sequence[int], stream: Optional[int] = None) -> None:
        hs = (ctypes.c_void_p * len(matrices))(*[m.handle.value for m in matrices])
        outs = (ctypes.c_void_p * len(d_outputs))(*d_outputs)
        _check(load_library().ctox_hip_matrix_dispatch_fanout(self.handle, hs, len(matrices), d_input, batch,
                                                              outs, stream))

    def launch_fused_matvec(self, dtype: TensorDType, d_weights: int, d_input: int, d_s_in: Optional[int],
                            d_s_out: Optional[int], d_bias: Optional[int], d_output: int, rows: int,
                            columns: int, activation: Activation = Activation.Identity, batch: int = 1,
                            stream: Optional[int] = None) -> None:
        _check(load_library().ctox_hip_launch_fused_matvec(
            self.handle, int(dtype), d_weights, d_input, d_s_in, d_s_out, d_bias, d_output, rows, columns,
            int(activation), batch, stream))

    def register_tiled_weights(self, dtype: TensorDType, d_weights: int, rows: int, columns: int,
                               stream: Optional[int] = None) -> None:
        """Batch-1 raw launches on d_weights use a tiled copy made now."""
        _check(load_library().ctox_hip_register_tiled_weights(self.handle, int(dtype), d_weights, rows, columns,
                                                              stream))

    def unregister_tiled_weights(self, d_weights: int) -> None:
        load_library().ctox_hip_unregister_tiled_weights(self.handle, d_weights)

    # -- gated delta (Q/src/reference.rs:230-415)
    def gated_delta_step(self, q, k, v, log_decay, beta, state: np.ndarray, heads: int, key_dim: int,
                         value_dim: int) -> np.ndarray:
        """Updates `state` (f32, C-contiguous) in place and returns the output."""
        q, k, v, ld, b = (_f32(a) for a in (q, k, v, log_decay, beta))
        _require_state(state)
        out = np.empty(heads * value_dim, dtype=np.float32)
        _check(load_library().ctox_hip_gated_delta_step(
            self.handle, q.ctypes.data, k.ctypes.data, v.ctypes.data, ld.ctypes.data, b.ctypes.data,
            state.ctypes.data, heads, key_dim, value_dim, out.ctypes.data))
        return out

    def gated_delta_sequence(self, q, k, v, log_decay, beta, state: np.ndarray, tokens: int, heads: int,
                             key_dim: int, value_dim: int, chunk: int = 0) -> np.ndarray:
        q, k, v, ld, b = (_f32(a) for a in (q, k, v, log_decay, beta))
        _require_state(state)
        out = np.empty(tokens * heads * value_dim, dtype=np.float32)
        _check(load_library().ctox_hip_gated_delta_sequence(
            self.handle, q.ctypes.data, k.ctypes.data, v.ctypes.data, ld.ctypes.data, b.ctypes.data,
            state.ctypes.data, tokens, heads, key_dim, value_dim, chunk, out.ctypes.data))
        return out

    def gated_delta_sequence_device(self, d_q: int, d_k: int, d_v: int, d_log_decay: int, d_beta: int,
                                    d_state: int, tokens: int, heads: int, key_dim: int, value_dim: int,
                                    chunk: int, d_out: int, stream: Optional[int] = None) -> None:
        _check(load_library().ctox_hip_gated_delta_sequence_device(
            self.handle, d_q, d_k, d_v, d_log_decay, d_beta, d_state, tokens, heads, key_dim, value_dim,
            chunk, d_out, stream))

    def gated_delta_step_device(self, d_q: int, d_k: int, d_v: int, d_log_decay: int, d_beta: int,
                                d_state: int, heads: int, key_dim: int, value_dim: int, d_out: int,
                                stream: Optional[int] = None) -> None:
        _check(load_library().ctox_hip_gated_delta_step_device(
            self.handle, d_q, d_k, d_v, d_log_decay, d_beta, d_state, heads, key_dim, value_dim, d_out,
            stream))

    # ---- decode-step glue and token selection (device pointers) ----
    def gdn_gates_device(self, d_a: int, d_b: int, d_a_log: int, d_dt_bias: int, tokens: int, heads: int,
                         d_log_decay: int, d_beta: int, stream: Optional[int] = None) -> None:
        """Q/src/decoder.rs:881-902."""
        _check(load_library().ctox_hip_gdn_gates_device(self.handle, d_a, d_b, d_a_log, d_dt_bias, tokens, heads,
                                                        d_log_decay, d_beta, stream))

    def repeat_heads_device(self, d_in: int, rows: int, heads: int, dim: int, repeats: int, d_out: int,
                            stream: Optional[int] = None) -> None:
        """Q/src/decoder.rs:47-65."""
        _check(load_library().ctox_hip_repeat_heads_device(self.handle, d_in, rows, heads, dim, repeats, d_out,
                                                           stream))

    def greedy_tokens_device(self, d_logits: int, rows: int, vocab: int, d_tokens: int,
                             stream: Optional[int] = None) -> None:
        """Q/src/engine.rs:906-913 per row."""
        _check(load_library().ctox_hip_greedy_tokens_device(self.handle, d_logits, rows, vocab, d_tokens, stream))

    def verify_greedy_mtp_device(self, d_draft: int, d_target: int, d_bonus: int, drafts: int, vocab: int,
                                 d_out: int, stream: Optional[int] = None) -> None:
        """Q/src/engine.rs:915-963; d_out: 3 + drafts uint32."""
        _check(load_library().ctox_hip_verify_greedy_mtp_device(self.handle, d_draft, d_target, d_bonus, drafts,
                                                                vocab, d_out, stream))

    def mtp_accept_device(self, d_draft: int, d_target: int, d_bonus: int, d_tokens: int, drafts: int, vocab: int,
                          temperature: float, d_rng: int, d_out: int, stream: Optional[int] = None) -> None:
        """Rejection-sampling accept (no crate counterpart); d_rng: Pcg32 state, d_out: 2 uint32."""
        _check(load_library().ctox_hip_mtp_accept_device(self.handle, d_draft, d_target, d_bonus, d_tokens, drafts,
                                                         vocab, temperature, d_rng, d_out, stream))

    # ---- layer glue (device pointers, fp32) ----
    def rms_norm_device(self, d_x: int, rows: int, cols: int, d_w: int, eps: float, d_out: int,
                        stream: Optional[int] = None) -> None:
        """Q/src/reference.rs:38-62."""
        _check(load_library().ctox_hip_rms_norm_device(self.handle, d_x, rows, cols, d_w, eps, d_out, stream))

    def rms_norm_gated_device(self, d_x: int, d_gate: int, rows: int, cols: int, d_w: int, eps: float, d_out: int,
                              stream: Optional[int] = None) -> None:
        """Q/src/reference.rs:66-93."""
        _check(load_library().ctox_hip_rms_norm_gated_device(self.handle, d_x, d_gate, rows, cols, d_w, eps, d_out,
                                                             stream))

    def swiglu_device(self, d_gate: int, d_up: int, n: int, d_out: int, stream: Optional[int] = None) -> None:
        """Q/src/reference.rs:96-112."""
        _check(load_library().ctox_hip_swiglu_device(self.handle, d_gate, d_up, n, d_out, stream))

    def sigmoid_gate_device(self, d_values: int, d_gate: int, n: int, stream: Optional[int] = None) -> None:
        """Q/src/reference.rs:502-515 (in place)."""
        _check(load_library().ctox_hip_sigmoid_gate_device(self.handle, d_values, d_gate, n, stream))

    def causal_conv_update_device(self, d_input: int, d_state: int, d_weight: int, channels: int, kernel: int,
                                  d_out: int, stream: Optional[int] = None) -> None:
        """Q/src/reference.rs:159-187."""
        _check(load_library().ctox_hip_causal_conv_update_device(self.handle, d_input, d_state, d_weight, channels,
                                                                 kernel, d_out, stream))

    def partial_rope_device(self, d_q: int, d_k: int, rows: int, q_heads: int, k_heads: int, head_dim: int,
                            rotary_dim: int, position: int, theta: float, stream: Optional[int] = None) -> None:
        """Q/src/reference.rs:115-155 (in place; row t at position + t)."""
        _check(load_library().ctox_hip_partial_rope_device(self.handle, d_q, d_k, rows, q_heads, k_heads, head_dim,
                                                           rotary_dim, position, theta, stream))

    def gated_delta_strided_device(self, d_q: int, d_k: int, d_v: int, qk_stride: int, v_stride: int, d_log_decay: int,
                                   d_beta: int, d_state: int, tokens: int, heads: int, key_heads: int, key_dim: int,
                                   value_dim: int, chunk: int, d_out: int, stream: Optional[int] = None) -> None:
        """Recurrence over strided q/k/v with repeated key heads (Q/src/decoder.rs:868-913)."""
        _check(load_library().ctox_hip_gated_delta_strided_device(self.handle, d_q, d_k, d_v, qk_stride, v_stride,
                                                                  d_log_decay, d_beta, d_state, tokens, heads,
                                                                  key_heads, key_dim, value_dim, chunk, d_out,
                                                                  stream))

    def gdn_gates_strided_device(self, d_a: int, d_b: int, in_stride: int, d_a_log: int, d_dt_bias: int,
                                 tokens: int, heads: int, d_log_decay: int, d_beta: int,
                                 stream: Optional[int] = None) -> None:
        """Q/src/decoder.rs:881-902 on token rows of a fused projection."""
        _check(load_library().ctox_hip_gdn_gates_strided_device(self.handle, d_a, d_b, in_stride, d_a_log, d_dt_bias,
                                                                tokens, heads, d_log_decay, d_beta, stream))

    def causal_conv_rows_device(self, d_input: int, in_stride: int, d_state: int, d_weight: int, channels: int,
                                kernel: int, rows: int, d_out: int, stream: Optional[int] = None) -> None:
        """Q/src/reference.rs:159-187 over consecutive tokens."""
        _check(load_library().ctox_hip_causal_conv_rows_device(self.handle, d_input, in_stride, d_state, d_weight,
                                                               channels, kernel, rows, d_out, stream))

    # ---- paged KV cache (device pointers) ----
    def kv_pack_q4_device(self, d_q4_pages: int, d_keys: int, d_values: int, token_count: int,
                          component_values: int, physical_slot: int, first_token_in_page: int, q4_page_bytes: int,
                          stream: Optional[int] = None) -> None:
        """Q/src/kv_cache.rs:200-206 on the device."""
        _check(load_library().ctox_hip_kv_pack_q4_device(self.handle, d_q4_pages, d_keys, d_values, token_count,
                                                         component_values, physical_slot, first_token_in_page,
                                                         q4_page_bytes, stream))

    def attn_prep_device(self, d_proj: int, proj_stride: int, d_q_norm: int, d_k_norm: int, rows: int, q_heads: int,
                         kv_heads: int, head_dim: int, rotary_dim: int, position: int, theta: float, eps: float,
                         d_q4_pages: int, q4_page_bytes: int, slots, positions_in_page, d_q_out: int,
                         stream: Optional[int] = None) -> None:
        """Fused q/k norm + partial RoPE + Q4 K/V append (Q/src/decoder.rs:687-800, Q/src/kv_cache.rs:200-206)."""
        sl = (ctypes.c_uint32 * len(slots))(*slots)
        ps = (ctypes.c_uint32 * len(positions_in_page))(*positions_in_page)
        _check(load_library().ctox_hip_attn_prep_device(self.handle, d_proj, proj_stride, d_q_norm, d_k_norm, rows,
                                                        q_heads, kv_heads, head_dim, rotary_dim, position, theta, eps,
                                                        d_q4_pages, q4_page_bytes, sl, ps, d_q_out, None, None, 0,
                                                        stream))

    def kv_demote_device(self, d_q4_page: int, d_q2_page: int, tokens: int, blocks_per_token: int,
                         stream: Optional[int] = None) -> None:
        """Q/src/kv_cache.rs:216-236 on the device."""
        _check(load_library().ctox_hip_kv_demote_device(self.handle, d_q4_page, d_q2_page, tokens, blocks_per_token,
                                                        stream))

    def paged_gqa_device(self, d_query: int, d_q2_pages: int, d_q4_pages: int, d_descriptors: int,
                         params: PagedGqaParams, rows: int, d_out: int, stream: Optional[int] = None) -> None:
        """Q/src/reference.rs:420-499 over the paged cache."""
        _check(load_library().ctox_hip_paged_gqa_device(self.handle, d_query, d_q2_pages, d_q4_pages, d_descriptors,
                                                        ctypes.byref(params), rows, d_out, stream))

    def synchronize(self) -> None:
        _check(load_library().ctox_hip_synchronize(self.handle))

    def close(self) -> None:
        if getattr(self, "handle", None):
            load_library().ctox_hip_backend_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _require_state(state: np.ndarray) -> None:
    if state.dtype != np.float32 or not state.flags.c_contiguous:
        raise ShapeError("delta state must be a C-contiguous float32 array updated in place")
