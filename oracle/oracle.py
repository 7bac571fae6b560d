"""ctypes wrapper of the C oracle (oracle/libctox_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker or the timed CPU baseline. The
product path (ctox-llm_amd/) never imports this module.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libctox_oracle.so")

SCALAR, AVX2 = 0, 1
Q2B64, Q4B64, MIXED = 0, 1, 2
BLOCK_LEN, Q2_BLOCK_BYTES, Q4_BLOCK_BYTES = 64, 18, 34


class OracleError(Exception):
    def __init__(self, code: int):
        super().__init__(f"oracle status {code}")
        self.code = code


class _Scale(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("data", ctypes.c_void_p), ("len", ctypes.c_size_t)]


class _Segment(ctypes.Structure):
    _fields_ = [("group_index", ctypes.c_uint32), ("row_start", ctypes.c_uint64),
                ("row_end", ctypes.c_uint64), ("dtype", ctypes.c_int32),
                ("offset", ctypes.c_uint64), ("length", ctypes.c_uint64)]


class _Op(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int32), ("weights", ctypes.c_void_p),
                ("weights_len", ctypes.c_size_t), ("segments", ctypes.POINTER(_Segment)),
                ("n_segments", ctypes.c_size_t), ("rows", ctypes.c_size_t),
                ("columns", ctypes.c_size_t), ("input", ctypes.c_void_p),
                ("input_len", ctypes.c_size_t), ("s_in", _Scale), ("s_out", _Scale),
                ("bias", ctypes.c_void_p), ("bias_len", ctypes.c_size_t),
                ("activation", ctypes.c_int32)]


class _Pcg(ctypes.Structure):
    _fields_ = [("state", ctypes.c_uint64)]


_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OSError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        SZ = ctypes.c_size_t
        F = ctypes.c_float
        L.orc_f16_to_f32.restype = F
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [F]
        for n in ("orc_q2_value", "orc_q4_value"):
            getattr(L, n).restype = F
            getattr(L, n).argtypes = [P, SZ]
        for n in ("orc_packed_q2_dot", "orc_packed_q4_dot"):
            getattr(L, n).restype = F
            getattr(L, n).argtypes = [ctypes.c_int, F, P, P]
        L.orc_recovered_row.argtypes = [ctypes.c_int32, P, SZ, SZ, _Scale, F, P]
        L.orc_recovered_row_matvec.argtypes = [ctypes.c_int, ctypes.c_int32, P, SZ, P, SZ, F, P]
        L.orc_gated_delta_step.argtypes = [P, P, P, P, P, P, SZ, SZ, SZ, P]
        L.orc_gated_delta_step_f16_state.argtypes = [P, P, P, P, P, P, SZ, SZ, SZ, P]
        L.orc_gated_delta_sequence.argtypes = [P, P, P, P, P, P, SZ, SZ, SZ, SZ, P]
        L.orc_rms_norm_1p_weight.argtypes = [P, SZ, SZ, P, F, P]
        L.orc_rms_norm_gated.argtypes = [P, P, SZ, SZ, P, F, P]
        L.orc_swiglu.argtypes = [P, P, SZ, P]
        L.orc_causal_conv_silu_update.argtypes = [P, P, P, SZ, SZ, P]
        L.orc_apply_partial_rope.argtypes = [P, P, SZ, SZ, SZ, SZ, ctypes.c_uint64, F]
        L.orc_grouped_query_attention.argtypes = [P, P, P, SZ, SZ, SZ, SZ, SZ, SZ, P]
        L.orc_sigmoid_gate.argtypes = [P, P, SZ]
        L.orc_softplus.restype = F
        L.orc_softplus.argtypes = [F]
        L.orc_gdn_gates.argtypes = [P, P, P, P, SZ, P, P]
        L.orc_repeat_heads.argtypes = [P, SZ, SZ, SZ, P]
        L.orc_pcg32_init.argtypes = [ctypes.POINTER(_Pcg), ctypes.c_uint64]
        L.orc_pcg32_next_u32.restype = ctypes.c_uint32
        L.orc_pcg32_next_u32.argtypes = [ctypes.POINTER(_Pcg)]
        L.orc_pcg32_next_f32.restype = F
        L.orc_pcg32_next_f32.argtypes = [ctypes.POINTER(_Pcg)]
        L.orc_sample_with_draw.argtypes = [P, SZ, F, SZ, F, F, ctypes.POINTER(SZ)]
        L.orc_greedy_token.argtypes = [P, SZ, ctypes.POINTER(ctypes.c_uint32)]
        L.orc_verify_greedy_mtp.argtypes = [P, P, P, SZ, SZ] + [ctypes.POINTER(ctypes.c_uint32)] * 2 + [P, ctypes.POINTER(ctypes.c_uint32)]
        L.orc_mtp_accept_sample.argtypes = [P, P, P, P, SZ, SZ, F, ctypes.POINTER(_Pcg),
                                            ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32)]
        L.orc_mtp_accept_sample_restricted.argtypes = [P, P, SZ, P, P, P, SZ, SZ, F, ctypes.POINTER(_Pcg),
                                                       ctypes.POINTER(ctypes.c_uint32),
                                                       ctypes.POINTER(ctypes.c_uint32)]
        L.orc_fused_matvec.argtypes = [ctypes.c_int, ctypes.POINTER(_Op), P]
        L.orc_fused_matvec_threads.argtypes = [ctypes.c_int, ctypes.POINTER(_Op), P, ctypes.c_int]
        L.orc_fused_matvec_fanout.argtypes = [ctypes.c_int, ctypes.POINTER(_Op), SZ, ctypes.POINTER(P)]
        L.orc_q2_quantize.argtypes = [P, P]
        L.orc_q4_quantize.argtypes = [P, P]
        L.orc_a8_quantize.argtypes = [P, ctypes.POINTER(F), P]
        _lib = L
    return _lib


def _ok(st: int) -> None:
    if st != 0:
        raise OracleError(st)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- f16
def f16_to_f32(bits: int) -> float:
    return lib().orc_f16_to_f32(bits)


def f32_to_f16(x: float) -> int:
    return lib().orc_f32_to_f16(x)


# ---------------------------------------------------------------- quant
def q2_quantize(values) -> bytes:
    v = _f32(values)
    out = (ctypes.c_uint8 * 18)()
    _ok(lib().orc_q2_quantize(v.ctypes.data, out))
    return bytes(out)


def q4_quantize(values) -> bytes:
    v = _f32(values)
    out = (ctypes.c_uint8 * 34)()
    _ok(lib().orc_q4_quantize(v.ctypes.data, out))
    return bytes(out)


def a8_quantize(values):
    v = _f32(values)
    codes = np.zeros(64, dtype=np.int8)
    s = ctypes.c_float()
    _ok(lib().orc_a8_quantize(v.ctypes.data, ctypes.byref(s), codes.ctypes.data))
    return s.value, codes


def q2_value(block: bytes, i: int) -> float:
    return lib().orc_q2_value(ctypes.c_char_p(block), i)


def q4_value(block: bytes, i: int) -> float:
    return lib().orc_q4_value(ctypes.c_char_p(block), i)


def packed_dot(dtype: int, profile: int, scale: float, codes: bytes, x) -> float:
    xv = _f32(x)
    fn = lib().orc_packed_q2_dot if dtype == Q2B64 else lib().orc_packed_q4_dot
    return fn(profile, scale, ctypes.c_char_p(codes), xv.ctypes.data)


def avx2_available() -> bool:
    return bool(lib().orc_avx2_available())


# ---------------------------------------------------------------- matvec
class MatVec:
    """Holds numpy buffers and the C descriptor of one fused matvec."""

    def __init__(self, dtype, weights, rows, columns, input, s_in=None, s_out=None, bias=None,
                 activation=0, segments: Sequence[tuple] = ()):
        self.w = np.ascontiguousarray(np.frombuffer(bytes(weights), dtype=np.uint8)
                                      if isinstance(weights, (bytes, bytearray)) else weights).view(np.uint8).reshape(-1)
        self.x = _f32(input)
        self.bias = None if bias is None else _f32(bias)
        self._scales = []
        self.segs = (_Segment * max(1, len(segments)))(*[_Segment(*s) for s in segments])
        self.c = _Op(int(dtype), self.w.ctypes.data, self.w.size, self.segs if segments else None,
                     len(segments), rows, columns, self.x.ctypes.data, self.x.size,
                     self._scale(s_in), self._scale(s_out),
                     None if self.bias is None else self.bias.ctypes.data,
                     0 if self.bias is None else self.bias.size, int(activation))
        self.rows = rows

    def _scale(self, s):
        """s: None, ("f32", array) or ("f16le", uint8 array)."""
        if s is None:
            return _Scale(0, None, 0)
        kind, data = s
        if kind == "f32":
            a = _f32(data)
            self._scales.append(a)
            return _Scale(1, a.ctypes.data, a.size)
        a = np.ascontiguousarray(data, dtype=np.uint8)
        self._scales.append(a)
        return _Scale(2, a.ctypes.data, a.size // 2)

    def run(self, profile: int = SCALAR, threads: int = 1) -> np.ndarray:
        out = np.empty(self.rows, dtype=np.float32)
        if threads > 1:
            _ok(lib().orc_fused_matvec_threads(profile, ctypes.byref(self.c), out.ctypes.data, threads))
        else:
            _ok(lib().orc_fused_matvec(profile, ctypes.byref(self.c), out.ctypes.data))
        return out


def fused_matvec(dtype, weights, rows, columns, input, s_in=None, s_out=None, bias=None,
                 activation=0, segments=(), profile=SCALAR) -> np.ndarray:
    return MatVec(dtype, weights, rows, columns, input, s_in, s_out, bias, activation, segments).run(profile)


def fanout(mvs: Sequence[MatVec], profile=SCALAR):
    arr = (_Op * len(mvs))(*[m.c for m in mvs])
    outs = [np.empty(m.rows, dtype=np.float32) for m in mvs]
    ptrs = (ctypes.c_void_p * len(outs))(*[o.ctypes.data for o in outs])
    _ok(lib().orc_fused_matvec_fanout(profile, arr, len(mvs), ptrs))
    return outs


def recovered_row(dtype, weights: bytes, columns, s_in, s_out) -> np.ndarray:
    w = np.frombuffer(bytes(weights), dtype=np.uint8)
    kind, data = s_in
    arr = _f32(data) if kind == "f32" else np.ascontiguousarray(data, dtype=np.uint8)
    sc = _Scale(1 if kind == "f32" else 2, arr.ctypes.data, arr.size if kind == "f32" else arr.size // 2)
    out = np.empty(columns, dtype=np.float32)
    _ok(lib().orc_recovered_row(dtype, w.ctypes.data, w.size, columns, sc, s_out, out.ctypes.data))
    return out


def recovered_row_matvec(dtype, weights: bytes, x, s_out, profile=SCALAR) -> float:
    w = np.frombuffer(bytes(weights), dtype=np.uint8)
    xv = _f32(x)
    r = ctypes.c_float()
    _ok(lib().orc_recovered_row_matvec(profile, dtype, w.ctypes.data, w.size, xv.ctypes.data, xv.size,
                                       s_out, ctypes.byref(r)))
    return r.value


# ---------------------------------------------------------------- gated delta
def gated_delta_step(q, k, v, log_decay, beta, state: np.ndarray, heads, key_dim, value_dim) -> np.ndarray:
    q, k, v, ld, b = (_f32(a) for a in (q, k, v, log_decay, beta))
    assert state.dtype == np.float32 and state.flags.c_contiguous
    out = np.empty(heads * value_dim, dtype=np.float32)
    _ok(lib().orc_gated_delta_step(q.ctypes.data, k.ctypes.data, v.ctypes.data, ld.ctypes.data, b.ctypes.data,
                                   state.ctypes.data, heads, key_dim, value_dim, out.ctypes.data))
    return out


def gated_delta_step_f16_state(q, k, v, log_decay, beta, state: np.ndarray, heads, key_dim, value_dim):
    q, k, v, ld, b = (_f32(a) for a in (q, k, v, log_decay, beta))
    assert state.dtype == np.uint16 and state.flags.c_contiguous
    out = np.empty(heads * value_dim, dtype=np.float32)
    _ok(lib().orc_gated_delta_step_f16_state(q.ctypes.data, k.ctypes.data, v.ctypes.data, ld.ctypes.data,
                                             b.ctypes.data, state.ctypes.data, heads, key_dim, value_dim,
                                             out.ctypes.data))
    return out


def gated_delta_sequence(q, k, v, log_decay, beta, state: np.ndarray, tokens, heads, key_dim, value_dim):
    q, k, v, ld, b = (_f32(a) for a in (q, k, v, log_decay, beta))
    assert state.dtype == np.float32 and state.flags.c_contiguous
    out = np.empty(tokens * heads * value_dim, dtype=np.float32)
    _ok(lib().orc_gated_delta_sequence(q.ctypes.data, k.ctypes.data, v.ctypes.data, ld.ctypes.data,
                                       b.ctypes.data, state.ctypes.data, tokens, heads, key_dim, value_dim,
                                       out.ctypes.data))
    return out


def rms_norm_1p_weight(x, rows, cols, w, eps):
    x, w = _f32(x), _f32(w)
    out = np.empty(rows * cols, dtype=np.float32)
    _ok(lib().orc_rms_norm_1p_weight(x.ctypes.data, rows, cols, w.ctypes.data, eps, out.ctypes.data))
    return out


def rms_norm_gated(x, gate, rows, cols, w, eps):
    x, g, w = _f32(x), _f32(gate), _f32(w)
    out = np.empty(rows * cols, dtype=np.float32)
    _ok(lib().orc_rms_norm_gated(x.ctypes.data, g.ctypes.data, rows, cols, w.ctypes.data, eps, out.ctypes.data))
    return out


def swiglu(gate, up):
    g, u = _f32(gate), _f32(up)
    out = np.empty(g.size, dtype=np.float32)
    _ok(lib().orc_swiglu(g.ctypes.data, u.ctypes.data, g.size, out.ctypes.data))
    return out


def causal_conv_silu_update(inp, state: np.ndarray, weight, channels, kernel):
    i, w = _f32(inp), _f32(weight)
    out = np.empty(channels, dtype=np.float32)
    _ok(lib().orc_causal_conv_silu_update(i.ctypes.data, state.ctypes.data, w.ctypes.data, channels, kernel,
                                          out.ctypes.data))
    return out


def apply_partial_rope(q: np.ndarray, k: np.ndarray, qh, kh, hd, rd, position, theta):
    _ok(lib().orc_apply_partial_rope(q.ctypes.data, k.ctypes.data, qh, kh, hd, rd, position, theta))


def grouped_query_attention(q, k, v, qh, kvh, qt, kvt, hd, q0):
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.empty(qt * qh * hd, dtype=np.float32)
    _ok(lib().orc_grouped_query_attention(q.ctypes.data, k.ctypes.data, v.ctypes.data, qh, kvh, qt, kvt, hd, q0,
                                          out.ctypes.data))
    return out


def sigmoid_gate(values: np.ndarray, gate):
    g = _f32(gate)
    _ok(lib().orc_sigmoid_gate(values.ctypes.data, g.ctypes.data, g.size))


def softplus(x: float) -> float:
    return lib().orc_softplus(x)


def gdn_gates(a, b, a_log, dt_bias):
    a, b, al, dt = (_f32(t) for t in (a, b, a_log, dt_bias))
    ld = np.empty(a.size, dtype=np.float32)
    be = np.empty(a.size, dtype=np.float32)
    lib().orc_gdn_gates(a.ctypes.data, b.ctypes.data, al.ctypes.data, dt.ctypes.data, a.size, ld.ctypes.data,
                        be.ctypes.data)
    return ld, be


def repeat_heads(values, heads, dim, repeats):
    v = _f32(values)
    out = np.empty(heads * dim * repeats, dtype=np.float32)
    _ok(lib().orc_repeat_heads(v.ctypes.data, heads, dim, repeats, out.ctypes.data))
    return out


# ---------------------------------------------------------------- sampler
class Pcg32:
    def __init__(self, seed: int):
        self.c = _Pcg()
        lib().orc_pcg32_init(ctypes.byref(self.c), seed)

    def next_u32(self) -> int:
        return lib().orc_pcg32_next_u32(ctypes.byref(self.c))

    def next_f32(self) -> float:
        return lib().orc_pcg32_next_f32(ctypes.byref(self.c))


def sample_with_draw(logits, temperature, top_k, top_p, draw) -> int:
    x = _f32(logits)
    t = ctypes.c_size_t()
    _ok(lib().orc_sample_with_draw(x.ctypes.data, x.size, temperature, top_k, top_p, draw, ctypes.byref(t)))
    return t.value


def greedy_token(logits) -> int:
    x = _f32(logits)
    t = ctypes.c_uint32()
    _ok(lib().orc_greedy_token(x.ctypes.data, x.size, ctypes.byref(t)))
    return t.value


def verify_greedy_mtp(draft, target, bonus):
    d, t = _f32(draft), _f32(target)
    drafts, vocab = d.shape
    b = None if bonus is None else _f32(bonus)
    nxt, ver, nacc = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32()
    acc = np.zeros(drafts, dtype=np.uint32)
    _ok(lib().orc_verify_greedy_mtp(d.ctypes.data, t.ctypes.data, None if b is None else b.ctypes.data, drafts,
                                    vocab, ctypes.byref(nxt), ctypes.byref(ver), acc.ctypes.data,
                                    ctypes.byref(nacc)))
    return nxt.value, ver.value, list(acc[: nacc.value])


def mtp_accept_sample(draft, target, bonus, draft_tokens, temperature, rng: Pcg32, draft_ids=None):
    """Rejection-sampling acceptance; with `draft_ids` the draft rows are
    restricted distributions over those strictly increasing token IDs."""
    d, t, b = _f32(draft), _f32(target), _f32(bonus)
    toks = np.ascontiguousarray(draft_tokens, dtype=np.uint32)
    nxt, nacc = ctypes.c_uint32(), ctypes.c_uint32()
    drafts = toks.size
    vocab = b.size
    ids = None if draft_ids is None else np.ascontiguousarray(draft_ids, dtype=np.uint32)
    dn = vocab if ids is None else ids.size
    if drafts and (d.size != drafts * dn or t.size != drafts * vocab):
        raise OracleError(1)
    _ok(lib().orc_mtp_accept_sample_restricted(
        d.ctypes.data if d.size else None, None if ids is None else ids.ctypes.data, dn,
        t.ctypes.data if t.size else None, b.ctypes.data, toks.ctypes.data, drafts, vocab, temperature,
        ctypes.byref(rng.c), ctypes.byref(nxt), ctypes.byref(nacc)))
    return nxt.value, nacc.value
