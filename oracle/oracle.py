"""ctypes binding of oracle/liboracle.so -- the CPU restatement of the
reference decode arithmetic.

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and
by the cpu_baseline leg of bench.py, always as the checker.  The product
(gateddeltanet_amd/) never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, c_float, c_int, c_size_t, c_uint16, c_uint32

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

REF, BF16W_FP32S, FP32, BF16X = 0, 1, 2, 3
LIBM, CR = 0, 1

FP = POINTER(c_float)


class Header(ctypes.Structure):
    _fields_ = [
        ("magic", ctypes.c_char * 8), ("version", c_uint32), ("vocab_size", c_uint32),
        ("hidden_size", c_uint32), ("num_layers", c_uint32), ("num_heads", c_uint32),
        ("num_v_heads", c_uint32), ("head_dim", c_uint32), ("intermediate_size", c_uint32),
        ("conv_size", c_uint32), ("max_seq_len", c_uint32), ("bos_token_id", ctypes.c_int32),
        ("eos_token_id", ctypes.c_int32), ("norm_eps", c_float),
    ]


_SIG = {
    "orc_rne_bits": (c_uint16, [c_uint32]),
    "orc_widen_bits": (c_uint32, [c_uint16]),
    "orc_bf16_round": (c_float, [c_float]),
    "orc_native_product_bits": (c_uint16, [c_uint16, c_uint16]),
    "orc_expf": (c_float, [c_float, c_int]),
    "orc_log1pf": (c_float, [c_float, c_int]),
    "orc_sigmoid": (c_float, [c_float, c_int]),
    "orc_silu": (c_float, [c_float, c_int]),
    "orc_softplus": (c_float, [c_float, c_int]),
    "orc_tree16": (c_float, [FP]),
    "orc_tree256": (c_float, [FP]),
    "orc_gemv": (None, [c_int, FP, FP, c_int, c_int, FP]),
    "orc_gemv_rows": (None, [c_int, FP, FP, c_int, c_int, FP]),
    "orc_gemv_tiny": (None, [FP, FP, c_int, c_int, FP]),
    "orc_rmsnorm": (None, [c_int, FP, FP, c_int, c_float, FP]),
    "orc_residual_rmsnorm": (None, [c_int, FP, FP, FP, c_int, c_float, FP, FP]),
    "orc_output_norm_gate": (None, [c_int, c_int, FP, FP, FP, c_int, c_int, c_float, FP]),
    "orc_conv_silu": (None, [c_int, c_int, FP, FP, FP, c_int, FP]),
    "orc_head_scalars": (None, [c_int, c_float, c_float, c_float, c_float, FP, FP]),
    "orc_recurrence_head": (None, [c_int, c_int, FP, FP, FP, c_float, c_float, c_float, c_float, FP, FP]),
    "orc_recurrence_head_scalars": (None, [c_int, FP, FP, FP, c_float, c_float, FP, FP]),
    "orc_swiglu": (None, [c_int, c_int, FP, FP, c_int, FP]),
    "orc_argmax": (c_int, [FP, c_int]),
    "orc_total_weight_floats": (c_size_t, [POINTER(Header)]),
    "orc_layer_offset": (c_size_t, [POINTER(Header), c_int]),
    "orc_layer_forward": (None, [c_int, c_int, POINTER(Header), FP, c_int, FP, FP, FP, FP]),
    "orc_decode_step": (c_int, [c_int, c_int, POINTER(Header), FP, FP, FP, c_int, FP, FP]),
    "orc_compute_logits": (None, [POINTER(Header), FP, FP, FP]),
    "orc_decode_step_trace": (c_int, [c_int, c_int, POINTER(Header), FP, FP, FP, c_int, FP, FP, FP]),
    "orc_set_threads": (None, [c_int]),
    "orc_rne_array": (None, [POINTER(c_uint32), POINTER(c_uint16), c_size_t]),
    "orc_native_product_array": (None, [POINTER(c_uint16), POINTER(c_uint16), POINTER(c_uint16), c_size_t]),
    "orc_native_product_sel_array": (None, [POINTER(c_uint16), POINTER(c_uint16), POINTER(c_uint16), c_size_t]),
    "orc_transcendental_array": (None, [c_int, c_int, FP, FP, c_size_t]),
}

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIG.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def _f(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(FP)


def header_from(cfg) -> Header:
    """Copy any ctypes struct with the GDNWeightHeader fields."""
    h = Header()
    for name, _ in Header._fields_:
        setattr(h, name, getattr(cfg, name))
    return h


def set_threads(n: int) -> None:
    lib().orc_set_threads(n)


def rne_array(bits: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint32)
    out = np.empty(b.size, np.uint16)
    lib().orc_rne_array(b.ctypes.data_as(POINTER(c_uint32)), out.ctypes.data_as(POINTER(c_uint16)), b.size)
    return out


def native_product_array(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.uint16)
    out = np.empty(w.size, np.uint16)
    lib().orc_native_product_array(w.ctypes.data_as(POINTER(c_uint16)), x.ctypes.data_as(POINTER(c_uint16)),
                                   out.ctypes.data_as(POINTER(c_uint16)), w.size)
    return out


def native_product_sel_array(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    """The branch-free form of the native product used inside the GEMV rows."""
    w = np.ascontiguousarray(w, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.uint16)
    out = np.empty(w.size, np.uint16)
    lib().orc_native_product_sel_array(w.ctypes.data_as(POINTER(c_uint16)), x.ctypes.data_as(POINTER(c_uint16)),
                                       out.ctypes.data_as(POINTER(c_uint16)), w.size)
    return out


def transcendental_array(which: str, x: np.ndarray, tmode: int = LIBM) -> np.ndarray:
    code = {"exp": 0, "log1p": 1, "sigmoid": 2, "silu": 3, "softplus": 4}[which]
    x = _f(x)
    out = np.empty_like(x)
    lib().orc_transcendental_array(code, tmode, _p(x), _p(out), x.size)
    return out


def tree16(p) -> float:
    p = _f(p)
    return float(lib().orc_tree16(_p(p)))


def tree256(a) -> float:
    a = _f(a)
    return float(lib().orc_tree256(_p(a)))


def gemv(contract: int, W, x, threads: bool = True) -> np.ndarray:
    W, x = _f(W), _f(x)
    M, K = W.shape
    y = np.empty(M, np.float32)
    fn = lib().orc_gemv if threads else lib().orc_gemv_rows
    fn(contract, _p(W), _p(x), M, K, _p(y))
    return y


def gemv_tiny(W, x) -> np.ndarray:
    W, x = _f(W), _f(x)
    M, K = W.shape
    y = np.empty(M, np.float32)
    lib().orc_gemv_tiny(_p(W), _p(x), M, K, _p(y))
    return y


def rmsnorm(contract: int, x, w, eps: float = 1e-6) -> np.ndarray:
    x, w = _f(x), _f(w)
    out = np.empty_like(x)
    lib().orc_rmsnorm(contract, _p(x), _p(w), x.size, eps, _p(out))
    return out


def residual_rmsnorm(contract: int, x, y, w, eps: float = 1e-6):
    x, y, w = _f(x), _f(y), _f(w)
    xo = np.empty_like(x)
    out = np.empty_like(x)
    lib().orc_residual_rmsnorm(contract, _p(x), _p(y), _p(w), x.size, eps, _p(xo), _p(out))
    return xo, out


def output_norm_gate(contract: int, o, g, w, nh: int, hd: int, eps: float = 1e-6, tmode: int = LIBM):
    o, g, w = _f(o), _f(g), _f(w)
    out = np.empty_like(o)
    lib().orc_output_norm_gate(contract, tmode, _p(o), _p(g), _p(w), nh, hd, eps, _p(out))
    return out


def conv_silu(contract: int, raw, conv_w, tails, tmode: int = LIBM):
    """tails [3][C] (row 0 oldest) is updated in a copy; returns (out, tails')."""
    raw, conv_w = _f(raw), _f(conv_w)
    t = _f(tails).copy()
    out = np.empty_like(raw)
    lib().orc_conv_silu(contract, tmode, _p(raw), _p(conv_w), _p(t), raw.size, _p(out))
    return out, t


def head_scalars(a: float, b: float, a_log: float, dt_bias: float, tmode: int = LIBM):
    beta = c_float()
    decay = c_float()
    lib().orc_head_scalars(tmode, a, b, a_log, dt_bias, ctypes.byref(beta), ctypes.byref(decay))
    return beta.value, decay.value


def recurrence_head(contract: int, q, k, v, a, b, a_log, dt_bias, S, tmode: int = LIBM):
    q, k, v = _f(q), _f(k), _f(v)
    S2 = _f(S).copy()
    o = np.empty(256, np.float32)
    lib().orc_recurrence_head(contract, tmode, _p(q), _p(k), _p(v), a, b, a_log, dt_bias, _p(S2), _p(o))
    return o, S2


def recurrence_head_scalars(contract: int, q, k, v, beta: float, decay: float, S):
    q, k, v = _f(q), _f(k), _f(v)
    S2 = _f(S).copy()
    o = np.empty(256, np.float32)
    lib().orc_recurrence_head_scalars(contract, _p(q), _p(k), _p(v), beta, decay, _p(S2), _p(o))
    return o, S2


def swiglu(contract: int, g, u, tmode: int = LIBM) -> np.ndarray:
    g, u = _f(g), _f(u)
    h = np.empty_like(g)
    lib().orc_swiglu(contract, tmode, _p(g), _p(u), g.size, _p(h))
    return h


def argmax(logits) -> int:
    l = _f(logits)
    return int(lib().orc_argmax(_p(l), l.size))


def layer_forward(contract: int, hdr: Header, blob: np.ndarray, layer: int, x, state, conv,
                  tmode: int = LIBM):
    """In-place on copies: returns (x', state', conv', attn_o)."""
    x = _f(x).copy()
    st = _f(state).copy()
    cv = _f(conv).copy()
    attn = np.empty(hdr.hidden_size, np.float32)
    lib().orc_layer_forward(contract, tmode, ctypes.byref(hdr), _p(blob), layer, _p(x), _p(st), _p(cv),
                            _p(attn))
    return x, st, cv, attn


def decode_step(contract: int, hdr: Header, blob: np.ndarray, state: np.ndarray, conv: np.ndarray,
                token: int, tmode: int = LIBM):
    """Advances state/conv IN PLACE (float32 contiguous arrays); returns
    (argmax, logits, final_hidden)."""
    assert state.dtype == np.float32 and state.flags["C_CONTIGUOUS"]
    assert conv.dtype == np.float32 and conv.flags["C_CONTIGUOUS"]
    logits = np.empty(hdr.vocab_size, np.float32)
    fh = np.empty(hdr.hidden_size, np.float32)
    tok = lib().orc_decode_step(contract, tmode, ctypes.byref(hdr), _p(blob), _p(state), _p(conv), token,
                                _p(logits), _p(fh))
    return int(tok), logits, fh


def decode_step_trace(contract: int, hdr: Header, blob: np.ndarray, state: np.ndarray, conv: np.ndarray,
                      token: int, tmode: int = LIBM):
    """decode_step that also returns the step's dense-GEMV input vectors:
    a list of (layer, kind, vector) with kind in qkvg, o, gu, down, then
    (None, "lm", final hidden)."""
    H, I, L = hdr.hidden_size, hdr.intermediate_size, hdr.num_layers
    per = 3 * H + I
    gin = np.empty(L * per + H, np.float32)
    logits = np.empty(hdr.vocab_size, np.float32)
    fh = np.empty(H, np.float32)
    tok = lib().orc_decode_step_trace(contract, tmode, ctypes.byref(hdr), _p(blob), _p(state), _p(conv), token,
                                      _p(logits), _p(fh), _p(gin))
    ins = []
    for l in range(L):
        b = gin[l * per:(l + 1) * per]
        ins += [(l, "qkvg", b[:H]), (l, "o", b[H:2 * H]), (l, "gu", b[2 * H:3 * H]), (l, "down", b[3 * H:])]
    ins.append((None, "lm", gin[L * per:]))
    return int(tok), logits, fh, ins


def compute_logits(hdr: Header, blob: np.ndarray, hidden) -> np.ndarray:
    h = _f(hidden)
    out = np.empty(hdr.vocab_size, np.float32)
    lib().orc_compute_logits(ctypes.byref(hdr), _p(blob), _p(h), _p(out))
    return out
