"""Python host mirror of the engine's C ABI (include/gdn_amd.h).

Names and argument meanings follow the reference's native decode API
(c_impl/gdn_model.h): ``Model`` wraps ``GDNModel`` (``gdn_model_load`` /
``gdn_model_free``), ``RunState`` wraps ``GDNRunState``
(``gdn_run_state_init`` / ``gdn_decode_step_host`` / ``gdn_run_state_free``),
and the module-level helpers wrap the seeded generators and the isolated
kernel hooks.  Errors raise ``GDNError`` where the C ABI returns -1.
"""
from __future__ import annotations

import ctypes
from typing import Dict, Optional, Sequence, Tuple

import numpy as np

from . import _lib as L

CONTRACT_REF = L.CONTRACT_REF
CONTRACT_BF16W_FP32S = L.CONTRACT_BF16W_FP32S
CONTRACT_FP32 = L.CONTRACT_FP32
PREFILL_SCAN = L.PREFILL_SCAN
PREFILL_CHUNKED = L.PREFILL_CHUNKED

LAYER_TENSORS = (
    "attn_norm", "a_log", "dt_bias", "q_proj", "k_proj", "v_proj", "a_proj", "b_proj",
    "q_conv", "k_conv", "v_conv", "g_proj", "o_norm", "o_proj", "mlp_norm",
    "mlp_gate_proj", "mlp_up_proj", "mlp_down_proj",
)


class GDNError(RuntimeError):
    pass


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise GDNError(f"{what} failed (rc={rc})")


def _f32(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def fptr(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(L.FP)


def iptr(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(L.IP)


def default_config(num_layers: int = 24) -> L.GDNWeightHeader:
    cfg = L.GDNWeightHeader()
    L.load().gdn_default_config(ctypes.byref(cfg), num_layers)
    return cfg


# The per-kernel step's activation buffers in device order (float32 counts;
# vocabularies of 32000, for which the LM head's 8-row partial buffer is
# 4032 long): residual ping-pong, final hidden, q|k|v after conv, gate,
# sigmoid(gate), a|b, attention output o, o_proj output, down output, SwiGLU
# output, LM-head partial maxima, embedding row, logits, q/k partial sums of
# squares, output-norm chunk sums.
ACTIVATION_LAYOUT = (("resid", 2048), ("resid_alt", 2048), ("fhid", 2048), ("qkv", 3 * 2048), ("gate", 2048),
                     ("sgate", 2048), ("ab", 64), ("attn", 2048), ("ybuf_o", 2048), ("dbuf", 2048), ("hbuf", 5632),
                     ("lm_val", 4032), ("xrow", 2048), ("logits", 32000), ("qkpart", 256), ("osum", 128))

# Exchange regions of the persistent step (word offsets, gdn_persist.h).
EXCHANGE_REGIONS = dict(qkv=0, g=6144, qk_part=8192, ab=8704, o=8768, osum=10816, y_o=11072, h=13120, y_down=18752,
                        argmax=20800)
EXCHANGE_WORDS = 21888


class Model:
    """A host model in .gdnw order (FP32 words)."""

    def __init__(self) -> None:
        self._m = L.GDNModel()
        self._live = False

    @classmethod
    def load(cls, path: str, fp32: bool = False) -> "Model":
        m = cls()
        fn = L.load().gdn_model_load_fp32 if fp32 else L.load().gdn_model_load
        _check(fn(ctypes.byref(m._m), path.encode()), "gdn_model_load")
        m._live = True
        return m

    @classmethod
    def synth(cls, num_layers: int = 24, seed: int = 0, std: float = 0.02, bf16: bool = True,
              config: Optional[L.GDNWeightHeader] = None) -> "Model":
        """Seeded random-init model: N(0, std) per tensor, norm weights = 1."""
        m = cls()
        cfg = config if config is not None else default_config(num_layers)
        _check(L.load().gdn_model_synth(ctypes.byref(m._m), ctypes.byref(cfg), seed, std,
                                        1 if bf16 else 0), "gdn_model_synth")
        m._live = True
        return m

    @property
    def config(self) -> L.GDNWeightHeader:
        return self._m.config

    @property
    def ptr(self):
        return ctypes.byref(self._m)

    @property
    def total_floats(self) -> int:
        return int(L.load().gdn_total_weight_floats(ctypes.byref(self._m.config)))

    @property
    def blob(self) -> np.ndarray:
        """The whole .gdnw payload as a float32 view (no copy)."""
        return np.ctypeslib.as_array(self._m.weight_data, shape=(self.total_floats,))

    def _view(self, p, n: int) -> np.ndarray:
        return np.ctypeslib.as_array(p, shape=(n,))

    def layer(self, i: int) -> Dict[str, np.ndarray]:
        c = self.config
        H, nh, hd, I, cs = c.hidden_size, c.num_heads, c.head_dim, c.intermediate_size, c.conv_size
        sizes = {
            "attn_norm": H, "a_log": nh, "dt_bias": nh, "q_proj": H * H, "k_proj": H * H,
            "v_proj": H * H, "a_proj": nh * H, "b_proj": nh * H, "q_conv": H * cs,
            "k_conv": H * cs, "v_conv": H * cs, "g_proj": H * H, "o_norm": hd, "o_proj": H * H,
            "mlp_norm": H, "mlp_gate_proj": I * H, "mlp_up_proj": I * H, "mlp_down_proj": H * I,
        }
        lw = self._m.layers[i]
        return {k: self._view(getattr(lw, k), n) for k, n in sizes.items()}

    @property
    def embeddings(self) -> np.ndarray:
        c = self.config
        return self._view(self._m.embeddings, c.vocab_size * c.hidden_size)

    @property
    def lm_head(self) -> np.ndarray:
        c = self.config
        return self._view(self._m.lm_head, c.vocab_size * c.hidden_size)

    @property
    def final_norm(self) -> np.ndarray:
        return self._view(self._m.final_norm, self.config.hidden_size)

    def save(self, path: str) -> None:
        _check(L.load().gdn_model_save(ctypes.byref(self._m), path.encode()), "gdn_model_save")

    def compute_logits(self, hidden: np.ndarray) -> np.ndarray:
        """The reference's independent scalar LM head (host)."""
        h = _f32(hidden)
        out = np.empty(self.config.vocab_size, np.float32)
        L.load().gdn_compute_logits(ctypes.byref(self._m), fptr(h), fptr(out))
        return out

    def free(self) -> None:
        if self._live:
            L.load().gdn_model_free(ctypes.byref(self._m))
            self._live = False

    def __del__(self) -> None:
        try:
            self.free()
        except Exception:
            pass


class RunState:
    """Device run state: weights in the engine layout, workspace, graph."""

    def __init__(self, model: Model, contract: int = CONTRACT_REF, max_tokens: int = 1) -> None:
        self.model = model
        self._s = L.GDNRunState()
        self._live = False
        _check(L.load().gdn_run_state_init_contract(ctypes.byref(self._s), model.ptr, max_tokens,
                                                    contract), "gdn_run_state_init")
        self._live = True
        c = model.config
        self.n_state = c.num_layers * c.num_heads * c.head_dim * c.head_dim
        self.n_conv = c.num_layers * 3 * (c.conv_size - 1) * c.hidden_size

    @property
    def ptr(self):
        return ctypes.byref(self._s)

    @property
    def contract(self) -> int:
        return int(L.load().gdn_get_contract(ctypes.byref(self._s)))

    def set_graph(self, use_graph: bool) -> None:
        _check(L.load().gdn_set_graph_mode(self.ptr, 1 if use_graph else 0), "gdn_set_graph_mode")

    def step_buffers(self, which: int, nbytes: int) -> np.ndarray:
        """gdn_test_step_buffers: the last step's exchange area (which = 0,
        uint32 words), activations (1, float32, ACTIVATION_LAYOUT), the
        persistent step's phase stamps (2, uint64) or the per-kernel step's
        (3, uint64)."""
        dt = {0: np.uint32, 1: np.float32, 2: np.uint64, 3: np.uint64}[which]
        out = np.empty(nbytes // np.dtype(dt).itemsize, dt)
        _check(L.load().gdn_test_step_buffers(self.ptr, which, out.ctypes.data, out.nbytes), "gdn_test_step_buffers")
        return out

    def activations(self) -> Dict[str, np.ndarray]:
        """The per-kernel step's activation buffers after the last step."""
        n = sum(size for _, size in ACTIVATION_LAYOUT)
        buf = self.step_buffers(1, 4 * n)
        out, o = {}, 0
        for name, size in ACTIVATION_LAYOUT:
            out[name] = buf[o:o + size]
            o += size
        return out

    def set_persistent(self, on: bool) -> None:
        """Switch between the persistent one-launch step (a run state made
        with GDN_PERSIST=1 in the environment has it) and the captured graph."""
        _check(L.load().gdn_set_persistent(self.ptr, 1 if on else 0), "gdn_set_persistent")

    @property
    def persistent(self) -> bool:
        return int(L.load().gdn_get_persistent(ctypes.byref(self._s))) == 1

    def decode_step(self, token: int) -> int:
        """gdn_decode_step_host; returns the device argmax token."""
        t = np.array([token], np.int32)
        _check(L.load().gdn_decode_step_host(self.model.ptr, self.ptr, iptr(t)), "gdn_decode_step_host")
        return self.token()

    def token(self) -> int:
        t = np.zeros(1, np.int32)
        _check(L.load().gdn_read_token(self.ptr, iptr(t)), "gdn_read_token")
        return int(t[0])

    def logits(self) -> np.ndarray:
        out = np.empty(self.model.config.vocab_size, np.float32)
        _check(L.load().gdn_read_logits(self.ptr, fptr(out), out.size), "gdn_read_logits")
        return out

    def final_hidden(self) -> np.ndarray:
        out = np.empty(self.model.config.hidden_size, np.float32)
        _check(L.load().gdn_read_final_hidden(self.ptr, fptr(out), out.size), "gdn_read_final_hidden")
        return out

    def load_state(self, recurrent: Optional[np.ndarray] = None, conv: Optional[np.ndarray] = None) -> None:
        lib = L.load()
        if recurrent is not None:
            r = _f32(recurrent).reshape(-1)
            _check(lib.gdn_load_recurrent_state(self.ptr, fptr(r), r.size), "gdn_load_recurrent_state")
        if conv is not None:
            cv = _f32(conv).reshape(-1)
            _check(lib.gdn_load_conv_tails(self.ptr, fptr(cv), cv.size), "gdn_load_conv_tails")

    def save_state(self) -> Tuple[np.ndarray, np.ndarray]:
        lib = L.load()
        r = np.empty(self.n_state, np.float32)
        cv = np.empty(self.n_conv, np.float32)
        _check(lib.gdn_save_recurrent_state(self.ptr, fptr(r), r.size), "gdn_save_recurrent_state")
        _check(lib.gdn_save_conv_tails(self.ptr, fptr(cv), cv.size), "gdn_save_conv_tails")
        return r, cv

    def load_gdnstate(self, path: str) -> Tuple[int, int]:
        pl = ctypes.c_uint32(0)
        seed = ctypes.c_int32(0)
        _check(L.load().gdn_load_gdnstate(self.ptr, self.model.ptr, path.encode(), ctypes.byref(pl),
                                          ctypes.byref(seed)), "gdn_load_gdnstate")
        return int(pl.value), int(seed.value)

    def save_gdnstate(self, path: str, prompt: Sequence[int] = (), seed_token: int = 0) -> None:
        p = np.ascontiguousarray(np.asarray(prompt, np.int32))
        _check(L.load().gdn_save_gdnstate(self.ptr, self.model.ptr, path.encode(), iptr(p), p.size,
                                          seed_token), "gdn_save_gdnstate")

    def teacher_forced(self, tokens: np.ndarray, n_steps: int, timing: bool = True):
        """Feed tokens[i % len] at step i; return (argmax, inner_ms, outer_ms)."""
        tk = np.ascontiguousarray(np.asarray(tokens, np.int32))
        am = np.empty(n_steps, np.int32)
        inner = np.empty(n_steps, np.float32) if timing else None
        outer = np.empty(n_steps, np.float32) if timing else None
        _check(L.load().gdn_run_teacher_forced(
            self.ptr, iptr(tk), tk.size, n_steps, iptr(am),
            fptr(inner) if timing else None, fptr(outer) if timing else None), "gdn_run_teacher_forced")
        return am, inner, outer

    KERNEL_KINDS = ("qkvg", "recur", "o_proj", "gate_up", "down", "lm_head", "argmax")

    def profile_kernels(self, rounds: int = 4) -> Dict[str, float]:
        """Average microseconds per launch of each kernel kind (advances state)."""
        out = np.zeros(len(self.KERNEL_KINDS), np.float32)
        _check(L.load().gdn_profile_kernels(self.ptr, rounds, fptr(out), out.size), "gdn_profile_kernels")
        return {k: float(v) for k, v in zip(self.KERNEL_KINDS, out)}

    def layer_steps(self, layer: int, x_in: np.ndarray) -> np.ndarray:
        """gdn_test_layer: run one layer over teacher-forced residual inputs."""
        x = _f32(x_in).reshape(-1, self.model.config.hidden_size)
        out = np.empty_like(x)
        _check(L.load().gdn_test_layer(self.ptr, layer, x.shape[0], fptr(x), fptr(out)), "gdn_test_layer")
        return out

    def free(self) -> None:
        if self._live:
            L.load().gdn_run_state_free(self.ptr)
            self._live = False

    def __del__(self) -> None:
        try:
            self.free()
        except Exception:
            pass


class BatchState:
    """Multi-stream decode (gdn_batch_*): n_streams independent streams, each
    with its own FP32 state, one token per stream per step; projections on
    the matrix cores.  No reference counterpart (the reference is batch-1)."""

    def __init__(self, model: Model, n_streams: int) -> None:
        self.model = model
        self._s = L.GDNBatchState()
        self._live = False
        _check(L.load().gdn_batch_init(ctypes.byref(self._s), model.ptr, n_streams), "gdn_batch_init")
        self._live = True
        self.n_streams = n_streams
        c = model.config
        self.n_state = c.num_layers * c.num_heads * c.head_dim * c.head_dim
        self.n_conv = c.num_layers * 3 * (c.conv_size - 1) * c.hidden_size

    @property
    def ptr(self):
        return ctypes.byref(self._s)

    def set_graph(self, use_graph: bool) -> None:
        _check(L.load().gdn_batch_set_graph_mode(self.ptr, 1 if use_graph else 0), "gdn_batch_set_graph_mode")

    def step(self, tokens: Sequence[int]) -> np.ndarray:
        """One token per stream in; the greedy next tokens out."""
        t = np.ascontiguousarray(np.asarray(tokens, np.int32))
        assert t.size == self.n_streams
        out = np.empty(self.n_streams, np.int32)
        _check(L.load().gdn_batch_decode_step(self.ptr, iptr(t), iptr(out)), "gdn_batch_decode_step")
        return out

    def prefill(self, stream: int, prompt: Sequence[int]) -> int:
        """gdn_batch_prefill: the prompt through one stream's state; returns
        the argmax of the last position (the .gdnstate seed token)."""
        p = np.ascontiguousarray(np.asarray(prompt, np.int32))
        seed = np.zeros(1, np.int32)
        _check(L.load().gdn_batch_prefill(self.ptr, stream, iptr(p), p.size, iptr(seed)), "gdn_batch_prefill")
        return int(seed[0])

    def set_prefill_mode(self, mode: int) -> None:
        """gdn_batch_set_prefill_mode: PREFILL_SCAN (default) or PREFILL_CHUNKED."""
        _check(L.load().gdn_batch_set_prefill_mode(self.ptr, mode), "gdn_batch_set_prefill_mode")

    def set_prefill_segment(self, tokens: int) -> None:
        """gdn_batch_set_prefill_segment: prefill tokens per segment (a multiple of 128)."""
        _check(L.load().gdn_batch_set_prefill_segment(self.ptr, tokens), "gdn_batch_set_prefill_segment")

    def logits(self, stream: int) -> np.ndarray:
        out = np.empty(self.model.config.vocab_size, np.float32)
        _check(L.load().gdn_batch_read_logits(self.ptr, stream, fptr(out), out.size), "gdn_batch_read_logits")
        return out

    def final_hidden(self, stream: int) -> np.ndarray:
        out = np.empty(self.model.config.hidden_size, np.float32)
        _check(L.load().gdn_batch_read_final_hidden(self.ptr, stream, fptr(out), out.size),
               "gdn_batch_read_final_hidden")
        return out

    def load_stream_state(self, stream: int, recurrent: Optional[np.ndarray] = None,
                          conv: Optional[np.ndarray] = None) -> None:
        r = _f32(recurrent).reshape(-1) if recurrent is not None else None
        cv = _f32(conv).reshape(-1) if conv is not None else None
        _check(L.load().gdn_batch_load_stream_state(
            self.ptr, stream, fptr(r) if r is not None else None, r.size if r is not None else 0,
            fptr(cv) if cv is not None else None, cv.size if cv is not None else 0), "gdn_batch_load_stream_state")

    def save_stream_state(self, stream: int) -> Tuple[np.ndarray, np.ndarray]:
        r = np.empty(self.n_state, np.float32)
        cv = np.empty(self.n_conv, np.float32)
        _check(L.load().gdn_batch_save_stream_state(self.ptr, stream, fptr(r), r.size, fptr(cv), cv.size),
               "gdn_batch_save_stream_state")
        return r, cv

    def teacher_forced(self, tokens: np.ndarray, timing: bool = True):
        """tokens [steps][n_streams]; returns (argmax [steps][n_streams], inner_ms, outer_ms)."""
        tk = np.ascontiguousarray(np.asarray(tokens, np.int32))
        steps = tk.shape[0]
        assert tk.shape == (steps, self.n_streams)
        am = np.empty((steps, self.n_streams), np.int32)
        inner = np.empty(steps, np.float32) if timing else None
        outer = np.empty(steps, np.float32) if timing else None
        _check(L.load().gdn_batch_run_teacher_forced(
            self.ptr, iptr(tk), steps, iptr(am), fptr(inner) if timing else None,
            fptr(outer) if timing else None), "gdn_batch_run_teacher_forced")
        return am, inner, outer

    KERNEL_KINDS = ("embed", "qkvg", "recur", "onorm", "o_proj", "layer_norm", "gate_up", "down",
                    "lm_head", "argmax")

    def profile_kernels(self, rounds: int = 2) -> Dict[str, float]:
        out = np.zeros(len(self.KERNEL_KINDS), np.float32)
        _check(L.load().gdn_batch_profile_kernels(self.ptr, rounds, fptr(out), out.size),
               "gdn_batch_profile_kernels")
        return {k: float(v) for k, v in zip(self.KERNEL_KINDS, out)}

    def free(self) -> None:
        if self._live:
            L.load().gdn_batch_free(self.ptr)
            self._live = False

    def __del__(self) -> None:
        try:
            self.free()
        except Exception:
            pass


# ---- seeded generators (counter-based SplitMix64 + Box-Muller) ----

def synth_normal(n: int, seed: int, stream: int, mean: float = 0.0, std: float = 1.0,
                 bf16: bool = False) -> np.ndarray:
    out = np.empty(n, np.float32)
    L.load().gdn_synth_normal(fptr(out), n, seed, stream, mean, std, 1 if bf16 else 0)
    return out


def synth_uniform(n: int, seed: int, stream: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    L.load().gdn_synth_uniform(fptr(out), n, seed, stream, lo, hi)
    return out


def synth_tokens(n: int, seed: int, stream: int, vocab: int = 32000) -> np.ndarray:
    out = np.empty(n, np.int32)
    L.load().gdn_synth_tokens(iptr(out), n, seed, stream, vocab)
    return out


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even to BF16 (finite values), widened back to FP32."""
    u = _f32(x).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32)


# ---- isolated kernels (test hooks) ----

def gemv(contract: int, W: np.ndarray, x: np.ndarray) -> np.ndarray:
    W = _f32(W)
    x = _f32(x)
    M, K = W.shape
    y = np.empty(M, np.float32)
    _check(L.load().gdn_test_gemv(contract, fptr(W), fptr(x), M, K, fptr(y)), "gdn_test_gemv")
    return y


def batch_gemm(W: np.ndarray, X: np.ndarray) -> np.ndarray:
    """gdn_test_batch_gemm: Y [64][N] = X [64][K] W[N][K]^T on the matrix cores."""
    W = _f32(W)
    X = _f32(X)
    N, K = W.shape
    assert X.shape == (L.MAX_STREAMS, K)
    Y = np.empty((L.MAX_STREAMS, N), np.float32)
    _check(L.load().gdn_test_batch_gemm(fptr(W), fptr(X), N, K, fptr(Y)), "gdn_test_batch_gemm")
    return Y


def prefill_gemm(kind: int, W: np.ndarray, X: np.ndarray):
    """gdn_test_prefill_gemm: (prefill GEMM [T][N], the step's GEMM per 64-token block [T][N])."""
    W = _f32(W)
    X = _f32(X)
    T, K = X.shape
    N = W.shape[-2]
    Y = np.empty((T, N), np.float32)
    Y_step = np.empty((T, N), np.float32)
    _check(L.load().gdn_test_prefill_gemm(kind, fptr(W), fptr(X), N, T, fptr(Y), fptr(Y_step)),
           "gdn_test_prefill_gemm")
    return Y, Y_step


def recurrence(contract: int, q, k, v, a, b, a_log, dt_bias, S):
    """q,k,v [steps][heads][256]; a,b,a_log,dt_bias [steps][heads];
    S [heads][256][256] -> (o [steps][heads][256], S')."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    steps, heads = q.shape[0], q.shape[1]
    a, b, a_log, dt_bias = _f32(a), _f32(b), _f32(a_log), _f32(dt_bias)
    S = _f32(S).copy()
    o = np.empty_like(q)
    _check(L.load().gdn_test_recurrence(contract, heads, steps, fptr(q), fptr(k), fptr(v), fptr(a),
                                        fptr(b), fptr(a_log), fptr(dt_bias), fptr(S), fptr(o)),
           "gdn_test_recurrence")
    return o, S
