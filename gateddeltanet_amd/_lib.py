"""ctypes declarations of libgdn_amd.so (include/gdn_amd.h).

The library is built in-tree by ``__graft_entry__.build()`` (or
``make -C gateddeltanet_amd/csrc``).  Loading fails loudly when it is
missing: there is no CPU fallback for any entry point of the engine.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char, c_float, c_int, c_int32, c_size_t, c_uint16, c_uint32, c_uint64, c_void_p

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libgdn_amd.so")

CONTRACT_REF = 0
CONTRACT_BF16W_FP32S = 1
CONTRACT_FP32 = 2
PREFILL_SCAN = 0     # GDN_PREFILL_SCAN: the recurrence in token order (bit-exact to steps)
PREFILL_CHUNKED = 1  # GDN_PREFILL_CHUNKED: the chunk-parallel (WY) form
MAX_STREAMS = 64  # GDN_MAX_STREAMS
CONTRACT_NAMES = {CONTRACT_REF: "ref", CONTRACT_BF16W_FP32S: "bf16w_fp32s", CONTRACT_FP32: "fp32"}

# Workspace layout in floats (gdn_model.h:54-75 of the reference).
WSF_HID, WSF_HEAD, WSF_MLP = 2048, 16, 5632
WSF_STATE, WSF_HEADBUF, WSF_LOGITS = 12582912, 442368, 32000
WS_OFF_X = 0
WS_OFF_X_NORM = WS_OFF_X + WSF_HID
WS_OFF_Q = WS_OFF_X_NORM + WSF_HID
WS_OFF_K = WS_OFF_Q + WSF_HID
WS_OFF_V = WS_OFF_K + WSF_HID
WS_OFF_A = WS_OFF_V + WSF_HID
WS_OFF_B = WS_OFF_A + WSF_HEAD
WS_OFF_GATE = WS_OFF_B + WSF_HEAD
WS_OFF_ATTN = WS_OFF_GATE + WSF_HID
WS_OFF_TMP_HIDDEN = WS_OFF_ATTN + WSF_HID
WS_OFF_MLP_GATE = WS_OFF_TMP_HIDDEN + WSF_HID
WS_OFF_MLP_UP = WS_OFF_MLP_GATE + WSF_MLP
WS_OFF_REC_STATE = WS_OFF_MLP_UP + WSF_MLP
WS_OFF_HEAD_BUF = WS_OFF_REC_STATE + WSF_STATE
WS_OFF_LOGITS = WS_OFF_HEAD_BUF + WSF_HEADBUF
WS_FLOATS = WS_OFF_LOGITS + WSF_LOGITS


class GDNWeightHeader(ctypes.Structure):
    _fields_ = [
        ("magic", c_char * 8),
        ("version", c_uint32),
        ("vocab_size", c_uint32),
        ("hidden_size", c_uint32),
        ("num_layers", c_uint32),
        ("num_heads", c_uint32),
        ("num_v_heads", c_uint32),
        ("head_dim", c_uint32),
        ("intermediate_size", c_uint32),
        ("conv_size", c_uint32),
        ("max_seq_len", c_uint32),
        ("bos_token_id", c_int32),
        ("eos_token_id", c_int32),
        ("norm_eps", c_float),
    ]


assert ctypes.sizeof(GDNWeightHeader) == 60

_LAYER_FIELDS = [
    "attn_norm", "a_log", "dt_bias", "q_proj", "k_proj", "v_proj", "a_proj", "b_proj",
    "q_conv", "k_conv", "v_conv", "g_proj", "o_norm", "o_proj", "mlp_norm",
    "mlp_gate_proj", "mlp_up_proj", "mlp_down_proj",
]


class GDNLayerWeights(ctypes.Structure):
    _fields_ = [(name, POINTER(c_float)) for name in _LAYER_FIELDS]


class GDNModel(ctypes.Structure):
    _fields_ = [
        ("config", GDNWeightHeader),
        ("weight_data", POINTER(c_float)),
        ("layers", POINTER(GDNLayerWeights)),
        ("embeddings", POINTER(c_float)),
        ("final_norm", POINTER(c_float)),
        ("lm_head", POINTER(c_float)),
    ]


GEMV_CHANNELS = 32
RECURRENT_STATE_PORTS, RECURRENT_STATE_FIRST_PORT = 4, 28
RECURRENT_STATE_STRIPE_BF16_BEATS = WSF_STATE // RECURRENT_STATE_PORTS // 32


class Beat512(ctypes.Structure):
    _fields_ = [("bytes", ctypes.c_ubyte * 64)]


class GDNRunState(ctypes.Structure):
    """gdn_model.h:153-160 field for field (host memory), engine appended."""
    _fields_ = [
        ("workspace", POINTER(Beat512)),
        ("x", POINTER(c_float)),
        ("recurrent_state", POINTER(c_float)),
        ("head_buffer", POINTER(c_float)),
        ("weight_shards", POINTER(Beat512) * GEMV_CHANNELS),
        ("aux_weights", POINTER(Beat512)),
        ("engine", c_void_p),
    ]


class GDNMixedMulStats(ctypes.Structure):
    _fields_ = [
        ("calls", c_uint64),
        ("special_inputs", c_uint64),
        ("flushed_inputs", c_uint64),
        ("flushed_outputs", c_uint64),
        ("overflows", c_uint64),
    ]


class GDNLogitsParity(ctypes.Structure):
    _fields_ = [
        ("checked_steps", c_uint32),
        ("argmax_mismatches", c_uint32),
        ("compared_values", c_uint64),
        ("exact_mismatches", c_uint64),
        ("nonfinite_mismatches", c_uint64),
        ("tolerance_failures", c_uint64),
        ("min_top5_overlap", c_uint32),
        ("reserved", c_uint32),
        ("max_abs_error", ctypes.c_double),
        ("max_rel_error", ctypes.c_double),
        ("squared_error_sum", ctypes.c_double),
        ("candidate_squared_sum", ctypes.c_double),
        ("reference_squared_sum", ctypes.c_double),
        ("dot_product_sum", ctypes.c_double),
        ("worst_step_nrmse", ctypes.c_double),
        ("min_step_cosine", ctypes.c_double),
        ("worst_max_abs_over_reference_rms", ctypes.c_double),
    ]


class GDNBatchState(ctypes.Structure):
    _fields_ = [
        ("engine", c_void_p),
        ("n_streams", c_uint32),
        ("reserved", c_uint32),
    ]


FP = POINTER(c_float)
IP = POINTER(c_int32)
LP = POINTER(GDNLogitsParity)
BP = POINTER(GDNBatchState)

# name -> (restype, argtypes).  Every symbol include/gdn_amd.h declares.
SIGNATURES = {
    "gdn_model_load": (c_int, [POINTER(GDNModel), ctypes.c_char_p]),
    "gdn_model_load_fp32": (c_int, [POINTER(GDNModel), ctypes.c_char_p]),
    "gdn_model_free": (None, [POINTER(GDNModel)]),
    "gdn_model_save": (c_int, [POINTER(GDNModel), ctypes.c_char_p]),
    "gdn_model_synth": (c_int, [POINTER(GDNModel), POINTER(GDNWeightHeader), c_uint64, c_float, c_int]),
    "gdn_validate_bf16_exact_weights": (c_int, [FP, POINTER(GDNWeightHeader)]),
    "gdn_total_weight_floats": (c_size_t, [POINTER(GDNWeightHeader)]),
    "gdn_default_config": (None, [POINTER(GDNWeightHeader), c_uint32]),
    "gdn_run_state_init": (c_int, [POINTER(GDNRunState), POINTER(GDNModel), c_uint32]),
    "gdn_run_state_init_contract": (c_int, [POINTER(GDNRunState), POINTER(GDNModel), c_uint32, c_int]),
    "gdn_run_state_free": (None, [POINTER(GDNRunState)]),
    "gdn_decode_step_host": (c_int, [POINTER(GDNModel), POINTER(GDNRunState), IP]),
    "gdn_read_token": (c_int, [POINTER(GDNRunState), IP]),
    "gdn_read_logits": (c_int, [POINTER(GDNRunState), FP, c_size_t]),
    "gdn_read_final_hidden": (c_int, [POINTER(GDNRunState), FP, c_size_t]),
    "gdn_load_recurrent_state": (c_int, [POINTER(GDNRunState), FP, c_size_t]),
    "gdn_load_conv_tails": (c_int, [POINTER(GDNRunState), FP, c_size_t]),
    "gdn_save_recurrent_state": (c_int, [POINTER(GDNRunState), FP, c_size_t]),
    "gdn_save_conv_tails": (c_int, [POINTER(GDNRunState), FP, c_size_t]),
    "gdn_load_gdnstate": (c_int, [POINTER(GDNRunState), POINTER(GDNModel), ctypes.c_char_p,
                                  POINTER(c_uint32), IP]),
    "gdn_save_gdnstate": (c_int, [POINTER(GDNRunState), POINTER(GDNModel), ctypes.c_char_p, IP,
                                  c_uint32, c_int32]),
    "gdn_write_gdnstate": (c_int, [POINTER(GDNWeightHeader), ctypes.c_char_p, FP, FP, IP, c_uint32, c_int32]),
    "gdn_run_teacher_forced": (c_int, [POINTER(GDNRunState), IP, c_uint32, c_uint32, IP, FP, FP]),
    "gdn_set_graph_mode": (c_int, [POINTER(GDNRunState), c_int]),
    "gdn_set_persistent": (c_int, [POINTER(GDNRunState), c_int]),
    "gdn_get_persistent": (c_int, [POINTER(GDNRunState)]),
    "gdn_test_step_buffers": (c_int, [POINTER(GDNRunState), c_int, c_void_p, c_size_t]),
    "gdn_profile_kernels": (c_int, [POINTER(GDNRunState), c_uint32, FP, c_uint32]),
    "gdn_get_contract": (c_int, [POINTER(GDNRunState)]),
    "gdn_compute_logits": (None, [POINTER(GDNModel), FP, FP]),
    "gdn_weight_shard_beats": (c_size_t, [POINTER(GDNWeightHeader)]),
    "gdn_weight_shard_bytes": (c_size_t, [POINTER(GDNWeightHeader)]),
    "gdn_validate_weight_shards": (c_int, [FP, POINTER(GDNWeightHeader), POINTER(POINTER(Beat512))]),
    "gdn_scatter_recurrent_state": (c_int, [POINTER(POINTER(Beat512)), FP, c_size_t]),
    "gdn_pack_conv_tails_bf16": (c_int, [POINTER(Beat512), FP, c_size_t]),
    "gdn_set_native_debug_buffers": (None, [FP, FP]),
    "gdn_reset_mixed_mul_stats": (None, []),
    "gdn_get_mixed_mul_stats": (GDNMixedMulStats, []),
    "gdn_stop_mixed_mul_stats": (None, []),
    "gdn_sync_host_state": (c_int, [POINTER(GDNRunState)]),
    "gdn_test_set_fp32_lane_bits": (None, [POINTER(Beat512), c_uint32, c_uint32]),
    "gdn_test_get_fp32_lane_bits": (c_uint32, [POINTER(Beat512), c_uint32]),
    "gdn_test_set_bf16_lane_bits": (None, [POINTER(Beat512), c_uint32, c_uint16]),
    "gdn_test_get_bf16_lane_bits": (c_uint16, [POINTER(Beat512), c_uint32]),
    "gdn_native_bf16_mul_to_fp32": (c_float, [c_uint16, c_uint16]),
    "gdn_test_fp32_to_bf16_rne_bits": (c_uint16, [c_uint32]),
    "gdn_test_bf16_to_fp32_bits": (c_uint32, [c_uint16]),
    "gdn_synth_normal": (None, [FP, c_size_t, c_uint64, c_uint64, c_float, c_float, c_int]),
    "gdn_synth_uniform": (None, [FP, c_size_t, c_uint64, c_uint64, c_float, c_float]),
    "gdn_synth_tokens": (None, [IP, c_size_t, c_uint64, c_uint64, c_uint32]),
    "gdn_test_gemv": (c_int, [c_int, FP, FP, c_uint32, c_uint32, FP]),
    "gdn_test_recurrence": (c_int, [c_int, c_uint32, c_uint32, FP, FP, FP, FP, FP, FP, FP, FP, FP]),
    "gdn_test_layer": (c_int, [POINTER(GDNRunState), c_uint32, c_uint32, FP, FP]),
    "gdn_test_libm_array": (None, [c_int, FP, FP, c_size_t]),
    "gdn_recurrence_noalloc": (c_int, [c_int, c_uint32, c_uint32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "gdn_logits_parity_init": (None, [LP]),
    "gdn_logits_parity_step": (None, [LP, FP, FP, c_uint32, c_uint32, c_int]),
    "gdn_logits_parity_nrmse": (ctypes.c_double, [LP]),
    "gdn_logits_parity_cosine": (ctypes.c_double, [LP]),
    "gdn_logits_gate_passes": (c_int, [LP]),
    "gdn_token_logprob": (ctypes.c_double, [FP, c_uint32, c_int32]),
    "gdn_strict_argmax": (c_uint32, [FP, c_uint32]),
    "gdn_batch_init": (c_int, [BP, POINTER(GDNModel), c_uint32]),
    "gdn_batch_free": (None, [BP]),
    "gdn_batch_decode_step": (c_int, [BP, IP, IP]),
    "gdn_batch_read_tokens": (c_int, [BP, IP]),
    "gdn_batch_read_logits": (c_int, [BP, c_uint32, FP, c_size_t]),
    "gdn_batch_read_final_hidden": (c_int, [BP, c_uint32, FP, c_size_t]),
    "gdn_batch_load_stream_state": (c_int, [BP, c_uint32, FP, c_size_t, FP, c_size_t]),
    "gdn_batch_save_stream_state": (c_int, [BP, c_uint32, FP, c_size_t, FP, c_size_t]),
    "gdn_batch_run_teacher_forced": (c_int, [BP, IP, c_uint32, IP, FP, FP]),
    "gdn_batch_prefill": (c_int, [BP, c_uint32, IP, c_uint32, IP]),
    "gdn_batch_set_prefill_mode": (c_int, [BP, c_int]),
    "gdn_batch_set_prefill_segment": (c_int, [BP, c_uint32]),
    "gdn_batch_profile_kernels": (c_int, [BP, c_uint32, FP, c_uint32]),
    "gdn_batch_set_graph_mode": (c_int, [BP, c_int]),
    "gdn_test_batch_gemm": (c_int, [FP, FP, c_uint32, c_uint32, FP]),
    "gdn_test_prefill_gemm": (c_int, [c_int, FP, FP, c_uint32, c_uint32, FP, FP]),
    "gdn_test_tile_bf16": (None, [POINTER(c_uint16), c_size_t, c_size_t, c_int, POINTER(c_uint16)]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load libgdn_amd.so and declare every entry point; raise if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "(the engine has no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib
