"""gateddeltanet_amd -- MI355X-native GatedDeltaNet-1.3B decode engine
(batch-1, plus multi-stream decode).

The compute path is libgdn_amd.so (hand-written gfx950 HIP kernels behind the
C ABI of include/gdn_amd.h); this package is its Python host mirror.
"""
from .engine import (  # noqa: F401
    ACTIVATION_LAYOUT,
    CONTRACT_BF16W_FP32S,
    BatchState,
    CONTRACT_FP32,
    CONTRACT_REF,
    EXCHANGE_REGIONS,
    EXCHANGE_WORDS,
    GDNError,
    PREFILL_CHUNKED,
    PREFILL_SCAN,
    Model,
    RunState,
    batch_gemm,
    bf16_round,
    default_config,
    gemv,
    prefill_gemm,
    recurrence,
    synth_normal,
    synth_tokens,
    synth_uniform,
)
