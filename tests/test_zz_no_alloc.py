"""gdn_recurrence_noalloc (the allocation-free variant of gdn_test_recurrence)
against gdn_test_recurrence, through the C ABI (gpu).

Bar: bit-exact (the same kernels' arithmetic on the same inputs).  Two calls
in a row share the library's fixed device scratch array: the first spans two
scratch fills (192 heads x 100 steps, 85 steps per fill), the second is
smaller (16 heads x 40 steps), so stale pairs from the first call would show
up in the second's results.  The test, as the caller, allocates its device
buffers through the HIP runtime the library itself loaded (libamdhip64 of
the ROCm install); the entry point allocates nothing.
"""
import ctypes
import os

import numpy as np
import pytest

import gateddeltanet_amd as g
from gateddeltanet_amd import _lib

pytestmark = pytest.mark.gpu


def _inputs(seed, steps, heads, contract):
    rng = np.random.default_rng(seed)
    q = rng.normal(0, 1, (steps, heads, 256)).astype(np.float32)
    k = rng.normal(0, 1, (steps, heads, 256)).astype(np.float32)
    v = rng.normal(0, 1, (steps, heads, 256)).astype(np.float32)
    a = rng.normal(0, 1, (steps, heads)).astype(np.float32)
    b = rng.normal(0, 1, (steps, heads)).astype(np.float32)
    al = rng.uniform(0, np.log(16), (steps, heads)).astype(np.float32)
    dt = rng.normal(0, 0.5, (steps, heads)).astype(np.float32)
    S = rng.normal(0, 0.01, (heads, 256, 256)).astype(np.float32)
    if contract != g.CONTRACT_FP32:
        q, k, v, a, b = map(g.bf16_round, (q, k, v, a, b))
    if contract == g.CONTRACT_REF:
        S = g.bf16_round(S)
    return q, k, v, a, b, al, dt, S


def _hip():
    """The libamdhip64 that libgdn_amd.so runs on: the process must map
    exactly one HIP runtime, so the caller-side allocations and copies here
    and the library's kernels share it."""
    _lib.load()
    paths = set()
    for line in open("/proc/self/maps"):
        fields = line.split()
        if len(fields) >= 6 and "libamdhip64.so" in fields[-1]:
            paths.add(os.path.realpath(fields[-1]))
    assert len(paths) == 1, f"expected one HIP runtime in the process, found {sorted(paths)}"
    hip = ctypes.CDLL(paths.pop())
    hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipFree.argtypes = [ctypes.c_void_p]
    return hip


H2D, D2H = 1, 2


def _to_device(hip, arr, keep):
    p = ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(p), arr.nbytes) == 0
    keep.append(p)
    assert hip.hipMemcpy(p, arr.ctypes.data, arr.nbytes, H2D) == 0
    return p


def _noalloc(contract, q, k, v, a, b, al, dt, S):
    hip = _hip()
    steps, heads = a.shape
    keep = []
    try:
        ins = [_to_device(hip, np.ascontiguousarray(x, np.float32), keep) for x in (q, k, v, a, b, al, dt)]
        if contract == g.CONTRACT_REF:
            s_host = (S.view(np.uint32) >> 16).astype(np.uint16)
        else:
            s_host = np.ascontiguousarray(S, np.float32).copy()
        dS = _to_device(hip, s_host, keep)
        o = np.zeros((steps, heads, 256), np.float32)
        do = _to_device(hip, o, keep)
        rc = _lib.load().gdn_recurrence_noalloc(contract, heads, steps, *ins, dS, do, None)
        assert rc == 0
        assert hip.hipDeviceSynchronize() == 0
        assert hip.hipMemcpy(o.ctypes.data, do, o.nbytes, D2H) == 0
        back = np.empty_like(s_host)
        assert hip.hipMemcpy(back.ctypes.data, dS, back.nbytes, D2H) == 0
    finally:
        for p in keep:
            hip.hipFree(p)
    if contract == g.CONTRACT_REF:
        S2 = (back.astype(np.uint32) << 16).view(np.float32)
    else:
        S2 = back
    return o, S2.reshape(heads, 256, 256)


def _same(a, b):
    return bool((np.asarray(a, np.float32).view(np.uint32) == np.asarray(b, np.float32).view(np.uint32)).all())


@pytest.mark.parametrize("contract", [g.CONTRACT_BF16W_FP32S, g.CONTRACT_REF, g.CONTRACT_FP32])
def test_noalloc_recurrence_matches_allocating_entry_point(contract):
    for seed, steps, heads in ((11 + contract, 100, 192), (23 + contract, 40, 16)):
        q, k, v, a, b, al, dt, S = _inputs(seed, steps, heads, contract)
        print(f"noalloc contract={contract} heads={heads} steps={steps}", flush=True)
        o_ref, S_ref = g.recurrence(contract, q, k, v, a, b, al, dt, S)
        o, S2 = _noalloc(contract, q, k, v, a, b, al, dt, S)
        assert _same(o, o_ref), (contract, heads, steps)
        assert _same(S2, S_ref), (contract, heads, steps)


def test_noalloc_rejects_oversized_and_bad_arguments():
    lib = _lib.load()
    null = ctypes.c_void_p(0)
    ptrs = [ctypes.c_void_p(1)] * 9
    assert lib.gdn_recurrence_noalloc(1, 16385, 1, *ptrs, null) == -1   # more heads than the scratch holds
    assert lib.gdn_recurrence_noalloc(7, 8, 1, *ptrs, null) == -1       # unknown contract
    assert lib.gdn_recurrence_noalloc(1, 8, 0, *ptrs, null) == 0        # nothing to do
    assert lib.gdn_recurrence_noalloc(1, 8, 1, *([null] + ptrs[1:]), null) == -1
