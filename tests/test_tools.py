"""Host logit tooling of libgdn_amd.so and the gdn_eval_amd command line,
without a GPU.

* gdn_token_logprob (host.cpp:1954-1995) against scipy's log_softmax in
  float64, plus the invariants that fix it: the probabilities of all targets
  sum to one and a constant shift of the logits changes nothing.
* gdn_strict_argmax (host.cpp:2348-2359): lowest index among equal maxima.
* The GPU-logit vector gate (host.cpp:77-110, :1439-1586) on inputs whose
  metrics have closed forms: identical vectors, a uniform scale (NRMSE = the
  scale error, cosine = 1), one displaced top-5 member, one large error, a
  NaN, and the FP32 tolerance at its edge.
* The CLI's argument and fixture validation, which runs before any device
  call.
"""
import ctypes
import os
import struct
import subprocess

import numpy as np
import pytest
from scipy.special import log_softmax

from gateddeltanet_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "gateddeltanet_amd", "gdn_eval_amd")


def fp(a):
    return a.ctypes.data_as(_lib.FP)


def logprob(v, t):
    v = np.ascontiguousarray(v, np.float32)
    return _lib.load().gdn_token_logprob(fp(v), v.size, t)


def argmax(v):
    v = np.ascontiguousarray(v, np.float32)
    return _lib.load().gdn_strict_argmax(fp(v), v.size)


class Gate:
    def __init__(self):
        self.lib = _lib.load()
        self.p = _lib.GDNLogitsParity()
        self.lib.gdn_logits_parity_init(ctypes.byref(self.p))

    def step(self, actual, reference, selected=None, tol=False):
        a = np.ascontiguousarray(actual, np.float32)
        r = np.ascontiguousarray(reference, np.float32)
        sel = int(np.argmax(r)) if selected is None else selected
        self.lib.gdn_logits_parity_step(ctypes.byref(self.p), fp(a), fp(r), a.size, sel, int(tol))
        return self

    @property
    def nrmse(self):
        return self.lib.gdn_logits_parity_nrmse(ctypes.byref(self.p))

    @property
    def cosine(self):
        return self.lib.gdn_logits_parity_cosine(ctypes.byref(self.p))

    @property
    def passes(self):
        return bool(self.lib.gdn_logits_gate_passes(ctypes.byref(self.p)))


def test_logprob_matches_log_softmax():
    rng = np.random.default_rng(3)
    for scale in (0.1, 3.0, 40.0):
        v = (rng.normal(0, scale, 32000)).astype(np.float32)
        want = log_softmax(v.astype(np.float64))
        for t in (0, 1, 17, 31999, int(np.argmax(v))):
            assert abs(logprob(v, t) - want[t]) <= 1e-9 * max(1.0, abs(want[t]))


def test_logprob_normalises_and_is_shift_invariant():
    rng = np.random.default_rng(4)
    # values on a 1/256 grid so that the +64 shift is exact in float32
    v = (np.round(rng.normal(0, 2, 257) * 256) / 256).astype(np.float32)
    lps = np.array([logprob(v, t) for t in range(v.size)])
    assert abs(np.exp(lps).sum() - 1.0) < 1e-12
    shifted = v + np.float32(64)
    assert ((shifted - np.float32(64)) == v).all()
    lps2 = np.array([logprob(shifted, t) for t in range(v.size)])
    assert np.abs(lps2 - lps).max() < 1e-12
    # single-entry vocabulary: log 1 = 0; uniform: -log V
    assert logprob(np.array([5.0], np.float32), 0) == 0.0
    assert abs(logprob(np.zeros(1000, np.float32), 3) + np.log(1000)) < 1e-12


def test_logprob_rejects_out_of_range_targets():
    v = np.zeros(10, np.float32)
    assert np.isnan(logprob(v, -1)) and np.isnan(logprob(v, 10))


def test_strict_argmax_first_of_ties():
    rng = np.random.default_rng(5)
    for _ in range(20):
        v = rng.integers(-3, 4, 500).astype(np.float32)
        assert argmax(v) == int(np.argmax(v))  # numpy also returns the first maximum
    v = np.full(100, -np.inf, np.float32)
    assert argmax(v) == 0
    v[70] = np.inf
    v[80] = np.inf
    assert argmax(v) == 70
    # a NaN never wins a strict '>' comparison, and one at index 0 stays best
    assert argmax(np.array([1.0, np.nan, 2.0], np.float32)) == 2
    assert argmax(np.array([np.nan, 1.0, 2.0], np.float32)) == 0


def test_gate_identical_vectors():
    rng = np.random.default_rng(6)
    g = Gate()
    for _ in range(3):
        r = rng.normal(0, 3, 32000).astype(np.float32)
        g.step(r, r)
    p = g.p
    assert p.checked_steps == 3 and p.compared_values == 96000
    assert p.exact_mismatches == 0 and p.argmax_mismatches == 0 and p.min_top5_overlap == 5
    assert g.nrmse == 0.0 and abs(g.cosine - 1.0) < 1e-15 and p.worst_step_nrmse == 0.0
    assert g.passes


def test_gate_uniform_scale_has_closed_form_metrics():
    rng = np.random.default_rng(7)
    r = rng.normal(0, 1, 4096).astype(np.float64)
    # reference r32, candidate (1 + eps) r32 rounded once to float32
    r32 = r.astype(np.float32)
    for eps, ok in ((0.005, True), (0.02, False)):
        a = (r32.astype(np.float64) * (1 + eps)).astype(np.float32)
        g = Gate().step(a, r32)
        a64, r64 = a.astype(np.float64), r32.astype(np.float64)
        # the rounding of a to float32 perturbs the closed form by < 2^-24 relative
        assert abs(g.nrmse - eps) < 1e-6
        assert abs(g.p.worst_step_nrmse - eps) < 1e-6
        assert abs(g.cosine - 1.0) < 1e-12 and abs(g.p.min_step_cosine - 1.0) < 1e-12
        assert abs(g.p.max_abs_error - np.abs(a64 - r64).max()) == 0.0
        rms = np.sqrt((r64 ** 2).mean())
        assert abs(g.p.worst_max_abs_over_reference_rms - np.abs(a64 - r64).max() / rms) < 1e-12
        assert g.p.min_top5_overlap == 5 and g.p.argmax_mismatches == 0
        assert g.passes is ok  # 2% > the 1% global NRMSE limit


def test_gate_top5_displacement_and_large_error():
    r = np.zeros(1000, np.float32)
    r[[10, 20, 30, 40, 50]] = [9, 8, 7, 6, 5]
    r[60] = 4.5
    a = r.copy()
    a[60], a[50] = 5.0, 4.5  # the 5th and 6th swap
    g = Gate().step(a, r)
    assert g.p.min_top5_overlap == 4 and g.p.argmax_mismatches == 0
    assert not g.passes
    # one error of 0.6 on an otherwise exact vector: max |err| > 0.5
    a = r.copy()
    a[500] = np.float32(0.6)
    g = Gate().step(a, r)
    assert g.p.min_top5_overlap == 5 and abs(g.p.max_abs_error - np.float32(0.6)) == 0.0
    assert not g.passes


def test_gate_argmax_and_nonfinite():
    r = np.arange(100, dtype=np.float32)
    g = Gate().step(r, r, selected=98)  # the run picked a token that is not the maximum
    assert g.p.argmax_mismatches == 1 and not g.passes
    a = r.copy()
    a[3] = np.nan
    g = Gate().step(a, r, tol=True)
    assert g.p.nonfinite_mismatches == 1 and g.p.tolerance_failures == 1 and g.p.exact_mismatches == 1
    assert not g.passes
    # bit-identical NaNs are no mismatch
    g = Gate().step(a, a, selected=99)
    assert g.p.nonfinite_mismatches == 0 and g.p.exact_mismatches == 0


def test_gate_fp32_tolerance_edge():
    # half the limit 1e-3 + 1e-4 |ref| passes, twice the limit fails
    ref = np.array([0.0, 100.0, -1000.0], np.float32)
    lim = 1e-3 + 1e-4 * np.abs(ref.astype(np.float64))
    inside = (ref.astype(np.float64) + 0.5 * lim).astype(np.float32)
    outside = (ref.astype(np.float64) + 2.0 * lim).astype(np.float32)
    g = Gate().step(inside, ref, selected=1, tol=True)
    assert g.p.tolerance_failures == 0 and g.p.exact_mismatches == 3
    g = Gate().step(outside, ref, selected=1, tol=True)
    assert g.p.tolerance_failures == 3
    g = Gate().step(outside, ref, selected=1, tol=False)
    assert g.p.tolerance_failures == 0


# ----------------------------------------------------------------- the CLI

def run_cli(*args):
    if not os.path.exists(CLI):
        pytest.fail(f"{CLI} is missing: build with __graft_entry__.build()")
    return subprocess.run([CLI, *args], capture_output=True, text=True, timeout=60)


def write_fixture(path, kind, body, magic=b"GDNREQ1\0", version=1, count=None):
    with open(path, "wb") as f:
        f.write(magic + struct.pack("<III", version, kind, len(body) if count is None else count))
        for rec in body:
            f.write(rec)


def ll_example(ctx, cont):
    return struct.pack(f"<II{len(ctx)}i{len(cont)}i", len(ctx), len(cont), *ctx, *cont)


def test_cli_usage_and_argument_errors():
    r = run_cli("--help")
    assert r.returncode == 0 and "--decode-from-state" in r.stdout and "--score" in r.stdout
    r = run_cli("--synth")
    assert r.returncode == 2 and "a mode is required" in r.stderr
    r = run_cli("--synth", "--decode-len", "x", "--decode-from-state", "s")
    assert r.returncode == 2 and "bad value" in r.stderr
    r = run_cli("--synth", "--bogus")
    assert r.returncode == 2 and "unknown option" in r.stderr
    r = run_cli("--synth", "--contract", "fp16", "--score")
    assert r.returncode == 2


def test_cli_rejects_bad_fixtures_before_device_work(tmp_path):
    bad = tmp_path / "bad.gdnreq"
    write_fixture(bad, 2, [ll_example([1, 2], [3])], magic=b"GDNREQ2\0")
    r = run_cli("--synth", str(bad), "--decode-from-state", "s.gdnstate")
    assert r.returncode == 2 and "not a GDNREQ1" in r.stderr
    write_fixture(bad, 2, [ll_example([1, 2], [3])], version=2)
    r = run_cli("--synth", str(bad), "--decode-from-state", "s.gdnstate")
    assert r.returncode == 2 and "version" in r.stderr
    write_fixture(bad, 2, [ll_example([1, 2], [3])], count=2)
    r = run_cli("--synth", str(bad), "--decode-from-state", "s.gdnstate")
    assert r.returncode == 2 and "truncated" in r.stderr
    write_fixture(bad, 2, [ll_example([1, 2], [3]) + b"\0"])
    r = run_cli("--synth", str(bad), "--decode-from-state", "s.gdnstate")
    assert r.returncode == 2 and "trailing" in r.stderr
    write_fixture(bad, 2, [ll_example([1, 2], [3])])
    r = run_cli("--synth", str(bad), "--score")
    assert r.returncode == 2 and "rolling fixture" in r.stderr
    write_fixture(bad, 5, [])
    r = run_cli("--synth", str(bad), "--score")
    assert r.returncode == 2 and "kind" in r.stderr
