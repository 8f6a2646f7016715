#!/usr/bin/env python3
"""Batch-1 GatedDeltaNet-1.3B decode on one MI355X.

Workload: the 24-layer GDN-1.3B (hidden 2048, 8 heads x 256, MLP 5632,
vocab 32000, untied LM head), random-init BF16 weights N(0, 0.02) with norm
weights = 1 (seed 0), in the bf16 arm (BF16 weights and operator boundaries,
FP32 recurrent state).  A uniform-random prompt of --warmup tokens builds the
state step by step (untimed); then --steps teacher-forced steps run over a
fixed uniform-random 4096-token stream consumed cyclically.  --contract fp32
runs BASELINE config 4 (FP32 weights, activations and state) the same way,
its GB/s taken at the FP32 byte count.

One step = token id in on the host -> one captured hipGraph of 122 kernels
-> argmax token id back on the host (the reference's "outer" boundary,
host.cpp:945-1047).  `value` is the mean outer ms/token over the timed steps
(wall clock of the whole loop / steps, with no timing events on the stream);
`inner_ms_median` is HIP events around the graph in a separate instrumented
run of up to 1024 steps (the two events cost about 5 us per token).  Achieved GB/s uses the algorithmic bytes per token
(weights + aux + state read/write + conv tails + embedding row + logits).

`roofline` is the dominant kernel kind (largest share of per-token kernel
time in the captured graph): its algorithmic bytes per launch over its mean
duration in the graph, first workgroup's start to last workgroup's end,
from in-kernel phase stamps (the 100 MHz real-time counter) of an
instrumented copy of the step's kernels over --stamp-steps steps, measured
here after the timed leg (gateddeltanet_amd/phase_stamps.py; the stamped
copy runs a few per cent slower, so its durations are upper bounds).  The
HIP-event figure per launch (each kind launched back to back eagerly over
every layer's weights, so it includes a kernel boundary) is printed beside
it.  `cpu_baseline` times the CPU oracle (a port of the reference's native
decode arithmetic, glibc transcendentals) on this host's cores for a few
tokens of the same workload, starting from the GPU's post-prompt state.
Nothing but the engine's own calls runs in a timed window: every step
returns after its argmax has reached host memory.

`secondary` (default run only; --eager or --no-secondary skip it): the other
BASELINE figures measured in the same process after the headline leg --
config 1 (one layer, 64 teacher-forced steps: GPU and CPU oracle), config 4
(FP32 arm, 1024 steps after a 64-token prompt, with its CPU oracle timing),
config 5 (64 streams, 256 timed steps) and the 4096-token prompt pass in
both recurrence modes.  --config 5 and --prefill N run those legs alone, at
full length.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "ms/token batch-1 GDN-1.3B decode (outer); achieved HBM GB/s vs peak"
PEAK_HBM_GBPS = 8000.0
FPGA_OUTER_MS = 8.233  # U55C FPGA outer ms/token, the reference's published figure (architecture.md:1215)

H, I, V, L = 2048, 5632, 32000, 24
# Algorithmic bytes per token (the figures of the hot-path scope table):
DENSE = 2_798_649_344        # 1,399,324,672 BF16 GEMV weights (24 layers + LM head)
AUX = 2_967_040              # norms, a/b rows, conv taps (BF16), a_log/dt_bias (FP32)
STATE_F32 = 100_663_296      # 24 x 8 x 256 x 256 FP32 state, read + write
CONV_BF16 = 1_769_472        # 24 x 3 x 3 x 2048 BF16 conv tails, read + write
EMB_ROW = 4_096              # one BF16 embedding row
LOGITS = 128_000             # FP32 logits written
BYTES_PER_TOKEN = {
    "bf16w_fp32s": DENSE + AUX + STATE_F32 + CONV_BF16 + EMB_ROW + LOGITS,   # 2,904,181,248
    "ref": DENSE + AUX + STATE_F32 // 2 + CONV_BF16 + EMB_ROW + LOGITS,      # 2,853,853,696
    "fp32": 5_707_569_664,   # FP32 weights, state, tails and row
}
# Algorithmic bytes per launch of each kernel kind (bf16 arm): weights at
# BF16 plus the state / conv-tail traffic the kernel must move.
from gateddeltanet_amd.phase_stamps import KERNEL_BYTES  # noqa: E402
# DRAM bytes per launch (FETCH_SIZE + WRITE_SIZE, scaled by a plain copy of
# known size) from the counter passes summarised in
# profiles/k_gemv_cu_gdn13b_bf16w_decode.md (bf16w_fp32s arm).  These are
# constants from that profile, not measured by this run (the bench line says
# so in roofline.traffic_source).
MEASURED_TRAFFIC = {
    "qkvg": 34_382_000, "recur": 4_507_000, "o_proj": 8_718_000, "gate_up": 46_666_000,
    "down": 23_417_000, "lm_head": 131_754_000, "argmax": 7_000,
}
# The FP32 arm's (profiles/k_gemv_cu_gdn13b_fp32_decode.md).
MEASURED_TRAFFIC_FP32 = {
    "qkvg": 67_955_000, "recur": 4_487_000, "o_proj": 17_107_000, "gate_up": 92_689_000,
    "down": 46_421_000, "lm_head": 262_742_000,
}
TRAFFIC_SOURCE = ("rocprofv3 FETCH_SIZE + WRITE_SIZE passes, copy-calibrated "
                  "(profiles/k_gemv_cu_gdn13b_bf16w_decode.md); a profile constant, not measured in this run")
TRAFFIC_SOURCE_FP32 = TRAFFIC_SOURCE.replace("bf16w", "fp32")
LAUNCHES_PER_TOKEN = {"qkvg": L, "recur": L, "qkvg_recur": L, "o_proj": L, "gate_up": L, "down": L, "lm_head": 1,
                      "argmax": 1}


def cpu_baseline(model, contract_id, state, conv, tokens, threads, single_tokens):
    from oracle import oracle as O
    hdr = O.header_from(model.config)
    blob = model.blob
    st = state.copy()
    cv = conv.copy()
    O.set_threads(threads)
    O.decode_step(contract_id, hdr, blob, st, cv, int(tokens[0]), O.LIBM)  # warm caches
    t0 = time.perf_counter()
    n = 0
    for tok in tokens[1:]:
        O.decode_step(contract_id, hdr, blob, st, cv, int(tok), O.LIBM)
        n += 1
    ms = (time.perf_counter() - t0) * 1000.0 / max(n, 1)
    single = None
    if single_tokens > 0:
        O.set_threads(1)
        t0 = time.perf_counter()
        for tok in tokens[:single_tokens]:
            O.decode_step(contract_id, hdr, blob, st, cv, int(tok), O.LIBM)
        single = (time.perf_counter() - t0) * 1000.0 / single_tokens
        O.set_threads(threads)
    return ms, n, single


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4096, help="timed teacher-forced tokens")
    ap.add_argument("--warmup", type=int, default=4096, help="untimed prompt tokens")
    ap.add_argument("--contract", default="bf16w_fp32s", choices=sorted(BYTES_PER_TOKEN))
    ap.add_argument("--profile-rounds", type=int, default=4)
    ap.add_argument("--stamp-steps", type=int, default=256,
                    help="steps of the phase-stamped graph the roofline is taken from (0: HIP events only)")
    ap.add_argument("--cpu-tokens", type=int, default=6, help="oracle tokens timed on all cores (0: skip)")
    ap.add_argument("--cpu-single-tokens", type=int, default=1, help="oracle tokens timed on one core")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy 256 MiB device to device three times (the known-size copy that scales "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    ap.add_argument("--config", type=int, default=3, choices=(3, 5),
                    help="3: batch-1 decode (the headline); 5: --streams independent streams per step "
                         "(multi-stream engine, matrix-core projections)")
    ap.add_argument("--streams", type=int, default=64, help="streams per step for --config 5")
    ap.add_argument("--prefill-mode", default="scan", choices=("scan", "chunked"),
                    help="--prefill recurrence: token-order scan (bit-exact) or the chunked WY form")
    ap.add_argument("--prefill", type=int, default=0,
                    help="instead: time the on-device prefill of an N-token uniform prompt (the GPU prompt pass "
                         "that produces a .gdnstate) against N batch-1 decode steps")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the secondary legs of the default run (config 4, config 5, prefill); "
                         "--eager skips them too")
    ap.add_argument("--eager", action="store_true",
                    help="launch the step's kernels one by one instead of the captured hipGraph "
                         "(for rocprofv3 kernel tracing, which aborts the queue on graph launches)")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch
        a = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": a.numel() * 4, "copies": 3}), flush=True)
        return
    if args.gpus != 1:
        print("bench.py: this build is a single-GPU decode engine; run with --gpus 1 "
              "(no multi-GPU figure is produced)", file=sys.stderr)
        sys.exit(2)

    if args.prefill > 0:
        return main_prefill(args)
    if args.config == 5:
        return main_streams(args)
    out = run_batch1(args.contract, args.steps, args.warmup, args.profile_rounds, args.eager,
                     args.cpu_tokens, args.cpu_single_tokens, args.stamp_steps)
    if args.contract == "bf16w_fp32s" and not args.eager and not args.no_secondary:
        out["secondary"] = secondary_legs()
    print(json.dumps(out), flush=True)


def run_batch1(contract_name, steps, warmup, profile_rounds, eager, cpu_tokens, cpu_single_tokens, stamp_steps=0):
    """One batch-1 decode run (or config 4 with the fp32
    contract): the bench line's fields as a dict."""
    import gateddeltanet_amd as g
    contract = {"ref": g.CONTRACT_REF, "bf16w_fp32s": g.CONTRACT_BF16W_FP32S, "fp32": g.CONTRACT_FP32}[contract_name]
    t_setup = time.perf_counter()
    model = g.Model.synth(num_layers=L, seed=0, std=0.02, bf16=(contract != g.CONTRACT_FP32))
    rs = g.RunState(model, contract)
    if eager:
        rs.set_graph(False)
    prompt = g.synth_tokens(max(warmup, 1), 0, 1, V)
    stream = g.synth_tokens(4096, 0, 2, V)
    if warmup > 0:
        rs.teacher_forced(prompt, warmup, timing=False)
    post_prompt = rs.save_state()
    setup_s = time.perf_counter() - t_setup

    # `value`: the wall clock of an uninstrumented loop (no timing events
    # on the stream; each step returns once its argmax is in host memory);
    # inner / outer medians: a separate instrumented run
    t0 = time.perf_counter()
    rs.teacher_forced(stream, steps, timing=False)
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1000.0 / steps
    _, inner, outer = rs.teacher_forced(stream, min(steps, 1024))

    prof = rs.profile_kernels(profile_rounds)
    per_token = {k: prof[k] * LAUNCHES_PER_TOKEN[k] for k in prof}
    stamps = None
    if stamp_steps > 0 and contract == g.CONTRACT_BF16W_FP32S and not eager:
        from gateddeltanet_amd import phase_stamps as ps
        S, inner_st, inner_pl = ps.stamped_steps(model, stamp_steps, 64, plain_state=rs)
        stamps = ps.summarize(S, L)
        stamps["inner_ms_stamped"] = inner_st
        stamps["inner_ms_plain"] = inner_pl
    if stamps is not None:
        dom, avg_us, _, _ = ps.roofline_from(stamps, KERNEL_BYTES, PEAK_HBM_GBPS)
        avg_source = (f"in-kernel phase stamps of the captured graph (instrumented copy), mean first-workgroup "
                      f"start to last-workgroup end over {stamp_steps} steps x {LAUNCHES_PER_TOKEN[dom]} launches")
    else:
        dom = max(per_token, key=per_token.get)
        avg_us = prof[dom]
        avg_source = "HIP events around back-to-back eager launches over every layer (includes the boundary)"
    kb = KERNEL_BYTES[dom] * (2 if contract == g.CONTRACT_FP32 and dom not in ("recur", "argmax") else 1)
    achieved_k = kb / (avg_us * 1e-6) / 1e9
    achieved_ev = kb / (prof[dom] * 1e-6) / 1e9
    inner_med = float(np.median(inner))
    bytes_tok = BYTES_PER_TOKEN[contract_name]
    achieved = bytes_tok / (inner_med * 1e-3) / 1e9
    achieved_outer = bytes_tok / (ms_per_step * 1e-3) / 1e9

    cpu = None
    if cpu_tokens > 0:
        threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
        ms_cpu, n_cpu, single = cpu_baseline(model, contract, post_prompt[0], post_prompt[1],
                                             stream[:cpu_tokens + 1], threads, cpu_single_tokens)
        cpu = {"value": round(ms_cpu, 3), "unit": "ms/token", "cores": threads, "kind": "port",
               "sample": f"{n_cpu} teacher-forced tokens of the same 24-layer model from the GPU's post-prompt "
                         f"state, CPU oracle (gdn_model.cpp arithmetic, glibc expf/log1pf, OpenMP rows), "
                         f"{threads} threads",
               "single_thread_ms_per_token": None if single is None else round(single, 3)}

    out = {
        "metric": METRIC,
        "value": round(ms_per_step, 5),
        "unit": "ms/token",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": round(ms_per_step / FPGA_OUTER_MS, 5),
        "dtype": "bf16" if contract != g.CONTRACT_FP32 else "fp32",
        "data": "synthetic (seeded random-init weights, uniform random token streams)",
        "config": {
            "workload": ("BASELINE config 4: GatedDeltaNet-1.3B decode with FP32 weights, activations and "
                         "state (precision control arm; GB/s at double the weight bytes), 24 layers, batch 1, "
                         if contract == g.CONTRACT_FP32 else
                         "BASELINE config 3: GatedDeltaNet-1.3B decode, 24 layers, batch 1, ")
                        + f"{warmup}-token uniform prompt then {steps} teacher-forced steps over a "
                        "fixed 4096-token uniform stream (cyclic), greedy argmax",
            "contract": contract_name,
            "state_dtype": "bf16" if contract == g.CONTRACT_REF else "fp32",
            "launch": "eager (122 kernel launches per token)" if eager
                      else "one hipGraph per token (122 kernels)",
        },
        "outer_ms_median": round(float(np.median(outer)), 5),
        "inner_ms_median": round(inner_med, 5),
        "inner_ms_p90": round(float(np.percentile(inner, 90)), 5),
        "bytes_per_token": bytes_tok,
        "achieved_GBps_inner": round(achieved, 1),
        "achieved_GBps_outer": round(achieved_outer, 1),
        "hbm_frac_inner": round(achieved / PEAK_HBM_GBPS, 4),
        "kernel_us_per_launch": {k: round(v, 3) for k, v in prof.items()},
        "kernel_us_per_token": {k: round(v, 2) for k, v in per_token.items()},
        "roofline": {
            "kernel": dom,
            "bound": "hbm",
            "achieved": round(achieved_k, 1),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(achieved_k / PEAK_HBM_GBPS, 4),
            "traffic": (MEASURED_TRAFFIC.get(dom) if contract == g.CONTRACT_BF16W_FP32S else
                        MEASURED_TRAFFIC_FP32.get(dom) if contract == g.CONTRACT_FP32 else None),
            "traffic_source": (TRAFFIC_SOURCE if contract == g.CONTRACT_BF16W_FP32S and dom in MEASURED_TRAFFIC else
                               TRAFFIC_SOURCE_FP32 if contract == g.CONTRACT_FP32 else None),
            "algorithmic_bytes_per_launch": kb,
            "avg_launch_us": round(avg_us, 3),
            "avg_launch_source": avg_source,
            "hip_event_us_per_launch": round(prof[dom], 3),
            "frac_hip_events": round(achieved_ev / PEAK_HBM_GBPS, 4),
        },
        "graph_stamps": None if stamps is None else {
            "steps": stamps["steps"],
            "span_us_mean": round(stamps["span_us_mean"], 1),
            "kernel_us_per_token": round(stamps["kernel_us_per_token"], 1),
            "gap_us_per_token": round(stamps["gap_us_per_token"], 1),
            "gap_us_per_boundary": round(stamps["gap_us_per_boundary"], 3),
            "inner_ms_stamped": round(stamps["inner_ms_stamped"], 5),
            "inner_ms_plain": round(stamps["inner_ms_plain"], 5),
            "kernels": {k: {"dur_us": round(v["dur_us_mean"], 3), "gap_before_us": round(v["gap_before_us_mean"], 3),
                            "input_ready_median_wg_us": round(v.get("input_ready_median_wg_us", float("nan")), 2)}
                        for k, v in stamps["kinds"].items()},
        },
        "cpu_baseline": cpu,
        "setup_s": round(setup_s, 1),
        "vs_baseline_note": "value / 8.233 ms (U55C FPGA outer ms/token, real checkpoint, same arithmetic volume)",
    }
    rs.free()
    model.free()
    return out


# The default run's secondary legs (the "secondary" block of the headline
# line): BASELINE configs 4 and 5 and the prompt pass, measured in the same
# process after the headline leg, at bounded lengths so that the default run
# still finishes within a few minutes.  Decode cost per token does not depend
# on the context length, so the shorter config-4/5 runs time the same step.
SEC_C4_STEPS, SEC_C4_WARMUP, SEC_C4_CPU_TOKENS = 1024, 64, 4
C1_STEPS = 64
SEC_C5_STREAMS, SEC_C5_STEPS, SEC_C5_WARMUP = 64, 256, 16
SEC_PREFILL_TOKENS = 4096


def secondary_legs():
    sec = {"note": "measured in this run after the headline leg, on the same GPU; not part of value"}

    def leg(name, fn):
        try:
            sec[name] = fn()
        except Exception as exc:  # a failed leg is reported; the headline line still prints
            sec[name] = {"error": f"{type(exc).__name__}: {exc}"}

    def c1():
        return run_config1()

    def c4():
        r = run_batch1("fp32", SEC_C4_STEPS, SEC_C4_WARMUP, 1, False, SEC_C4_CPU_TOKENS, 0)
        keep = ("value", "unit", "steps", "warmup", "inner_ms_median", "outer_ms_median", "bytes_per_token",
                "achieved_GBps_inner", "achieved_GBps_outer", "hbm_frac_inner", "kernel_us_per_launch",
                "roofline", "cpu_baseline")
        d = {k: r[k] for k in keep}
        d["workload"] = ("BASELINE config 4: FP32 weights, activations and state, 24 layers, batch 1; "
                         "GB/s at the FP32 byte count")
        return d

    def c5():
        r = run_streams(SEC_C5_STREAMS, SEC_C5_STEPS, SEC_C5_WARMUP, False, 1, 0)
        keep = ("value", "unit", "steps", "warmup", "ms_per_step", "inner_ms_median", "bytes_per_step",
                "achieved_GBps_inner", "hbm_frac_inner", "kernel_us_per_launch")
        d = {k: r[k] for k in keep}
        d["roofline"] = {k: r["roofline"][k] for k in ("kernel", "achieved", "frac", "avg_launch_us")}
        d["workload"] = r["config"]["workload"]
        d["parity"] = r["parity"]
        return d

    def pre(mode):
        r = run_prefill(SEC_PREFILL_TOKENS, mode, False, decode_steps=False)
        return {k: r[k] for k in ("value", "unit", "steps", "prefill_ms", "seed_token")}

    leg("config1_single_layer", c1)
    leg("config4_fp32", c4)
    leg("config5_64_streams", c5)
    leg("prefill_4096_chunked", lambda: pre("chunked"))
    leg("prefill_4096_scan", lambda: pre("scan"))
    return sec


def run_config1():
    """one layer (BF16 weights N(0, 0.02), seed 0), FP32
    state N(0, 0.01), zero conv tails, 64 teacher-forced N(0, 1) BF16 inputs:
    the GPU's layer kernels (gdn_test_layer: one call for the 64 steps, host
    copies of the inputs and outputs included) and the CPU oracle on all
    cores and on one, from the same state."""
    import gateddeltanet_amd as g
    from oracle import oracle as O
    m = g.Model.synth(num_layers=1, seed=0, std=0.02, bf16=True)
    try:
        S0 = g.synth_normal(8 * 256 * 256, 0, 1000, std=0.01)
        xs = g.synth_normal(C1_STEPS * H, 0, 1001, bf16=True).reshape(C1_STEPS, H)
        conv0 = np.zeros(3 * 3 * H, np.float32)
        rs = g.RunState(m, g.CONTRACT_BF16W_FP32S)
        try:
            rs.load_state(S0, conv0)
            rs.layer_steps(0, xs[:4])  # warm
            rs.load_state(S0, conv0)
            t0 = time.perf_counter()
            xo = rs.layer_steps(0, xs)
            gpu_ms = (time.perf_counter() - t0) * 1000.0 / C1_STEPS
        finally:
            rs.free()
        hdr = O.header_from(m.config)
        threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
        res = {}
        for n in (threads, 1):
            O.set_threads(n)
            st, cv = S0.copy(), conv0.copy()
            t0 = time.perf_counter()
            for s in range(C1_STEPS):
                xr, st, cv, _ = O.layer_forward(g.CONTRACT_BF16W_FP32S, hdr, m.blob, 0, xs[s], st, cv, O.LIBM)
            res[n] = (time.perf_counter() - t0) * 1000.0 / C1_STEPS
        O.set_threads(threads)
        same = bool((xo[-1].view(np.uint32) == np.asarray(xr, np.float32).view(np.uint32)).all())
        return {"workload": "BASELINE config 1: one GatedDeltaNet layer, 64 teacher-forced steps, FP32 state "
                            "N(0, 0.01), BF16 N(0, 1) inputs (bf16 weights, FP32-state contract)",
                "gpu_ms_per_step": round(gpu_ms, 4),
                "gpu_note": "gdn_test_layer over the 64 steps in one call, host copies included",
                "cpu_ms_per_step": round(res[threads], 3), "cpu_cores": threads,
                "cpu_single_thread_ms_per_step": round(res[1], 3),
                "cpu_kind": "port (CPU oracle: gdn_model.cpp arithmetic, glibc expf/log1pf)",
                "last_output_bit_exact": same}
    finally:
        m.free()


# Multi-stream decode: per step every stream reads the
# weights once between them and its own FP32 state and conv tails.
PER_STREAM = 102_565_120  # state read + write, conv tails, embedding row, logits (config 5 figure)
STREAM_KERNEL_BYTES = {  # per launch, per stream where the traffic is per stream
    "recur": 8 * 256 * 256 * 4 * 2,
}
# DRAM bytes per recurrence launch (k_brecur<128>) at 64 streams (FETCH_SIZE
# 137.14 MB + WRITE_SIZE 134.74 MB, scaled by a plain copy of known size) from
# the counter passes summarised in profiles/k_bgemm_gdn13b_64stream_decode.md:
# 1.013x the 268.4 MB of state it must read and write.
MEASURED_RECUR_TRAFFIC_64 = 271_884_000


def main_streams(args):
    """--streams independent streams (default 64), each
    with its own FP32 recurrent state and conv tails, one token per stream
    per step; --warmup untimed steps then --steps timed steps, teacher-forced
    with uniform-random tokens.  `value` is aggregate tokens/s (streams x
    steps / wall time of the timed loop, host tokens in -> host tokens out)."""
    steps = args.steps if args.steps != 4096 else 1024
    warm = args.warmup if args.warmup != 4096 else 64
    out = run_streams(args.streams, steps, warm, args.eager, args.profile_rounds, args.cpu_tokens)
    print(json.dumps(out), flush=True)


def run_streams(B, steps, warm, eager, profile_rounds, cpu_tokens):
    """One config-5 run; the bench line's fields as a dict."""
    import gateddeltanet_amd as g
    t_setup = time.perf_counter()
    model = g.Model.synth(num_layers=L, seed=0, std=0.02, bf16=True)
    bs = g.BatchState(model, B)
    if eager:
        bs.set_graph(False)
    toks = g.synth_tokens((warm + steps) * B, 0, 3, V).reshape(warm + steps, B)
    if warm:
        bs.teacher_forced(toks[:warm], timing=False)
    setup_s = time.perf_counter() - t_setup
    t0 = time.perf_counter()
    bs.teacher_forced(toks[warm:], timing=False)  # returns with every stream's token in host memory
    wall = time.perf_counter() - t0
    ms_step = wall * 1000.0 / steps
    _, inner, outer = bs.teacher_forced(toks[warm:warm + min(steps, 256)])
    inner_med = float(np.median(inner))
    bytes_step = DENSE + AUX + B * PER_STREAM
    prof = bs.profile_kernels(profile_rounds)
    per_step = {k: v * (1 if k in ("embed", "lm_head", "argmax") else L) for k, v in prof.items()}
    rb = STREAM_KERNEL_BYTES["recur"] * B
    cpu = None
    if cpu_tokens > 0:
        threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
        st = np.zeros(L * 8 * 256 * 256, np.float32)
        cv = np.zeros(L * 3 * 3 * H, np.float32)
        ms_cpu, n_cpu, _ = cpu_baseline(model, g.CONTRACT_BF16W_FP32S, st, cv, toks[:cpu_tokens + 1, 0],
                                        threads, 0)
        cpu = {"value": round(1000.0 / ms_cpu, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
               "sample": f"{n_cpu} tokens of one stream of the same 24-layer model, CPU oracle (gdn_model.cpp "
                         f"arithmetic, glibc expf/log1pf, OpenMP rows), {threads} threads; streams are "
                         "independent, so the CPU's aggregate rate is this rate"}
    out = {
        "metric": "aggregate tokens/s, 64-stream GDN-1.3B decode (BASELINE config 5)",
        "value": round(B * steps / (wall), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded random-init weights, uniform random token streams)",
        "config": {
            "workload": f"BASELINE config 5: {B} independent GatedDeltaNet-1.3B streams, 24 layers, FP32 "
                        f"states, {steps} teacher-forced steps (one token per stream per step)",
            "streams": B,
            "arithmetic": "BF16 operands, exact products summed in FP32 on the matrix cores for the "
                          "projections; batch-1 BF16W_FP32S arithmetic elsewhere",
            "launch": "eager" if eager else "one hipGraph per step (195 kernels)",
        },
        "parity": ("misses the batch-1 gates against the reference contract by design: exact products summed "
                   "in FP32 on the matrix cores vs the reference's BF16-rounded products in tree16 + bank order; "
                   "24 random layers: logits max-abs 0.24 (gate 2e-2), state rel-L2 5e-2 (gate 1e-3), 94% argmax "
                   "agreement (gate 99.9%); bit-exact where the sums are exact (one-hot model)"),
        "inner_ms_median": round(inner_med, 5),
        "outer_ms_median": round(float(np.median(outer)), 5),
        "bytes_per_step": bytes_step,
        "achieved_GBps_inner": round(bytes_step / (inner_med * 1e-3) / 1e9, 1),
        "hbm_frac_inner": round(bytes_step / (inner_med * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
        "kernel_us_per_launch": {k: round(v, 3) for k, v in prof.items()},
        "kernel_us_per_step": {k: round(v, 1) for k, v in per_step.items()},
        "roofline": {
            "kernel": "recur",
            "bound": "hbm",
            "achieved": round(rb / (prof["recur"] * 1e-6) / 1e9, 1),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(rb / (prof["recur"] * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4),
            "traffic": MEASURED_RECUR_TRAFFIC_64 if B == 64 else None,
            "algorithmic_bytes_per_launch": rb,
            "avg_launch_us": round(prof["recur"], 3),
        },
        "cpu_baseline": cpu,
        "setup_s": round(setup_s, 1),
    }
    bs.free()
    model.free()
    return out


def main_prefill(args):
    """The prompt pass: an N-token uniform prompt through one stream's state
    (gdn_batch_prefill: the prompt as one segment of up to 4096 tokens, run
    layer by layer -- projections as matrix-core GEMMs, the recurrence over
    64-token chunks in token order or in the WY form), timed against the same
    prompt as N batch-1 decode steps (BF16W_FP32S); `value` is prefill
    tokens/s.  The warm-up prefill also allocates the segment buffers."""
    print(json.dumps(run_prefill(args.prefill, args.prefill_mode, args.eager)), flush=True)


def run_prefill(n, mode, eager, decode_steps=True):
    """One prefill run; the bench line's fields as a dict (without the
    decode-steps comparison when decode_steps is false)."""
    import gateddeltanet_amd as g
    model = g.Model.synth(num_layers=L, seed=0, std=0.02, bf16=True)
    prompt = g.synth_tokens(n, 0, 1, V)
    bs = g.BatchState(model, 1)
    chunked = mode == "chunked"
    if chunked:
        bs.set_prefill_mode(g.PREFILL_CHUNKED)
    bs.prefill(0, prompt[:min(n, 128)])  # warm
    t0 = time.perf_counter()
    seed = bs.prefill(0, prompt)  # returns with the seed token (the prompt's last argmax) in host memory
    pre_s = time.perf_counter() - t0
    bs.free()
    dec_s = None
    if decode_steps:
        rs = g.RunState(model, g.CONTRACT_BF16W_FP32S)
        if eager:
            rs.set_graph(False)
        rs.teacher_forced(prompt[:16], 16, timing=False)
        rs.load_state(np.zeros(rs.n_state, np.float32), np.zeros(rs.n_conv, np.float32))
        t0 = time.perf_counter()
        rs.teacher_forced(prompt, n, timing=False)
        dec_s = time.perf_counter() - t0
        rs.free()
    model.free()
    out = {
        "metric": "prefill tokens/s, GDN-1.3B prompt pass (the .gdnstate producer)",
        "value": round(n / pre_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": n,
        "warmup": 0,
        "ms_per_step": round(pre_s * 1000.0 / n, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded random-init weights, uniform random prompt)",
        "config": {"workload": f"{n}-token prompt through one stream, 24 layers, FP32 state, "
                                f"segments of 4096 tokens layer by layer, recurrence chunks of 64",
                   "prefill_mode": mode,
                   "arithmetic": ("the multi-stream step's, with the recurrence in the chunk-parallel (WY) form "
                                  "(FP32 re-association)" if chunked else "the multi-stream step's, bit for bit")},
        "prefill_ms": round(pre_s * 1000.0, 2),
        "decode_steps_ms": None if dec_s is None else round(dec_s * 1000.0, 2),
        "speedup_vs_decode_steps": None if dec_s is None else round(dec_s / pre_s, 2),
        "seed_token": seed,
    }
    return out


if __name__ == "__main__":
    main()
