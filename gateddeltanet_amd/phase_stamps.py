"""Per-kernel phase stamps of the captured decode step.

A run state made with GDN_GRAPH_STAMPS=1 in the environment has every kernel
of its step (the 122 nodes of the hipGraph for 24 layers) store, from each
workgroup's thread 0, the 100 MHz real-time counter at four points: start,
input ready (the GEMV input built in LDS / the recurrence's products formed),
products done (after the workgroup barrier that ends the weight stream / the
recurrence's column chains) and end (after a final workgroup barrier).  The
stores go through ordinary vector stores after each point; with the variable
unset the kernels only test a null pointer.

This module runs stamped teacher-forced steps and reduces them to the
per-kernel figures of the step as the graph runs it:

* duration: first workgroup's start to last workgroup's end;
* input ready: median and last workgroup, from the kernel's start;
* products done: last workgroup, from the kernel's start;
* gap: the previous kernel's last end to this kernel's first start, i.e. the
  graph's kernel boundary on the real kernel shapes.

python -m gateddeltanet_amd.phase_stamps --steps 256 --md out.md runs the
BASELINE config-3 workload (24 layers, BF16 weights, FP32 state) and writes
the summary.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from typing import Dict, List, Tuple

import numpy as np

TICK_US = 0.01  # the real-time counter runs at 100 MHz
PEAK_HBM_GBPS = 8000.0
H, I, V = 2048, 5632, 32000
# Algorithmic bytes per launch of each kernel kind (bf16 arm): weights at
# BF16 plus the state / conv-tail / activation traffic the kernel must move.
KERNEL_BYTES = {
    "qkvg": 4 * H * H * 2 + 2 * 8 * H * 2 + 3 * H * 4 * 4 + 3 * 3 * H * 2 * 2 + 2 * H * 2,
    "recur": 8 * 256 * 256 * 4 * 2,
    # the fused QKVG + recurrence launch: both kernels' bytes
    "qkvg_recur": (4 * H * H * 2 + 2 * 8 * H * 2 + 3 * H * 4 * 4 + 3 * 3 * H * 2 * 2 + 2 * H * 2
                   + 8 * 256 * 256 * 4 * 2),
    "o_proj": H * H * 2 + 256 * 2,
    "gate_up": 2 * I * H * 2 + H * 2,
    "down": H * I * 2,
    "lm_head": V * H * 2 + H * 2 + V * 4,
    "argmax": (V // 125) * 8,
}
SLOTS = 4
STAMP_WGS = 256
KINDS = ("qkvg", "recur", "o_proj", "gate_up", "down")


def node_table(layers: int, lm_wgs: int = 256) -> List[Tuple[str, int, int]]:
    """(kind, layer, workgroups) of each node in step order."""
    out = []
    for l in range(layers):
        for k in KINDS:
            out.append((k, l, 128 if k == "recur" else 256))
    out.append(("lm_head", layers, lm_wgs))
    out.append(("argmax", layers, 1))
    return out


def collect(rs, tokens: np.ndarray, n_steps: int, layers: int) -> np.ndarray:
    """Run n_steps teacher-forced steps on a stamped run state; the stamps of
    each step as int64 ticks [steps][nodes][256][4]."""
    nodes = 5 * layers + 2
    out = np.empty((n_steps, nodes, STAMP_WGS, SLOTS), np.int64)
    nbytes = 8 * nodes * STAMP_WGS * SLOTS
    for i in range(n_steps):
        rs.decode_step(int(tokens[i % len(tokens)]))
        out[i] = rs.step_buffers(3, nbytes).reshape(nodes, STAMP_WGS, SLOTS).astype(np.int64)
    return out


def present_nodes(S: np.ndarray, layers: int, lm_wgs: int = 256) -> List[Tuple[int, str, int, int]]:
    """(index, kind, layer, workgroups) of the nodes the step launched: a
    node's slots stay zero when the step does not launch it (the recurrence
    when it runs inside the fused QKVG launch)."""
    return [(j, k, l, w) for j, (k, l, w) in enumerate(node_table(layers, lm_wgs)) if (S[:, j, :w, 0] != 0).any()]


def per_node(S: np.ndarray, layers: int, lm_wgs: int = 256) -> Dict[str, np.ndarray]:
    """Per step and launched node (us): start (from the step's first start),
    duration, input ready (median / last workgroup), products done (last
    workgroup), gap before the node (0 for the first)."""
    nodes = present_nodes(S, layers, lm_wgs)
    S = S[:, [j for j, _, _, _ in nodes]]
    table = [(k, l, w) for _, k, l, w in nodes]
    n = S.shape[0]
    N = len(table)
    start = np.empty((n, N))
    end = np.empty((n, N))
    ready_med = np.full((n, N), np.nan)
    ready_max = np.full((n, N), np.nan)
    prod_max = np.full((n, N), np.nan)
    for j, (kind, _, w) in enumerate(table):
        blk = S[:, j, :w, :]
        s0 = blk[:, :, 0].min(axis=1)
        start[:, j] = s0
        end[:, j] = blk[:, :, 3].max(axis=1)
        if kind != "argmax":
            rel1 = blk[:, :, 1] - s0[:, None]
            ready_med[:, j] = np.median(rel1, axis=1)
            ready_max[:, j] = rel1.max(axis=1)
            prod_max[:, j] = (blk[:, :, 2] - s0[:, None]).max(axis=1)
    t0 = start[:, :1]
    gap = np.zeros((n, N))
    gap[:, 1:] = start[:, 1:] - end[:, :-1]
    return {
        "start": (start - t0) * TICK_US,
        "dur": (end - start) * TICK_US,
        "ready_med": ready_med * TICK_US,
        "ready_max": ready_max * TICK_US,
        "prod_max": prod_max * TICK_US,
        "gap": gap * TICK_US,
        "span": (end[:, -1] - start[:, 0]) * TICK_US,
    }


def summarize(S: np.ndarray, layers: int, lm_wgs: int = 256) -> Dict[str, object]:
    """Means over steps (and layers, for the per-layer kinds)."""
    P = per_node(S, layers, lm_wgs)
    table = [(k, l, w) for _, k, l, w in present_nodes(S, layers, lm_wgs)]
    fused = not any(k == "recur" for k, _, _ in table)
    kinds = {}
    for kind in KINDS + ("lm_head", "argmax"):
        cols = [j for j, (k, _, _) in enumerate(table) if k == kind]
        if not cols:
            continue
        if kind == "qkvg" and fused:
            kind = "qkvg_recur"  # the QKVG launch that also runs the recurrence
        d = P["dur"][:, cols]
        row = {
            "launches_per_token": len(cols),
            "dur_us_mean": float(d.mean()),
            "dur_us_median": float(np.median(d)),
            "dur_us_p90": float(np.percentile(d, 90)),
            "gap_before_us_mean": float(P["gap"][:, [j for j in cols if j != 0]].mean()),
            "us_per_token": float(d.mean() * len(cols)),
        }
        if kind != "argmax":
            row["input_ready_median_wg_us"] = float(np.nanmean(P["ready_med"][:, cols]))
            row["input_ready_last_wg_us"] = float(np.nanmean(P["ready_max"][:, cols]))
            row["products_done_last_wg_us"] = float(np.nanmean(P["prod_max"][:, cols]))
        kinds[kind] = row
    busy = float(P["dur"].sum(axis=1).mean())
    gaps = float(P["gap"].sum(axis=1).mean())
    return {
        "steps": int(S.shape[0]),
        "nodes": len(table),
        "span_us_mean": float(P["span"].mean()),
        "span_us_median": float(np.median(P["span"])),
        "kernel_us_per_token": busy,
        "gap_us_per_token": gaps,
        "gap_us_per_boundary": gaps / (len(table) - 1),
        "kinds": kinds,
    }


def roofline_from(summary: Dict[str, object], kernel_bytes: Dict[str, int], peak_gbps: float):
    """The dominant kind (largest stamped time per token) and its achieved
    rate: algorithmic bytes per launch over the mean stamped duration."""
    kinds = summary["kinds"]
    dom = max((k for k in kinds if k in kernel_bytes), key=lambda k: kinds[k]["us_per_token"])
    us = kinds[dom]["dur_us_mean"]
    gbps = kernel_bytes[dom] / (us * 1e-6) / 1e9
    return dom, us, gbps, gbps / peak_gbps


def markdown(summary: Dict[str, object], kernel_bytes: Dict[str, int], peak_gbps: float, command: str,
             inner_ms: float, inner_ms_plain: float) -> str:
    k = summary["kinds"]
    lines = [
        "# Captured decode step, per-kernel phase stamps (GDN-1.3B, bf16 weights, FP32 state)",
        "",
        "Command (GPU box, repository root):",
        "",
        "```",
        command,
        "```",
        "",
        f"{summary['steps']} teacher-forced steps of the 24-layer model, each one launch of the captured "
        f"hipGraph of {summary['nodes']} kernels (the recurrence inside the QKVG launch when that has the fused "
        "form); every workgroup's thread 0 stores the 100 MHz real-time "
        "counter at its start, input ready, products done and end.  Figures are means over the steps "
        "(and the 24 layers for the per-layer kernels); times within a kernel are from its first "
        "workgroup's start; the gap is the previous kernel's last end to this kernel's first start.",
        "",
        "| kernel | per token | duration us (mean / median / p90) | input ready, median WG / last WG (us) | "
        "products done, last WG (us) | gap before (us) | algorithmic bytes | GB/s | frac of 8 TB/s |",
        "|---|---:|---:|---:|---:|---:|---:|---:|---:|",
    ]
    for kind in ("qkvg", "qkvg_recur") + KINDS[1:] + ("lm_head", "argmax"):
        if kind not in k:
            continue
        r = k[kind]
        b = kernel_bytes.get(kind)
        rate = b / (r["dur_us_mean"] * 1e-6) / 1e9 if b and kind != "argmax" else None
        ready = (f"{r['input_ready_median_wg_us']:.2f} / {r['input_ready_last_wg_us']:.2f}"
                 if "input_ready_median_wg_us" in r else "-")
        prod = f"{r['products_done_last_wg_us']:.2f}" if "products_done_last_wg_us" in r else "-"
        lines.append(
            f"| {kind} | {r['launches_per_token']} | {r['dur_us_mean']:.3f} / {r['dur_us_median']:.2f} / "
            f"{r['dur_us_p90']:.2f} | {ready} | {prod} | {r['gap_before_us_mean']:.3f} | "
            f"{b if b else '-':} | {'%.1f' % rate if rate else '-'} | "
            f"{'%.4f' % (rate / peak_gbps) if rate else '-'} |")
    dom, us, gbps, frac = roofline_from(summary, kernel_bytes, peak_gbps)
    lines += [
        "",
        f"- Step span (first kernel's start to the argmax's end): {summary['span_us_mean']:.1f} us mean, "
        f"{summary['span_us_median']:.1f} us median.",
        f"- Kernel time {summary['kernel_us_per_token']:.1f} us + boundary gaps "
        f"{summary['gap_us_per_token']:.1f} us per token ({summary['gap_us_per_boundary']:.3f} us per "
        f"boundary over {summary['nodes'] - 1} boundaries).",
        f"- Inner ms/token (HIP events around the graph) of the stamped run state: {inner_ms:.4f}; "
        f"of an unstamped run state in the same process: {inner_ms_plain:.4f}.",
        f"- Dominant kernel by stamped time per token: **{dom}**, {us:.3f} us per launch, "
        f"{kernel_bytes[dom]:,} algorithmic bytes -> {gbps:.1f} GB/s, frac {frac:.4f} of 8 TB/s.",
        "",
    ]
    return "\n".join(lines)


def stamped_steps(model, steps: int, warmup: int, plain_state=None):
    """Stamped steps of `model` (BF16W_FP32S, the contract the stamped
    kernels are built for) after a warmup-token prompt, plus the inner
    ms/token (median of 256 HIP-event-timed steps) of the stamped run state
    and of an unstamped one (plain_state if given)."""
    import gateddeltanet_amd as g
    old = os.environ.get("GDN_GRAPH_STAMPS")
    os.environ["GDN_GRAPH_STAMPS"] = "1"
    try:
        rs = g.RunState(model, g.CONTRACT_BF16W_FP32S)
    finally:
        if old is None:
            del os.environ["GDN_GRAPH_STAMPS"]
        else:
            os.environ["GDN_GRAPH_STAMPS"] = old
    plain = plain_state if plain_state is not None else g.RunState(model, g.CONTRACT_BF16W_FP32S)
    try:
        vocab = model.config.vocab_size
        prompt = g.synth_tokens(max(warmup, 1), 0, 1, vocab)
        stream = g.synth_tokens(4096, 0, 2, vocab)
        if warmup:
            rs.teacher_forced(prompt, warmup, timing=False)
        S = collect(rs, stream, steps, model.config.num_layers)
        inner = float(np.median(rs.teacher_forced(stream, 256)[1]))
        inner_plain = float(np.median(plain.teacher_forced(stream, 256)[1]))
    finally:
        rs.free()
        if plain_state is None:
            plain.free()
    return S, inner, inner_plain


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--md", default=None, help="write the markdown summary here")
    ap.add_argument("--json", action="store_true", help="print the summary as one JSON line")
    args = ap.parse_args(argv)
    import gateddeltanet_amd as g
    t0 = time.perf_counter()
    model = g.Model.synth(num_layers=24, seed=0, std=0.02, bf16=True)
    try:
        S, inner, inner_plain = stamped_steps(model, args.steps, args.warmup)
    finally:
        model.free()
    summ = summarize(S, 24)
    print(f"phase_stamps: {args.steps} stamped steps in {time.perf_counter() - t0:.1f} s", flush=True)
    cmd = "python -m gateddeltanet_amd.phase_stamps " + " ".join(argv if argv is not None else sys.argv[1:])
    md = markdown(summ, KERNEL_BYTES, PEAK_HBM_GBPS, cmd, inner, inner_plain)
    if args.md:
        with open(args.md, "w") as f:
            f.write(md)
    print(md, flush=True)
    if args.json:
        summ["inner_ms_stamped"] = inner
        summ["inner_ms_plain"] = inner_plain
        print(json.dumps(summ), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
