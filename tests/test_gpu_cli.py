"""gdn_eval_amd end to end on the GPU (gpu): the command-line driver against
the same model stepped through the library in this process.

* decode-from-state (gdn_eval.cpp:269-529): the trajectory, the GDNLOG1
  logits and GDNHID1 hidden dumps, the post-decode GDNSDMP1 state dump
  (gdn_eval.cpp:464-491) and .gdnstate equal the in-process run bit for bit;
  the host check passes (exit 0); a second run, with an inter-step delay
  (host.cpp:1772-1775), against the first run's logits dump reports no exact
  mismatch and passes the vector gate.  --ftz is refused with a message.
* the steady teacher-forced benchmark (host.cpp:2150-2256) reports every
  step it was asked for; its timed protocol (idle window, timed warmup,
  timed intervals) reports ordered windows and consistent rates.
* rolling scoring (host.cpp:1943-2070) over a kind-3 fixture, with the model
  read from a .gdnw file, gives the log-likelihood of a blank-state
  teacher-forced run scored with float64 log-softmax in numpy.

The CLI builds its model with --synth=1 (seed 0, std 0.02, BF16-rounded),
the same call as Model.synth(num_layers=1) here.
"""
import json
import os
import shutil
import struct
import subprocess
import time

import numpy as np
import pytest
from scipy.special import log_softmax

import gateddeltanet_amd as g
from gateddeltanet_amd import _lib
from test_gpu_dropin import decode_stripes

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "gateddeltanet_amd", "gdn_eval_amd")
N_DECODE = 6
PROMPT = [11, 2222, 333, 31999, 0, 7, 7, 1234]


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return a.shape == b.shape and bool((a.view(np.uint32) == b.view(np.uint32)).all())


def run_cli(*args, timeout=300):
    print(f"[cli] {' '.join(args)}", flush=True)
    r = subprocess.run([CLI, *args], capture_output=True, text=True, timeout=timeout)
    return r


def read_dump(path, magic):
    raw = open(path, "rb").read()
    assert raw[:8] == magic
    version, width, steps = struct.unpack("<III", raw[8:20])
    assert version == 1
    return np.frombuffer(raw[20:], np.float32).reshape(steps, width)


@pytest.fixture(scope="module")
def model():
    m = g.Model.synth(num_layers=1, seed=0, std=0.02, bf16=True)
    yield m
    m.free()


@pytest.fixture(scope="module")
def decoded(model, tmp_path_factory):
    """A .gdnstate after PROMPT, and the in-process decode from it."""
    d = tmp_path_factory.mktemp("cli")
    state = str(d / "prompt.gdnstate")
    rs = g.RunState(model)
    try:
        for t in PROMPT:
            seed = rs.decode_step(t)
        rs.save_gdnstate(state, PROMPT, seed)
        traj, logits, hidden = [seed], [], []
        for _ in range(1, N_DECODE):
            traj.append(rs.decode_step(traj[-1]))
            logits.append(rs.logits())
            hidden.append(rs.final_hidden())
        rec, conv = rs.save_state()
    finally:
        rs.free()
    return dict(dir=d, state=state, traj=traj, logits=np.stack(logits), hidden=np.stack(hidden),
                rec=rec, conv=conv)


def test_decode_from_state_matches_library(model, decoded):
    d = decoded["dir"]
    out, ldump, hdump, sdump, sdmp = (str(d / n) for n in ("dec.json", "l.gdnlog", "h.gdnhid", "after.gdnstate",
                                                           "after.sdmp"))
    r = run_cli("--synth=1", out, "--decode-from-state", decoded["state"], "--decode-len", str(N_DECODE),
                "--logits-dump", ldump, "--hidden-dump", hdump, "--save-gdnstate", sdump, "--dump-state", sdmp)
    assert r.returncode == 0, r.stderr
    res = json.load(open(out))
    ex = res["examples"][0]
    assert res["kind"] == 2 and res["decode_len"] == N_DECODE
    assert ex["gen_traj"] == decoded["traj"] and ex["tf_argmax"] == decoded["traj"]
    assert len(ex["per_step_tpot_ms"]) == N_DECODE and ex["per_step_tpot_ms"][0] == 0.0
    lp = res["logits_parity"]
    assert lp["checked_steps"] == N_DECODE - 1 and lp["compared_values"] == (N_DECODE - 1) * 32000
    assert lp["cpu_tolerance_failures"] == 0 and lp["argmax_mismatches"] == 0
    assert same_bits(read_dump(ldump, b"GDNLOG1\0"), decoded["logits"])
    assert same_bits(read_dump(hdump, b"GDNHID1\0"), decoded["hidden"])
    rs = g.RunState(model)
    try:
        pl, seed = rs.load_gdnstate(sdump)
        rec, conv = rs.save_state()
    finally:
        rs.free()
    assert seed == decoded["traj"][-1]
    assert same_bits(rec, decoded["rec"]) and same_bits(conv, decoded["conv"])
    # GDNSDMP1: header, the four BF16 stripes in the reference's map, then the
    # head buffer (72 conv-tail stripes of 384 beats; the first 3 hold this
    # 1-layer model's BF16 tails in their first 192 beats, the rest zero)
    raw = open(sdmp, "rb").read()
    assert raw[:8] == b"GDNSDMP1"
    beats, ports, hb_beats, zero = struct.unpack("<4I", raw[8:24])
    assert (beats, ports, hb_beats, zero) == (_lib.RECURRENT_STATE_STRIPE_BF16_BEATS, 4, _lib.WSF_HEADBUF // 16, 0)
    assert len(raw) == 24 + (4 * beats + hb_beats) * 64
    rows = 8 * 256
    bits = decode_stripes(raw[24:24 + 4 * beats * 64], rows)
    assert (bits.astype(np.uint32) << 16 == decoded["rec"].view(np.uint32).reshape(rows, 256)).all()
    hb = np.frombuffer(raw[24 + 4 * beats * 64:], np.uint16).reshape(72, 384, 32)
    assert (hb[:3, :192].reshape(-1).astype(np.uint32) << 16 == decoded["conv"].view(np.uint32)).all()
    assert (hb[3:] == 0).all() and (hb[:, 192:] == 0).all()

    # the same run against its own dump, a step every 20 ms: exact, and
    # inside the vector gate; the delay sits outside the step's tpot
    out2 = str(d / "dec2.json")
    t0 = time.monotonic()
    r = run_cli("--synth=1", out2, "--decode-from-state", decoded["state"], "--decode-len", str(N_DECODE),
                "--logits-reference", ldump, "--no-host-check", "--interstep-delay-ms", "20")
    assert r.returncode == 0, r.stderr
    assert time.monotonic() - t0 >= 0.02 * (N_DECODE - 1)
    assert max(json.load(open(out2))["examples"][0]["per_step_tpot_ms"]) < 20.0
    res2 = json.load(open(out2))
    assert res2["logits_parity"]["exact_reference_mismatches"] == 0
    vg = res2["vector_gate"]
    assert vg["passes"] is True and vg["global_nrmse"] == 0.0 and vg["min_top5_overlap"] == 5
    assert res2["examples"][0]["gen_traj"] == decoded["traj"]


def test_ftz_refused(decoded):
    r = run_cli("--synth=1", "--decode-from-state", decoded["state"], "--ftz")
    assert r.returncode != 0 and "--ftz is not supported" in r.stderr


def test_decode_length_from_ll_fixture(decoded):
    """With no --decode-len, N is the first golden continuation length."""
    d = decoded["dir"]
    fx = d / "ll.gdnreq"
    ctx, cont = PROMPT, decoded["traj"][:4]
    with open(fx, "wb") as f:
        f.write(b"GDNREQ1\0" + struct.pack("<III", 1, 2, 1))
        f.write(struct.pack(f"<II{len(ctx)}i{len(cont)}i", len(ctx), len(cont), *ctx, *cont))
    out = str(d / "ll.json")
    r = run_cli("--synth=1", str(fx), out, "--decode-from-state", decoded["state"], "--no-host-check")
    assert r.returncode == 0, r.stderr
    assert json.load(open(out))["examples"][0]["gen_traj"] == decoded["traj"][:4]


def test_benchmark_mode(decoded):
    d = decoded["dir"]
    toks = d / "tokens.txt"
    toks.write_text(" ".join(str(t) for t in PROMPT) + "\n")
    out = str(d / "bench.json")
    r = run_cli("--synth=1", out, "--decode-from-state", decoded["state"], "--benchmark-tokens", str(toks),
                "--benchmark-steps", "40", "--benchmark-warmup", "8")
    assert r.returncode == 0, r.stderr
    res = json.load(open(out))
    assert res["schema"] == "gdn-steady-tpot-v1" and res["token_stream_length"] == len(PROMPT)
    iv = res["intervals"][0]
    assert iv["steps"] == 40 and iv["tokens_per_second"] > 0
    for k in ("production_tpot", "kernel"):
        s = iv[k]
        assert 0 < s["min_ms"] <= s["median_ms"] <= s["p95_ms"] <= s["max_ms"]
    assert iv["kernel"]["median_ms"] <= iv["production_tpot"]["median_ms"]


def test_benchmark_timed_protocol(decoded):
    """The reference's timed protocol (host.cpp:2150-2256): a loaded-idle
    window, a timed warmup, then timed intervals, each with its wall-clock
    bounds and step summaries."""
    d = decoded["dir"]
    toks = d / "tokens_timed.txt"
    toks.write_text(" ".join(str(t) for t in PROMPT) + "\n")
    out = str(d / "bench_timed.json")
    r = run_cli("--synth=1", out, "--decode-from-state", decoded["state"], "--benchmark-tokens", str(toks),
                "--benchmark-idle-seconds", "1", "--benchmark-warmup-seconds", "1",
                "--benchmark-interval-seconds", "1", "--benchmark-intervals", "2")
    assert r.returncode == 0, r.stderr
    res = json.load(open(out))
    assert res["schema"] == "gdn-steady-tpot-v1" and res["warmup_steps"] > 0
    assert res["warmup_start_unix"] - res["idle_start_unix"] >= 0.99
    assert res["warmup_end_unix"] - res["warmup_start_unix"] >= 0.99
    ivs = res["intervals"]
    assert [iv["index"] for iv in ivs] == [0, 1]
    prev_end = res["warmup_end_unix"]
    for iv in ivs:
        assert iv["start_unix"] >= prev_end and iv["end_unix"] - iv["start_unix"] >= 0.99
        prev_end = iv["end_unix"]
        assert iv["steps"] > 0
        assert abs(iv["tokens_per_second"] - iv["steps"] / (iv["end_unix"] - iv["start_unix"])) < 1e-2 * iv["tokens_per_second"]
        for k in ("production_tpot", "kernel"):
            s = iv[k]
            assert 0 < s["min_ms"] <= s["median_ms"] <= s["p95_ms"] <= s["max_ms"]


def test_rolling_score_matches_library(model, tmp_path):
    fx = tmp_path / "rolling.gdnreq"
    docs = [
        (12, 40, [([5, 6, 7], [8, 9])]),
        (30, 120, [([100, 200], [300]), ([31999, 1, 2, 3], [4, 5, 6])]),
    ]
    with open(fx, "wb") as f:
        f.write(b"GDNREQ1\0" + struct.pack("<III", 1, 3, len(docs)))
        for words, nbytes, windows in docs:
            f.write(struct.pack("<III", words, nbytes, len(windows)))
            for ctx, cont in windows:
                f.write(struct.pack(f"<II{len(ctx)}i{len(cont)}i", len(ctx), len(cont), *ctx, *cont))
    if shutil.disk_usage(tmp_path).free < 3 * model.total_floats * 4:
        pytest.skip("not enough scratch disk for a one-layer .gdnw")
    weights = str(tmp_path / "m.gdnw")
    model.save(weights)
    out = str(tmp_path / "score.json")
    r = run_cli(weights, str(fx), out, "--score")
    assert r.returncode == 0, r.stderr
    res = json.load(open(out))

    total, scored = 0.0, 0
    rs = g.RunState(model)
    try:
        for _, _, windows in docs:
            for ctx, cont in windows:
                rs.load_state(np.zeros(rs.n_state, np.float32), np.zeros(rs.n_conv, np.float32))
                toks = ctx + cont
                for i in range(len(toks) - 1):
                    rs.decode_step(toks[i])
                    if i + 1 < len(ctx):
                        continue
                    total += log_softmax(rs.logits().astype(np.float64))[toks[i + 1]]
                    scored += 1
    finally:
        rs.free()
    assert res["documents"] == 2 and res["windows"] == 3 and res["scored_tokens"] == scored == 6
    assert res["words"] == 42 and res["bytes"] == 160
    assert abs(res["total_logprob"] - total) <= 1e-9 * abs(total)
    assert abs(res["word_perplexity"] - np.exp(-total / 42)) <= 1e-9 * np.exp(-total / 42)

    # --score-doc-limit keeps the first document only
    r = run_cli(weights, str(fx), out, "--score", "--score-doc-limit", "1")
    assert r.returncode == 0, r.stderr
    assert json.load(open(out))["scored_tokens"] == 2


def read_gdnstate(path, layers=1):
    raw = open(path, "rb").read()
    assert raw[:8] == b"GDNSTAT1"
    v = struct.unpack("<9I", raw[8:44])
    plen = v[7]
    prompt = list(struct.unpack(f"<{plen}i", raw[44:44 + 4 * plen]))
    off = 44 + 4 * plen
    n_rec = layers * 8 * 256 * 256
    rec = np.frombuffer(raw[off:off + 4 * n_rec], np.float32)
    conv = np.frombuffer(raw[off + 4 * n_rec:], np.float32)
    return v, prompt, rec, conv


def test_prefill_mode_writes_the_stepped_state(model, tmp_path):
    """--prefill (the GPU prompt pass of export_gdn_state.py) writes the
    state, tails, prompt and seed of the prompt stepped through the
    multi-stream engine; --round-bf16 makes it loadable by the REF
    contract; a decode-from-state run continues from it."""
    prompt = [int(t) for t in g.synth_tokens(100, 50, 0)]
    ptxt = tmp_path / "prompt.txt"
    ptxt.write_text(" ".join(map(str, prompt)) + "\n")
    st, out = str(tmp_path / "p.gdnstate"), str(tmp_path / "p.json")
    r = run_cli("--synth=1", out, "--prefill", str(ptxt), "--dump-state", st)
    assert r.returncode == 0, r.stderr
    res = json.load(open(out))
    v, got_prompt, rec, conv = read_gdnstate(st)
    bs = g.BatchState(model, 1)
    try:
        for t in prompt:
            seed = int(bs.step([t])[0])
        rec_ref, conv_ref = bs.save_stream_state(0)
    finally:
        bs.free()
    assert res["prompt_len"] == 100 and res["seed_token"] == seed == v[8] and got_prompt == prompt
    assert same_bits(rec, rec_ref) and same_bits(conv, conv_ref)

    # an LL fixture's context as the prompt, rounded for the REF contract
    fx = tmp_path / "ll.gdnreq"
    ctx, cont = prompt[:37], [1, 2]
    with open(fx, "wb") as f:
        f.write(b"GDNREQ1\0" + struct.pack("<III", 1, 2, 1))
        f.write(struct.pack(f"<II{len(ctx)}i{len(cont)}i", len(ctx), len(cont), *ctx, *cont))
    st2 = str(tmp_path / "p2.gdnstate")
    r = run_cli("--synth=1", str(tmp_path / "p2.json"), "--prefill", str(fx), "--dump-state", st2, "--round-bf16")
    assert r.returncode == 0, r.stderr
    v2, p2, rec2, conv2 = read_gdnstate(st2)
    assert p2 == ctx and v2[7] == 37
    assert ((rec2.view(np.uint32) & 0xFFFF) == 0).all() and ((conv2.view(np.uint32) & 0xFFFF) == 0).all()
    rs = g.RunState(model, g.CONTRACT_REF)
    try:
        assert rs.load_gdnstate(st2) == (37, v2[8])
    finally:
        rs.free()
    r = run_cli("--synth=1", str(tmp_path / "d.json"), "--decode-from-state", st, "--decode-len", "4",
                "--contract", "bf16w")
    assert r.returncode == 0, r.stderr
    assert json.load(open(tmp_path / "d.json"))["examples"][0]["gen_traj"][0] == seed


def test_prefill_chunked_mode_matches_library(model, tmp_path):
    """--prefill-chunked writes what the library's chunked prefill leaves
    (same kernels, so bit for bit), over a prompt that ends mid-chunk."""
    prompt = [int(t) for t in g.synth_tokens(150, 51, 0)]
    ptxt = tmp_path / "prompt.txt"
    ptxt.write_text(" ".join(map(str, prompt)) + "\n")
    st, out = str(tmp_path / "c.gdnstate"), str(tmp_path / "c.json")
    r = run_cli("--synth=1", out, "--prefill", str(ptxt), "--dump-state", st, "--prefill-chunked")
    assert r.returncode == 0, r.stderr
    v, got_prompt, rec, conv = read_gdnstate(st)
    bs = g.BatchState(model, 1)
    try:
        bs.set_prefill_mode(g.PREFILL_CHUNKED)
        seed = bs.prefill(0, prompt)
        rec_ref, conv_ref = bs.save_stream_state(0)
    finally:
        bs.free()
    assert json.load(open(out))["seed_token"] == seed == v[8] and got_prompt == prompt
    assert same_bits(rec, rec_ref) and same_bits(conv, conv_ref)
