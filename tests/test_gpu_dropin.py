"""The drop-in boundary on the GPU (gpu).

* tests/dropin/gdn_dropin_decode runs the reference driver's call sequence
  (gdn_eval.cpp:202-529, :612-690) against the C ABI: the .gdnstate
  recurrent section is read into run_state.recurrent_state and handed to
  gdn_scatter_recurrent_state through weight_shards[28..31] +
  gdn_weight_shard_beats(); the conv section goes through
  gdn_pack_conv_tails_bf16(head_buffer); the debug buffers receive every
  step's hidden vector and logits; the token line of workspace X_NORM must
  equal a host scan of the logits.  Its trajectory equals the library run in
  this process, its logits pass the reference driver's tolerance against the
  scalar LM head, its native-product counters match counts derived from the
  weights, and its GDNSDMP1-style dump decodes (with the reference's stripe
  map, all_bf16_layout_test.cpp) to the state this process reaches.
* the product counters' exact path: LM-head rows that overflow and flush
  every product are counted as the pinned oracle product classifies them.
* a vocabulary that is no multiple of the LM head's 125-row workgroups
  (32008) decodes bit-exactly against the oracle.
* the step deadline (GDN_KERNEL_WAIT_TIMEOUT_MS) fails the step and the run
  state without waiting for the GPU.
"""
import ctypes
import json
import os
import struct
import subprocess

import numpy as np
import pytest

import gateddeltanet_amd as g
from gateddeltanet_amd import _lib

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DROPIN = os.path.join(ROOT, "tests", "dropin", "gdn_dropin_decode")


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return a.shape == b.shape and bool(((a.view(np.uint32) == b.view(np.uint32)) | nan).all())


def small_model(layers, vocab, seed=0):
    cfg = g.default_config(layers)
    cfg.vocab_size = vocab
    return g.Model.synth(config=cfg, seed=seed, std=0.02, bf16=True)


def write_gdnstate(path, cfg, rec, conv, prompt, seed):
    with open(path, "wb") as f:
        f.write(b"GDNSTAT1")
        f.write(struct.pack("<9I", 1, cfg.num_layers, cfg.num_heads, cfg.head_dim, cfg.head_dim,
                            cfg.hidden_size, cfg.conv_size, len(prompt), seed))
        f.write(np.asarray(prompt, np.int32).tobytes())
        f.write(np.ascontiguousarray(rec, np.float32).tobytes())
        f.write(np.ascontiguousarray(conv, np.float32).tobytes())


def _classes(bits16):
    ex = (bits16 >> 7) & 0xFF
    return (ex == 0) | (ex == 0xFF), (ex == 0) & ((bits16 & 0x7F) != 0)


def slot_weights(m, layer, kind):
    lw = m.layer(layer) if layer is not None else None
    if kind == "qkvg":
        return [lw[n].reshape(2048, 2048) for n in ("q_proj", "k_proj", "v_proj", "g_proj")]
    if kind == "o":
        return [lw["o_proj"].reshape(2048, 2048)]
    if kind == "gu":
        return [lw["mlp_gate_proj"].reshape(5632, 2048), lw["mlp_up_proj"].reshape(5632, 2048)]
    if kind == "down":
        return [lw["mlp_down_proj"].reshape(2048, 5632)]
    return [m.lm_head.reshape(m.config.vocab_size, 2048)]


def expected_input_counts(m, traces, host_lm_head):
    """Special and flushed (subnormal) operand pairs of every native product
    of the steps whose GEMV inputs the oracle traced: a pair counts when
    either operand is special (zero exponent, NaN, infinity) or, for the
    flushed count, subnormal -- the reference's counting rule
    (gdn_model.cpp:421-425).  host_lm_head adds the driver's scalar LM head
    (gdn_compute_logits) on the final hidden vector."""
    cols = {}
    special = flushed = 0
    for ins in traces:
        for layer, kind, x in ins:
            reps = 2 if (kind == "lm" and host_lm_head) else 1
            if (layer, kind) not in cols:
                ws = slot_weights(m, layer, kind)
                bits = [(w.view(np.uint32) >> 16).astype(np.uint16) for w in ws]
                cs = sum(_classes(b)[0].sum(axis=0) for b in bits)
                cf = sum(_classes(b)[1].sum(axis=0) for b in bits)
                cols[(layer, kind)] = (cs, cf, sum(w.shape[0] for w in ws))
            cs, cf, M = cols[(layer, kind)]
            xs, xf = _classes((x.view(np.uint32) >> 16).astype(np.uint16))
            special += reps * int(np.where(xs, M, cs).sum())
            flushed += reps * int(np.where(xf, M, cf).sum())
    return special, flushed


def decode_stripes(raw, rows):
    """The reference's stripe map (all_bf16_layout_test.cpp:41-61): value
    high_half*128 + pair*64 + subhalf*32 + island*16 + lane of row r sits in
    stripe island + 2 high_half, beat 2 r + pair, BF16 lane 16 subhalf + lane."""
    beats = _lib.RECURRENT_STATE_STRIPE_BF16_BEATS
    st = np.frombuffer(raw, np.uint16).reshape(4, beats, 32)
    out = np.zeros((rows, 256), np.uint16)
    for port in range(4):
        island, high = port & 1, port >> 1
        for pair in range(2):
            for sub in range(2):
                v0 = high * 128 + pair * 64 + sub * 32 + island * 16
                out[:, v0:v0 + 16] = st[port, pair:2 * rows:2, 16 * sub:16 * sub + 16]
    return out


def test_reference_driver_call_sequence(orc, tmp_path):
    steps = 5
    m = small_model(2, 512, seed=3)
    c = m.config
    # planted native-multiplier inputs: a zero column in layer 0's q_proj and
    # ten subnormal (BF16-exact) weights in layer 1's down_proj
    q0 = m.layer(0)["q_proj"].reshape(2048, 2048)
    q0[:, 5] = 0.0
    dn = m.layer(1)["mlp_down_proj"]
    dn[100:110] = np.uint32(0x00030000).view(np.float32)
    rng = np.random.default_rng(8)
    rec = g.bf16_round(rng.normal(0, 0.01, 2 * 8 * 256 * 256).astype(np.float32))
    conv = g.bf16_round(rng.normal(0, 1, 2 * 3 * 3 * 2048).astype(np.float32))
    seed_tok = 77
    wpath, spath = str(tmp_path / "m.gdnw"), str(tmp_path / "s.gdnstate")
    out, dump = str(tmp_path / "out.json"), str(tmp_path / "dump.bin")
    m.save(wpath)
    write_gdnstate(spath, c, rec, conv, [1, 2, 3], seed_tok)
    print(f"[dropin] {DROPIN} steps={steps}", flush=True)
    env = dict(os.environ, GDN_COUNTER_TRACE="1")
    r = subprocess.run([DROPIN, wpath, spath, str(steps), out, dump], capture_output=True, text=True, timeout=300,
                       env=env)
    print(r.stderr[-4000:], flush=True)
    assert r.returncode == 0, r.stderr
    res = json.load(open(out))
    print(res["stats"], flush=True)

    rs = g.RunState(m, g.CONTRACT_REF)
    try:
        rs.load_state(rec, conv)
        traj = [seed_tok]
        for _ in range(steps):
            traj.append(rs.decode_step(traj[-1]))
        rec2, conv2 = rs.save_state()
    finally:
        rs.free()
    assert res["traj"] == traj
    assert res["tolerance_failures"] == 0 and res["argmax_mismatches"] == 0

    dense = 2 * (4 * 2048 * 2048 + 2048 * 2048 + 3 * 5632 * 2048) + 512 * 2048
    st = res["stats"]
    # device GEMVs + the driver's scalar LM head, every step
    assert st["calls"] == steps * (dense + 512 * 2048)
    # the pairs with a special or subnormal operand: the planted weights
    # against every normal activation, plus whole rows against the exact
    # zeros BF16 residual adds produce (R(a + b) = 0 when a = -b), taken from
    # the oracle's GEMV inputs along the same trajectory
    hdr = orc.header_from(c)
    ost, ocv = rec.copy(), conv.copy()
    traces = []
    for s_ in range(steps):
        tok, _, _, ins = orc.decode_step_trace(0, hdr, m.blob, ost, ocv, traj[s_], orc.LIBM)
        assert tok == traj[s_ + 1]
        traces.append(ins)
    want_special, want_flushed = expected_input_counts(m, traces, host_lm_head=True)
    assert want_special >= steps * (2048 + 10) and want_flushed >= steps * 10
    assert (st["special_inputs"], st["flushed_inputs"]) == (want_special, want_flushed)
    assert st["flushed_outputs"] == 0 and st["overflows"] == 0

    raw = open(dump, "rb").read()
    assert raw[:8] == b"GDNSDMP1"
    beats, ports, hb_beats, _ = struct.unpack("<4I", raw[8:24])
    assert (beats, ports, hb_beats) == (_lib.RECURRENT_STATE_STRIPE_BF16_BEATS, 4, _lib.WSF_HEADBUF // 16)
    body = raw[24:]
    rows = 2 * 8 * 256
    bits = decode_stripes(body[:4 * beats * 64], rows)
    assert (bits.astype(np.uint32) << 16 == rec2.view(np.uint32).reshape(rows, 256)).all()
    hb = np.frombuffer(body[4 * beats * 64:], np.uint16).reshape(72, 384, 32)
    tails = hb[:6, :192].reshape(6 * 6144).astype(np.uint32) << 16
    assert (tails == conv2.view(np.uint32)).all()
    assert (hb[6:] == 0).all() and (hb[:, 192:] == 0).all()


def test_product_counters_exact_path(orc):
    """LM-head row 0 holds 2^127 and row 1 2^-126 in every column: the
    kernel's fast-path verdict fails, the exact per-product path runs, and
    the counters must hold, per step, the overflows and flushes that the
    pinned oracle product gives for those rows against the step's LM-head
    input (the final hidden vector).  The logits stay bit-exact against the
    oracle, infinities and NaNs included."""
    m = small_model(1, 512, seed=5)
    lm = m.lm_head.reshape(512, 2048)
    lm[0, :] = np.float32(2.0 ** 127)
    lm[1, :] = np.float32(2.0 ** -126)
    hdr = orc.header_from(m.config)
    st = np.zeros(8 * 256 * 256, np.float32)
    cv = np.zeros(3 * 3 * 2048, np.float32)
    lib = _lib.load()
    rs = g.RunState(m, g.CONTRACT_BF16W_FP32S)
    want_flush = want_over = 0
    traces = []
    lm_bits = (lm.view(np.uint32) >> 16).astype(np.uint16)
    try:
        lib.gdn_reset_mixed_mul_stats()
        for tok in (3, 400, 17):
            rs.decode_step(tok)
            _, logits, fh, ins = orc.decode_step_trace(1, hdr, m.blob, st, cv, tok, orc.LIBM)
            traces.append(ins)
            assert same_bits(rs.logits(), logits)
            xb = (fh.view(np.uint32) >> 16).astype(np.uint16)
            ex = (xb >> 7) & 0xFF
            normal = (ex != 0) & (ex != 0xFF)
            p = orc.native_product_array(lm_bits.ravel(), np.tile(xb, 512)).reshape(512, 2048)
            want_over += int((((p & 0x7FFF) == 0x7F80) & normal).sum())
            want_flush += int((((p & 0x7FFF) == 0) & normal).sum())
        s = lib.gdn_get_mixed_mul_stats()
    finally:
        lib.gdn_stop_mixed_mul_stats()
        rs.free()
    assert want_over > 0 and want_flush > 0
    assert s.calls == 3 * ((4 * 2048 * 2048 + 2048 * 2048 + 3 * 5632 * 2048) + 512 * 2048)
    assert (s.flushed_outputs, s.overflows) == (want_flush, want_over)
    assert (s.special_inputs, s.flushed_inputs) == expected_input_counts(m, traces, host_lm_head=False)


def test_vocab_not_multiple_of_125(orc):
    """32008 = 8 x 4001: the LM head runs its 8-row workgroups and writes a
    vocabulary-sized logits buffer (not the 32000-float workspace slot)."""
    m = small_model(1, 32008, seed=9)
    hdr = orc.header_from(m.config)
    st = np.zeros(8 * 256 * 256, np.float32)
    cv = np.zeros(3 * 3 * 2048, np.float32)
    rs = g.RunState(m, g.CONTRACT_BF16W_FP32S)
    try:
        for tok in (32007, 5):
            got = rs.decode_step(tok)
            want, logits, _ = orc.decode_step(1, hdr, m.blob, st, cv, tok, orc.LIBM)
            assert got == want
            assert same_bits(rs.logits(), logits)
    finally:
        rs.free()


def test_step_deadline_fails_the_run_state():
    """A deadline far below one step's duration: gdn_decode_step_host returns
    -1 without waiting for the GPU (which finishes the step on its own), and
    the run state refuses later steps.  24 layers, so the step's GPU time
    (about 0.8 ms) outlasts whatever the first graph launch takes on the
    host before the wait starts (a 1-layer step could finish first)."""
    m = small_model(24, 512, seed=1)
    os.environ["GDN_KERNEL_WAIT_TIMEOUT_MS"] = "0.0001"
    try:
        rs = g.RunState(m, g.CONTRACT_BF16W_FP32S)
    finally:
        del os.environ["GDN_KERNEL_WAIT_TIMEOUT_MS"]
    try:
        with pytest.raises(g.GDNError):
            rs.decode_step(3)
        with pytest.raises(g.GDNError):
            rs.decode_step(4)
    finally:
        rs.free()
    rs = g.RunState(m, g.CONTRACT_BF16W_FP32S)   # the default deadline
    try:
        rs.decode_step(3)
    finally:
        rs.free()


def test_null_token_pointers_are_refused():
    """The stepping entry points refuse missing token arrays with -1 before
    any device work, and the run states stay usable."""
    lib = _lib.load()
    m = small_model(1, 512, seed=3)
    rs = g.RunState(m, g.CONTRACT_BF16W_FP32S)
    bs = g.BatchState(m, 2)
    try:
        assert lib.gdn_decode_step_host(m.ptr, rs.ptr, None) == -1
        assert lib.gdn_run_teacher_forced(rs.ptr, None, 4, 4, None, None, None) == -1
        nxt = (ctypes.c_int32 * 2)()
        toks = (ctypes.c_int32 * 2)(1, 2)
        assert lib.gdn_batch_decode_step(bs.ptr, None, nxt) == -1
        assert lib.gdn_batch_decode_step(bs.ptr, toks, None) == -1
        assert lib.gdn_batch_run_teacher_forced(bs.ptr, None, 3, None, None, None) == -1
        # both engines still step
        assert 0 <= rs.decode_step(7) < 512
        assert lib.gdn_batch_decode_step(bs.ptr, toks, nxt) == 0
        assert all(0 <= int(v) < 512 for v in nxt)
    finally:
        bs.free()
        rs.free()
