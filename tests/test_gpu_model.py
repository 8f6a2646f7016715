"""The decode engine end to end against the oracle, through the C ABI (gpu).

* Bit-exact against the oracle in ORC_LIBM mode, the reference's arithmetic
  with glibc's expf/log1pf (the engine evaluates glibc's methods, gdn_libm.h):
  one layer over 64 teacher-forced steps, the full
  24-layer model for several tokens in the REF and bf16 (FP32-state)
  contracts and in the FP32 control arm.
* The BASELINE gates (argmax identical, logits max-abs <= 2e-2 (bf16) /
  1e-4 (fp32), recurrent state relative L2 <= 1e-3) follow; the long
  trajectories are in test_gpu_long_horizon.py.
* Host behaviour: graph and eager launches agree, .gdnstate round trip,
  token range check, teacher-forced loop equals single steps, and a step
  taken from a GPU-evolved state (after a long prompt) still matches.
"""
import numpy as np
import pytest

import gateddeltanet_amd as g

pytestmark = pytest.mark.gpu

L_FULL = 24


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(((a.view(np.uint32) == b.view(np.uint32)) | nan).all())


@pytest.fixture(scope="module")
def model_bf16():
    m = g.Model.synth(num_layers=L_FULL, seed=0, std=0.02, bf16=True)
    yield m
    m.free()


@pytest.fixture(scope="module")
def model_1layer():
    m = g.Model.synth(num_layers=1, seed=0, std=0.02, bf16=True)
    yield m
    m.free()


def zero_state(m):
    c = m.config
    return (np.zeros(c.num_layers * 8 * 256 * 256, np.float32),
            np.zeros(c.num_layers * 3 * 3 * 2048, np.float32))


@pytest.mark.parametrize("contract", [g.CONTRACT_REF, g.CONTRACT_BF16W_FP32S])
def test_single_layer_64_steps(orc, model_1layer, contract):
    """one layer, initial state N(0, 0.01) (BF16-rounded
    for REF), zero conv tails, 64 teacher-forced N(0,1) BF16 inputs."""
    m = model_1layer
    hdr = orc.header_from(m.config)
    S0 = g.synth_normal(8 * 256 * 256, 0, 1000, std=0.01)
    if contract == g.CONTRACT_REF:
        S0 = g.bf16_round(S0)
    xs = g.synth_normal(64 * 2048, 0, 1001, bf16=True).reshape(64, 2048)
    rs = g.RunState(m, contract)
    try:
        rs.load_state(S0, np.zeros(3 * 3 * 2048, np.float32))
        xo = rs.layer_steps(0, xs)
        gS, gC = rs.save_state()
    finally:
        rs.free()
    st, cv = S0.copy(), np.zeros(3 * 3 * 2048, np.float32)
    for s in range(64):
        xr, st, cv, _ = orc.layer_forward(contract, hdr, m.blob, 0, xs[s], st, cv, orc.LIBM)
        assert same_bits(xo[s], xr), s
    assert same_bits(gS, st)
    assert same_bits(gC, cv)


@pytest.mark.parametrize("contract", [g.CONTRACT_REF, g.CONTRACT_BF16W_FP32S])
def test_full_model_bit_exact(orc, model_bf16, contract):
    m = model_bf16
    hdr = orc.header_from(m.config)
    st, cv = zero_state(m)
    rs = g.RunState(m, contract)
    try:
        for tok in g.synth_tokens(5, 7, 0):
            gt = rs.decode_step(int(tok))
            ot, ol, ofh = orc.decode_step(contract, hdr, m.blob, st, cv, int(tok), orc.LIBM)
            assert gt == ot
            assert same_bits(rs.logits(), ol)
            assert same_bits(rs.final_hidden(), ofh)
        gS, gC = rs.save_state()
    finally:
        rs.free()
    assert same_bits(gS, st)
    assert same_bits(gC, cv)


def test_fp32_control_arm(orc):
    """BASELINE config 4 (FP32 weights, activations and state): bit-exact to
    the oracle (glibc transcendentals) over a few tokens; the 1024-step run is
    in test_gpu_long_horizon.py."""
    m = g.Model.synth(num_layers=L_FULL, seed=0, std=0.02, bf16=False)
    hdr = orc.header_from(m.config)
    st, cv = zero_state(m)
    rs = g.RunState(m, g.CONTRACT_FP32)
    try:
        for tok in g.synth_tokens(4, 8, 0):
            gt = rs.decode_step(int(tok))
            gl = rs.logits()
            ot, ol, _ = orc.decode_step(2, hdr, m.blob, st, cv, int(tok), orc.LIBM)
            assert gt == ot and same_bits(gl, ol)
        gS, _ = rs.save_state()
    finally:
        rs.free()
        m.free()
    assert same_bits(gS, st)


def test_bf16_gates_against_libm_reference(orc, model_bf16):
    """BASELINE gates for the bf16 arm (FP32 state) against the reference
    arithmetic with glibc expf/log1pf, over 12 teacher-forced tokens (met
    with equality: the logits and state are bit-exact)."""
    m = model_bf16
    hdr = orc.header_from(m.config)
    st, cv = zero_state(m)
    rs = g.RunState(m, g.CONTRACT_BF16W_FP32S)
    agree = 0
    toks = g.synth_tokens(12, 9, 0)
    try:
        for tok in toks:
            gt = rs.decode_step(int(tok))
            ot, ol, _ = orc.decode_step(1, hdr, m.blob, st, cv, int(tok), orc.LIBM)
            agree += int(gt == ot)
            gl = rs.logits()
            assert np.abs(gl - ol).max() <= 2e-2
            assert same_bits(gl, ol)
        gS, _ = rs.save_state()
    finally:
        rs.free()
    assert agree == len(toks)
    assert np.linalg.norm(gS - st) / np.linalg.norm(st) <= 1e-3


def test_graph_and_eager_agree(model_bf16):
    m = model_bf16
    toks = g.synth_tokens(4, 10, 0)
    out = []
    for use_graph in (True, False):
        rs = g.RunState(m, g.CONTRACT_BF16W_FP32S)
        try:
            rs.set_graph(use_graph)
            logits = []
            for t in toks:
                rs.decode_step(int(t))
                logits.append(rs.logits())
            out.append((np.stack(logits), rs.save_state()[0]))
        finally:
            rs.free()
    assert same_bits(out[0][0], out[1][0]) and same_bits(out[0][1], out[1][1])


def test_teacher_forced_loop_matches_single_steps(model_bf16):
    m = model_bf16
    toks = g.synth_tokens(16, 11, 0)
    rs = g.RunState(m, g.CONTRACT_REF)
    try:
        am, inner, outer = rs.teacher_forced(toks, 16)
        s1 = rs.save_state()[0]
    finally:
        rs.free()
    rs = g.RunState(m, g.CONTRACT_REF)
    try:
        single = [rs.decode_step(int(t)) for t in toks]
        s2 = rs.save_state()[0]
    finally:
        rs.free()
    assert list(am) == single
    assert same_bits(s1, s2)
    assert (inner > 0).all() and (outer >= inner * 0.5).all()


def test_gdnstate_round_trip_and_token_check(tmp_path, model_bf16):
    m = model_bf16
    toks = g.synth_tokens(6, 12, 0)
    p = str(tmp_path / "s.gdnstate")
    rs = g.RunState(m, g.CONTRACT_REF)
    try:
        for t in toks[:3]:
            rs.decode_step(int(t))
        rs.save_gdnstate(p, prompt=toks[:3], seed_token=int(toks[3]))
        for t in toks[3:]:
            rs.decode_step(int(t))
        want = rs.logits()
        with pytest.raises(g.GDNError):
            rs.decode_step(m.config.vocab_size)
        with pytest.raises(g.GDNError):
            rs.decode_step(-1)
    finally:
        rs.free()
    rs = g.RunState(m, g.CONTRACT_REF)
    try:
        plen, seed = rs.load_gdnstate(p)
        assert plen == 3 and seed == int(toks[3])
        for t in toks[3:]:
            rs.decode_step(int(t))
        assert same_bits(rs.logits(), want)
    finally:
        rs.free()


def test_step_from_gpu_evolved_state(orc, model_bf16):
    """Size-independent check at the full workload: run a 256-token prompt on
    the GPU, export its state, and take two more steps on both sides from
    that state: bit-exact to the CR oracle."""
    m = model_bf16
    hdr = orc.header_from(m.config)
    rs = g.RunState(m, g.CONTRACT_BF16W_FP32S)
    try:
        rs.teacher_forced(g.synth_tokens(256, 13, 0), 256, timing=False)
        st, cv = rs.save_state()
        assert np.isfinite(st).all() and np.isfinite(cv).all()
        for tok in (17, 31999):
            gt = rs.decode_step(tok)
            ot, ol, _ = orc.decode_step(1, hdr, m.blob, st, cv, tok, orc.LIBM)
            assert gt == ot and same_bits(rs.logits(), ol)
    finally:
        rs.free()
