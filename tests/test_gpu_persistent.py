"""The opt-in persistent step (GDN_PERSIST=1) against the captured graph (gpu).

The persistent step runs a whole token in one cooperative launch; its stages
hand values over as tagged words.  It must give the graph step's results bit
for bit: tokens, logits, final hidden state, recurrent state and conv tails,
over the full 24-layer model and several steps, in both BF16 contracts.  The
exchange area is also checked against the graph step's activation buffers of
the same step (each exchanged value is the BF16 of the activation, or an
FP32 split in two halves), and the phase stamps must be ordered within every
layer."""
import numpy as np
import pytest

import gateddeltanet_amd as g

pytestmark = pytest.mark.gpu

L_FULL = 24
TOKENS = [1, 31999, 12345, 7, 500, 20000, 3, 99]


@pytest.fixture(scope="module")
def model24():
    m = g.Model.synth(num_layers=L_FULL, seed=0, std=0.02, bf16=True)
    yield m
    m.free()


def persistent_state(model, contract, monkeypatch, stamps=False):
    monkeypatch.setenv("GDN_PERSIST", "1")
    if stamps:
        monkeypatch.setenv("GDN_PERSIST_STAMPS", "1")
    rs = g.RunState(model, contract)
    monkeypatch.delenv("GDN_PERSIST")
    monkeypatch.delenv("GDN_PERSIST_STAMPS", raising=False)
    if not rs.persistent:
        rs.free()
        pytest.skip("this device cannot hold the persistent step's grid")
    return rs


def run(rs, tokens):
    out, lg, fh = [], [], []
    for t in tokens:
        out.append(rs.decode_step(t))
        lg.append(rs.logits().copy())
        fh.append(rs.final_hidden().copy())
    return out, np.stack(lg), np.stack(fh), rs.save_state()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_default_is_graph(model24):
    rs = g.RunState(model24, g.CONTRACT_BF16W_FP32S)
    try:
        assert not rs.persistent
        with pytest.raises(RuntimeError):
            rs.set_persistent(True)
    finally:
        rs.free()


@pytest.mark.parametrize("contract", [g.CONTRACT_REF, g.CONTRACT_BF16W_FP32S])
def test_persistent_equals_graph(model24, contract, monkeypatch):
    gr = g.RunState(model24, contract)
    pr = persistent_state(model24, contract, monkeypatch)
    try:
        a = run(gr, TOKENS)
        b = run(pr, TOKENS)
        assert a[0] == b[0]
        assert (bits(a[1]) == bits(b[1])).all()
        assert (bits(a[2]) == bits(b[2])).all()
        assert (bits(a[3][0]) == bits(b[3][0])).all()
        assert (bits(a[3][1]) == bits(b[3][1])).all()
        # switching to the graph and back continues the same trajectory
        pr.set_persistent(False)
        assert not pr.persistent
        gr_next = [gr.decode_step(t) for t in (11, 12)]
        pr_next = [pr.decode_step(t) for t in (11, 12)]
        pr.set_persistent(True)
        assert pr.persistent
        gr_next.append(gr.decode_step(13))
        pr_next.append(pr.decode_step(13))
        assert gr_next == pr_next
        assert (bits(gr.logits()) == bits(pr.logits())).all()
    finally:
        gr.free()
        pr.free()


def test_teacher_forced_persistent(model24, monkeypatch):
    gr = g.RunState(model24, g.CONTRACT_BF16W_FP32S)
    pr = persistent_state(model24, g.CONTRACT_BF16W_FP32S, monkeypatch)
    try:
        toks = np.random.default_rng(3).integers(0, 32000, 24).astype(np.int32)
        am_g = gr.teacher_forced(toks, toks.size, timing=False)[0]
        am_p = pr.teacher_forced(toks, toks.size, timing=False)[0]
        assert np.array_equal(am_g, am_p)
        assert (bits(gr.save_state()[0]) == bits(pr.save_state()[0])).all()
    finally:
        gr.free()
        pr.free()


def _bf16_bits(words):
    return (words & 0xFFFF).astype(np.uint32) << 16


def _f32_bits(words):
    return (((words[1::2] & 0xFFFF) << 16) | (words[0::2] & 0xFFFF)).astype(np.uint32)


def test_exchange_matches_activations(monkeypatch):
    """One layer, one step: every exchanged value against the graph step's
    activation buffer it stands for, and every word carries one tag per
    exchange."""
    m = g.Model.synth(num_layers=1, seed=0, std=0.02, bf16=True)
    gr = g.RunState(m, g.CONTRACT_BF16W_FP32S)
    pr = persistent_state(m, g.CONTRACT_BF16W_FP32S, monkeypatch)
    try:
        assert gr.decode_step(1) == pr.decode_step(1)
        A = gr.activations()
        W = pr.step_buffers(0, 4 * g.EXCHANGE_WORDS)
        X = g.EXCHANGE_REGIONS
        H, I = 2048, 5632

        def region(name, n):
            w = W[X[name]:X[name] + n]
            assert np.unique(w >> 16).size == 1, name
            return w

        def bf16_of(x):
            return bits(g.bf16_round(np.asarray(x, np.float32)))

        assert (_bf16_bits(region("qkv", 3 * H)) == bf16_of(A["qkv"])).all()
        assert (_bf16_bits(region("g", H)) == bf16_of(A["gate"])).all()
        assert (_f32_bits(region("qk_part", 512)) == bits(A["qkpart"])).all()
        assert (_bf16_bits(region("o", H)) == bf16_of(A["attn"])).all()
        assert (_f32_bits(region("osum", 256)) == bits(A["osum"])).all()
        assert (_bf16_bits(region("y_o", H)) == bf16_of(A["ybuf_o"])).all()
        assert (_bf16_bits(region("h", I)) == bf16_of(A["hbuf"])).all()
        assert (_bf16_bits(region("y_down", H)) == bf16_of(A["dbuf"])).all()
    finally:
        gr.free()
        pr.free()
        m.free()


def test_phase_stamps_ordered(model24, monkeypatch):
    pr = persistent_state(model24, g.CONTRACT_BF16W_FP32S, monkeypatch, stamps=True)
    try:
        pr.decode_step(5)
        S = pr.step_buffers(2, 8 * 256 * (L_FULL + 1) * 16).reshape(256, L_FULL + 1, 16).astype(np.int64)
        layers = S[:, :L_FULL, :13]
        assert (layers > 0).all()
        # within a workgroup the layer's phases are in order, and layer l+1
        # starts after layer l ends
        assert (np.diff(layers, axis=2) >= 0).all()
        assert (S[:, 1:L_FULL, 0] >= S[:, :L_FULL - 1, 12]).all()
        lm = S[:, L_FULL, :4]
        assert (np.diff(lm, axis=1) >= 0).all()
    finally:
        pr.free()
