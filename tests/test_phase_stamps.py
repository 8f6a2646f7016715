"""The phase-stamp reduction (host only) on synthetic stamps with known
figures, and (gpu) stamps of the captured step: every workgroup of every
kernel stamped, in order, one kernel after the other."""
import numpy as np
import pytest

import gateddeltanet_amd as g
from gateddeltanet_amd import phase_stamps as ps


def synthetic(layers, steps, dur=100, ready=30, prod=80, gap=50):
    """Each kernel: every workgroup starts at the kernel's start, stamps its
    input at +ready, products at +prod and ends at +dur (ticks), except that
    the last of several workgroups starts 2 ticks late; kernels follow after
    gap."""
    table = ps.node_table(layers)
    S = np.zeros((steps, len(table), ps.STAMP_WGS, ps.SLOTS), np.int64)
    for s in range(steps):
        t = 1000 + 100000 * s
        for j, (_, _, w) in enumerate(table):
            S[s, j, :w] = [t, t + ready, t + prod, t + dur]
            if w > 1:
                S[s, j, w - 1] = [t + 2, t + ready + 2, t + prod + 2, t + dur + 2]
                t += 2
            t += dur + gap
    return S


def test_summary_of_synthetic_stamps():
    L = 3
    S = synthetic(L, 4)
    sm = ps.summarize(S, L)
    assert sm["nodes"] == 5 * L + 2
    for kind, r in sm["kinds"].items():
        assert r["dur_us_mean"] == pytest.approx(1.00 if kind == "argmax" else 1.02)
        assert r["gap_before_us_mean"] == pytest.approx(0.50)
        if kind != "argmax":
            assert r["input_ready_median_wg_us"] == pytest.approx(0.30)
            assert r["input_ready_last_wg_us"] == pytest.approx(0.32)
            assert r["products_done_last_wg_us"] == pytest.approx(0.82)
    assert sm["kinds"]["qkvg"]["launches_per_token"] == L
    n = 5 * L + 2
    assert sm["span_us_mean"] == pytest.approx((n - 1) * 1.02 + 1.00 + (n - 1) * 0.5)
    assert sm["kernel_us_per_token"] + sm["gap_us_per_token"] == pytest.approx(sm["span_us_mean"])
    dom, us, gbps, frac = ps.roofline_from(sm, ps.KERNEL_BYTES, ps.PEAK_HBM_GBPS)
    # equal durations: the kind with the most launches per token wins the tie
    # among the per-layer kinds (the first of them in dict order)
    assert dom == "qkvg" and us == pytest.approx(1.02)
    assert gbps == pytest.approx(ps.KERNEL_BYTES["qkvg"] / 1.02e-6 / 1e9)
    md = ps.markdown(sm, ps.KERNEL_BYTES, ps.PEAK_HBM_GBPS, "cmd", 0.8, 0.79)
    assert "| gate_up | 3 |" in md and "cmd" in md


def test_recurrence_and_argmax_use_their_own_workgroup_counts():
    table = ps.node_table(24)
    assert len(table) == 122
    assert [w for k, _, w in table if k == "recur"] == [128] * 24
    assert table[-1] == ("argmax", 24, 1)
    # stamps beyond a kernel's workgroups are ignored (left zero on the device)
    S = synthetic(2, 2)
    S[:, 1, 128:] = 0
    S[:, -1, 1:] = 0
    assert ps.summarize(S, 2)["kinds"]["recur"]["dur_us_mean"] == pytest.approx(1.02)


def test_unlaunched_nodes_are_dropped():
    """A step that runs its recurrence inside the QKVG launch leaves the
    recurrence nodes' slots zero: they drop out, and the gaps join the
    launched neighbours."""
    L = 2
    S = synthetic(L, 3)
    for l in range(L):
        S[:, 5 * l + 1] = 0
    nodes = ps.present_nodes(S, L)
    assert len(nodes) == 4 * L + 2 and all(k != "recur" for _, k, _, _ in nodes)
    sm = ps.summarize(S, L)
    assert "recur" not in sm["kinds"] and sm["nodes"] == 4 * L + 2
    # the QKVG launch that runs the recurrence is accounted with both kernels' bytes
    assert "qkvg" not in sm["kinds"] and sm["kinds"]["qkvg_recur"]["launches_per_token"] == L
    assert ps.KERNEL_BYTES["qkvg_recur"] == ps.KERNEL_BYTES["qkvg"] + ps.KERNEL_BYTES["recur"]
    # QKVG -> o_proj now spans the recurrence's 1.02 us and two 0.5 us gaps
    assert sm["kinds"]["o_proj"]["gap_before_us_mean"] == pytest.approx(2.02)
    assert "| recur |" not in ps.markdown(sm, ps.KERNEL_BYTES, ps.PEAK_HBM_GBPS, "cmd", 0.8, 0.79)


@pytest.mark.gpu
def test_graph_stamps_cover_every_kernel(monkeypatch):
    L = 24
    m = g.Model.synth(num_layers=L, seed=0, std=0.02, bf16=True)
    monkeypatch.setenv("GDN_GRAPH_STAMPS", "1")
    rs = g.RunState(m, g.CONTRACT_BF16W_FP32S)
    monkeypatch.delenv("GDN_GRAPH_STAMPS")
    plain = g.RunState(m, g.CONTRACT_BF16W_FP32S)
    try:
        toks = [3, 1000, 31999, 5]
        nodes = 5 * L + 2
        S = np.empty((len(toks), nodes, ps.STAMP_WGS, ps.SLOTS), np.int64)
        for i, t in enumerate(toks):
            # stamping changes no result
            assert rs.decode_step(t) == plain.decode_step(t)
            assert (rs.logits().view(np.uint32) == plain.logits().view(np.uint32)).all()
            S[i] = rs.step_buffers(3, S[i].nbytes).reshape(nodes, ps.STAMP_WGS, ps.SLOTS).astype(np.int64)
        nodes = ps.present_nodes(S, L)
        assert len(nodes) == 5 * L + 2
        for j, kind, _, w in nodes:
            blk = S[:, j, :w]
            assert (blk[:, :, 0] > 0).all() and (blk[:, :, 3] > 0).all(), kind
            if kind != "argmax":
                assert (np.diff(blk, axis=2) >= 0).all(), kind
            else:
                assert (blk[:, :, 3] >= blk[:, :, 0]).all()
        # graph order: each kernel starts after the previous one ends
        P = ps.per_node(S, L)
        assert (P["gap"][:, 1:] > 0).all()
        sm = ps.summarize(S, L)
        assert 0 < sm["span_us_mean"] < 5000
    finally:
        rs.free()
        plain.free()
        m.free()
