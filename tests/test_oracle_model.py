"""The oracle's model composition against a textbook fp64 GatedDeltaNet.

The fp64 model below is written from the layer's mathematics (the
reference's lit_gpt GatedDeltaNet block with its recurrent formulation,
chunk.py:688-718, and the decode wiring of gdn_forward, gdn_model.cpp:
3741-3890): RMSNorm -> q/k/v/g and a/b projections -> causal depthwise conv
(width 4) + SiLU on q/k/v -> per-head L2-normalised gated delta rule ->
per-head RMSNorm * g * sigmoid(g) -> o_proj + residual -> RMSNorm -> SwiGLU
MLP + residual, then final RMSNorm and the LM head.  It pins which tensor
feeds which operation; rounding and reduction orders are pinned by
test_oracle_ops.py and test_oracle_bf16.py.
"""
import numpy as np
import pytest

import gateddeltanet_amd as g


def small_model(layers=2, vocab=512, seed=0, bf16=False):
    cfg = g.default_config(layers)
    cfg.vocab_size = vocab
    return g.Model.synth(config=cfg, seed=seed, bf16=bf16)


def rms(x, w, eps=1e-6):
    return x / np.sqrt(np.mean(x * x) + eps) * w


def silu(x):
    return x / (1.0 + np.exp(-x))


def softplus(x):
    return np.log1p(np.exp(x))


def textbook_step(m, state, conv, token):
    c = m.config
    H, nh, hd, I = c.hidden_size, c.num_heads, c.head_dim, c.intermediate_size
    x = m.embeddings.reshape(c.vocab_size, H)[token].astype(np.float64)
    for l in range(c.num_layers):
        w = {k: v.astype(np.float64) for k, v in m.layer(l).items()}
        xn = rms(x, w["attn_norm"])
        q = w["q_proj"].reshape(H, H) @ xn
        k = w["k_proj"].reshape(H, H) @ xn
        v = w["v_proj"].reshape(H, H) @ xn
        gg = w["g_proj"].reshape(H, H) @ xn
        a = w["a_proj"].reshape(nh, H) @ xn
        b = w["b_proj"].reshape(nh, H) @ xn
        outs = []
        for kind, (raw, cw) in enumerate(((q, w["q_conv"]), (k, w["k_conv"]), (v, w["v_conv"]))):
            tails = conv[l, kind]                     # [3][H], oldest first
            window = np.vstack([tails, raw[None, :]])  # [4][H]
            s = (window.T * cw.reshape(H, 4)).sum(axis=1)
            outs.append(silu(s))
            conv[l, kind] = np.vstack([tails[1:], raw[None, :]])
        qc, kc, vc = outs
        o = np.zeros(H)
        for h in range(nh):
            sl = slice(h * hd, (h + 1) * hd)
            qn = qc[sl] / np.sqrt((qc[sl] ** 2).sum() + 1e-6)
            kn = kc[sl] / np.sqrt((kc[sl] ** 2).sum() + 1e-6)
            beta = 1.0 / (1.0 + np.exp(-b[h]))
            decay = np.exp(-np.exp(w["a_log"][h]) * softplus(a[h] + w["dt_bias"][h]))
            S = state[l, h]
            S[:] = decay * S + np.outer(kn, beta * (vc[sl] - decay * (S.T @ kn)))
            o[sl] = S.T @ qn / np.sqrt(hd)
        og = np.concatenate([rms(o[h * hd:(h + 1) * hd], w["o_norm"]) for h in range(nh)]) * gg * (
            1.0 / (1.0 + np.exp(-gg)))
        x = x + w["o_proj"].reshape(H, H) @ og
        xn2 = rms(x, w["mlp_norm"])
        hh = silu(w["mlp_gate_proj"].reshape(I, H) @ xn2) * (w["mlp_up_proj"].reshape(I, H) @ xn2)
        x = x + w["mlp_down_proj"].reshape(H, I) @ hh
    xf = rms(x, m.final_norm.astype(np.float64))
    return m.lm_head.reshape(c.vocab_size, H).astype(np.float64) @ xf


@pytest.mark.parametrize("contract,rtol", [(2, 2e-4), (1, 4e-2)])
def test_oracle_decode_matches_textbook(orc, contract, rtol):
    m = small_model(bf16=(contract != 2))
    c = m.config
    hdr = orc.header_from(c)
    L = c.num_layers
    rng = np.random.default_rng(12)
    state0 = rng.normal(0, 0.01, (L, 8, 256, 256)).astype(np.float32)
    st = state0.reshape(-1).copy()
    cv = np.zeros(L * 3 * 3 * 2048, np.float32)
    st64 = state0.astype(np.float64)
    cv64 = np.zeros((L, 3, 3, 2048))
    for token in (5, 77, 300):
        tok, logits, _ = orc.decode_step(contract, hdr, m.blob, st, cv, token, orc.CR)
        ref = textbook_step(m, st64, cv64, token)
        err = np.abs(logits - ref).max() / np.abs(ref).max()
        assert err < rtol, err
        assert tok == int(np.argmax(logits))
    np.testing.assert_allclose(st.reshape(st64.shape), st64, rtol=0, atol=rtol * np.abs(st64).max())


def test_compute_logits_matches_gemv(orc):
    """gdn_compute_logits (sequential sum) agrees with the banked LM head to
    the reference's own tolerance (gdn_eval.cpp:375-379)."""
    m = small_model(layers=1, bf16=True)
    hdr = orc.header_from(m.config)
    h = g.bf16_round(np.random.default_rng(13).normal(0, 1, 2048).astype(np.float32))
    a = orc.compute_logits(hdr, m.blob, h)
    b = orc.gemv(0, m.lm_head.reshape(m.config.vocab_size, 2048), h)
    assert (np.abs(a - b) <= 1e-3 + 1e-4 * np.abs(b)).all()


def test_compute_logits_sums_in_hidden_order(orc):
    """gdn_compute_logits, gdn_model.cpp:3953-3961: sum += product for
    hidden index 0..H-1 in order, from +0.0f.

    Row 0: products 2^24 (index 0), 1 (index 1), 1, 1 (indices 1000, 1001).
    In order each +1 onto 2^24 is a tie that rounds back: 2^24.  A reversed
    sum gives 2^24 + 4, and the banked GEMV order (the 1s at 1000, 1001 meet
    first in one half-beat) gives 2^24 + 2.
    Row 1: products 1, 1, 1 (indices 10..12) then 2^24 (index 13): in order
    3 + 2^24 = 2^24 + 3, which rounds to 2^24 + 4; reversed gives 2^24.
    Every product is exact (BF16 operands 4096 and 1)."""
    m = small_model(layers=1, bf16=True)
    hdr = orc.header_from(m.config)
    H = 2048
    lm = m.lm_head.reshape(m.config.vocab_size, H)
    lm[0:2] = 0.0
    lm[0, [0, 1, 1000, 1001]] = [4096.0, 1.0, 1.0, 1.0]
    lm[1, [10, 11, 12, 13]] = [1.0, 1.0, 1.0, 4096.0]
    h = np.zeros(H, np.float32)
    h[[0, 1, 1000, 1001, 10, 11, 12]] = 1.0
    h[0] = h[13] = 4096.0
    logits = orc.compute_logits(hdr, m.blob, h)
    assert logits[0] == np.float32(2.0 ** 24)
    assert logits[1] == np.float32(2.0 ** 24 + 4)
    # the banked LM head of the decode path groups the same products otherwise
    banked = orc.gemv(0, lm[0:2], h)
    assert banked[0] == np.float32(2.0 ** 24 + 2)
