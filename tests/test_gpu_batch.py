"""Multi-stream decode (gdn_batch_*) on the GPU (gpu).

The projections run on the matrix cores: exact products of the BF16
operands summed in FP32 in the hardware's order.  Every other operator is
the BF16W_FP32S arithmetic of the batch-1 engine.

Bit-exact checks:
  * the GEMM on integer-valued operands (every partial sum exact in FP32)
    equals the integer product, at K = 2048 and K = 5632;
  * a 24-layer model whose projection rows each hold a single power of two
    (every projection sum then has one nonzero term, so summation order and
    product rounding cannot matter): the multi-stream engine equals the
    batch-1 engine and the oracle (BF16W_FP32S, glibc transcendentals) bit for bit -- tokens,
    logits and every stream's state -- which pins the whole composition
    (norms, a/b rows, conv tails, recurrence, output norm, SwiGLU, residual
    adds, LM head and the argmax tie rule);
  * stream s's results do not depend on the other streams (a permutation
    permutes outputs bit for bit; a one-stream engine reproduces stream 0);
  * graph and eager launches agree; per-stream state load/save round-trips.
Tolerance checks on a random model, where exact products differ from the
reference's rounded products (the oracle's ORC_BF16X arm is the exact-product
arithmetic; it is 3-4e-2 from the BF16W arm after one layer):
  * one layer against ORC_BF16X: logits within 2e-2 (summation order only),
    argmax equal or a near tie;
  * 24 layers against the batch-1 engine: the measured gap is reported and
    bounded loosely (the random-init model amplifies rounding differences).
"""
import numpy as np
import pytest

import gateddeltanet_amd as g

pytestmark = pytest.mark.gpu

B = 64
LOGIT_TOL = 2e-2
STATE_TOL = 1e-3


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return a.shape == b.shape and bool((a.view(np.uint32) == b.view(np.uint32)).all())


def check_argmax(ref_logits, ref_tok, got_tok, max_err):
    """Equal, or a near tie in the reference logits."""
    if ref_tok == got_tok:
        return True
    return ref_logits[ref_tok] - ref_logits[got_tok] <= 2 * max_err


@pytest.fixture(scope="module")
def model():
    m = g.Model.synth(num_layers=24, seed=0, std=0.02, bf16=True)
    yield m
    m.free()


@pytest.mark.parametrize("K,N", [(2048, 256), (5632, 64)])
def test_batch_gemm_exact_on_integers(K, N):
    rng = np.random.default_rng(K)
    W = rng.integers(-8, 9, (N, K)).astype(np.float32)
    X = rng.integers(-8, 9, (64, K)).astype(np.float32)
    Y = g.batch_gemm(W, X)
    want = X.astype(np.int64) @ W.astype(np.int64).T
    assert (Y.astype(np.int64) == want).all()
    # a transposed operand or a wrong stream/row mapping cannot pass this
    assert not (want == want[:, ::-1]).all()


@pytest.mark.parametrize("K,N", [(2048, 512), (5632, 128)])
def test_batch_gemm_rounding_bound(K, N):
    rng = np.random.default_rng(K + 1)
    W = g.bf16_round(rng.normal(0, 0.02, (N, K)).astype(np.float32)).reshape(N, K)
    X = g.bf16_round(rng.normal(0, 1, (64, K)).astype(np.float32)).reshape(64, K)
    Y = g.batch_gemm(W, X).astype(np.float64)
    exact = X.astype(np.float64) @ W.astype(np.float64).T
    bound = K * 2.0 ** -24 * (np.abs(X).astype(np.float64) @ np.abs(W).astype(np.float64).T)
    assert (np.abs(Y - exact) <= bound).all()
    assert np.abs(Y - exact).max() > 0 or K == 0  # genuinely FP32 sums


@pytest.mark.parametrize("kind,N,T", [(0, 256, 192), (0, 128, 64), (1, 256, 130), (2, 128, 64), (2, 512, 130),
                                      (3, 5632, 70), (3, 5632, 1000)])
def test_prefill_gemm_equals_step_gemm(kind, N, T):
    """The prefill's projection GEMMs form every sum of the step's GEMMs bit
    for bit: the q/k/v/g configuration (8 classes of k tiles), o_proj's and
    down's (4 classes x 4 splits, split sums in order) and gate/up + SwiGLU
    (k_bgu's layout; 1000 tokens take the XCD super-tile placement); token
    counts that leave partial 64- and 128-token tiles.  Row counts that are multiples of 256 run k_pgemm_a (weights
    straight into registers, as the engine's q/k/v/g and down launches), the
    others k_pgemm (128 rows x 128 tokens, both operands through LDS)."""
    rng = np.random.default_rng(100 + kind)
    K = 5632 if kind == 2 else 2048
    shape = (2, N, K) if kind == 3 else (N, K)
    W = g.bf16_round(rng.normal(0, 0.02, shape).astype(np.float32)).reshape(shape)
    X = g.bf16_round(rng.normal(0, 1, (T, K)).astype(np.float32)).reshape(T, K)
    y, y_step = g.prefill_gemm(kind, W, X)
    assert np.isfinite(y_step).all() and np.abs(y_step).max() > 0
    assert same_bits(y, y_step)


def batch1_reference(m, tokens, init=None):
    """Per-stream batch-1 runs (BF16W_FP32S): logits [steps][B][V], tokens,
    final states."""
    steps, nb = tokens.shape
    rs = g.RunState(m, g.CONTRACT_BF16W_FP32S)
    logits = np.empty((steps, nb, m.config.vocab_size), np.float32)
    toks = np.empty((steps, nb), np.int64)
    states = []
    try:
        for s in range(nb):
            if init is None:
                rs.load_state(np.zeros(rs.n_state, np.float32), np.zeros(rs.n_conv, np.float32))
            else:
                rs.load_state(*init[s])
            for i in range(steps):
                toks[i, s] = rs.decode_step(int(tokens[i, s]))
                logits[i, s] = rs.logits()
            states.append(rs.save_state())
    finally:
        rs.free()
    return logits, toks, states


def one_hot_model(num_layers, seed):
    """Synthetic model whose dense projection rows are single +-2^k entries."""
    m = g.Model.synth(num_layers=num_layers, seed=seed, std=0.02, bf16=True)
    c = m.config
    rng = np.random.default_rng(seed)

    def fill(view, rows, cols):
        w = view.reshape(rows, cols)
        w[:] = 0.0
        pick = rng.integers(0, cols, rows)
        val = rng.choice(np.array([-2.0, -1.0, -0.5, 0.5, 1.0, 2.0], np.float32), rows)
        w[np.arange(rows), pick] = val

    H, I = c.hidden_size, c.intermediate_size
    for i in range(num_layers):
        lw = m.layer(i)
        for name in ("q_proj", "k_proj", "v_proj", "g_proj", "o_proj"):
            fill(lw[name], H, H)
        fill(lw["mlp_gate_proj"], I, H)
        fill(lw["mlp_up_proj"], I, H)
        fill(lw["mlp_down_proj"], H, I)
    fill(m.lm_head, c.vocab_size, H)
    return m


def equal_values(a, b):
    """Equal as numbers (a zero's sign may differ: sums of signed zeros)."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return a.shape == b.shape and bool(((a == b) | (np.isnan(a) & np.isnan(b))).all())


@pytest.fixture(scope="module")
def onehot():
    m = one_hot_model(24, 7)
    yield m
    m.free()


def test_one_hot_model_bit_exact_to_batch1(onehot):
    m, steps = onehot, 3
    tokens = g.synth_tokens(steps * B, 20, 0).reshape(steps, B)
    ref_logits, ref_toks, ref_states = batch1_reference(m, tokens)
    bs = g.BatchState(m, B)
    try:
        for i in range(steps):
            got = bs.step(tokens[i])
            assert (got == ref_toks[i]).all(), i
            for s in range(B):
                assert equal_values(bs.logits(s), ref_logits[i, s]), (i, s)
        for s in range(B):
            r, c = bs.save_stream_state(s)
            assert equal_values(r, ref_states[s][0]) and equal_values(c, ref_states[s][1]), s
    finally:
        bs.free()


def test_one_hot_partial_stream_group(onehot):
    """37 streams: the last 16-stream MFMA group is partly empty, the gate/up
    epilogue and the split post-down norm see a stream count that is no
    multiple of 16; every stream still equals its batch-1 run bit for bit."""
    m, steps, nb = onehot, 2, 37
    tokens = g.synth_tokens(steps * nb, 27, 0).reshape(steps, nb)
    ref_logits, ref_toks, ref_states = batch1_reference(m, tokens)
    bs = g.BatchState(m, nb)
    try:
        for i in range(steps):
            got = bs.step(tokens[i])
            assert (got == ref_toks[i]).all(), i
            for s in range(nb):
                assert equal_values(bs.logits(s), ref_logits[i, s]), (i, s)
        for s in range(nb):
            r, c = bs.save_stream_state(s)
            assert equal_values(r, ref_states[s][0]) and equal_values(c, ref_states[s][1]), s
    finally:
        bs.free()


def test_one_hot_model_bit_exact_to_oracle(orc, onehot):
    m = onehot
    hdr = orc.header_from(m.config)
    nb, steps = 2, 2
    tokens = g.synth_tokens(steps * nb, 26, 0).reshape(steps, nb)
    bs = g.BatchState(m, nb)
    try:
        st = [np.zeros(24 * 8 * 256 * 256, np.float32) for _ in range(nb)]
        cv = [np.zeros(24 * 3 * 3 * 2048, np.float32) for _ in range(nb)]
        for i in range(steps):
            got = bs.step(tokens[i])
            for s in range(nb):
                ot, ol, oh = orc.decode_step(1, hdr, m.blob, st[s], cv[s], int(tokens[i, s]), orc.LIBM)
                assert got[s] == ot
                assert equal_values(bs.logits(s), ol) and equal_values(bs.final_hidden(s), oh)
        for s in range(nb):
            r, c = bs.save_stream_state(s)
            assert equal_values(r, st[s]) and equal_values(c, cv[s])
    finally:
        bs.free()


def test_random_model_gap_to_batch1(model):
    """Exact products vs the reference's rounded products over 24 layers of
    a random-init model: report the gap, bound it loosely."""
    steps = 2
    tokens = g.synth_tokens(steps * B, 21, 0).reshape(steps, B)
    ref_logits, ref_toks, ref_states = batch1_reference(model, tokens)
    bs = g.BatchState(model, B)
    try:
        got_toks = np.stack([bs.step(tokens[i]) for i in range(steps)])
        got_last = np.stack([bs.logits(s) for s in range(B)])
        got_states = [bs.save_stream_state(s)[0] for s in range(B)]
    finally:
        bs.free()
    err = np.abs(got_last - ref_logits[-1]).max()
    rel = max(np.linalg.norm(got_states[s] - ref_states[s][0]) / np.linalg.norm(ref_states[s][0])
              for s in range(B))
    agree = (got_toks == ref_toks).mean()
    print(f"[batch] random 24-layer model vs batch-1: logits max-abs {err:.3e}, state rel-L2 {rel:.3e}, "
          f"argmax agreement {agree:.3f}", flush=True)
    assert err <= 0.5 and rel <= 0.1 and agree >= 0.8


def test_one_hot_model_from_loaded_states(onehot):
    """Nonzero per-stream states (random recurrent state and conv tails)
    loaded into both engines, then two steps: bit-exact to batch-1."""
    m, nb, steps = onehot, 8, 2
    init = []
    for s in range(nb):
        rec = g.synth_normal(m.config.num_layers * 8 * 256 * 256, 30 + s, 0, std=0.01)
        conv = g.bf16_round(g.synth_normal(m.config.num_layers * 3 * 3 * 2048, 30 + s, 1, std=0.5))
        init.append((rec, conv))
    tokens = g.synth_tokens(steps * nb, 22, 0).reshape(steps, nb)
    ref_logits, ref_toks, ref_states = batch1_reference(m, tokens, init)
    bs = g.BatchState(m, nb)
    try:
        for s in range(nb):
            bs.load_stream_state(s, *init[s])
            r, c = bs.save_stream_state(s)
            assert same_bits(r, init[s][0]) and same_bits(c, init[s][1])
        for i in range(steps):
            got = bs.step(tokens[i])
            assert (got == ref_toks[i]).all(), i
            for s in range(nb):
                assert equal_values(bs.logits(s), ref_logits[i, s]), (i, s)
        for s in range(nb):
            r, c = bs.save_stream_state(s)
            assert equal_values(r, ref_states[s][0]) and equal_values(c, ref_states[s][1]), s
    finally:
        bs.free()


def test_streams_are_independent(model):
    steps = 2
    tokens = g.synth_tokens(steps * B, 23, 0).reshape(steps, B)
    perm = np.random.default_rng(5).permutation(B)
    runs = []
    for order in (np.arange(B), perm):
        bs = g.BatchState(model, B)
        try:
            toks = [bs.step(tokens[i][order]) for i in range(steps)]
            runs.append((np.stack(toks), np.stack([bs.logits(s) for s in range(B)]),
                         bs.save_stream_state(int(np.argmax(order == 0)))[0]))
        finally:
            bs.free()
    inv = np.argsort(perm)
    assert (runs[1][0][:, inv] == runs[0][0]).all()
    assert same_bits(runs[1][1][inv], runs[0][1])
    assert same_bits(runs[1][2], runs[0][2])
    one = g.BatchState(model, 1)
    try:
        for i in range(steps):
            t1 = one.step(tokens[i][:1])
        assert t1[0] == runs[0][0][-1, 0]
        assert same_bits(one.logits(0), runs[0][1][0])
    finally:
        one.free()


def test_batch_graph_eager_and_teacher_forced(model):
    nb, steps = 16, 3
    tokens = g.synth_tokens(steps * nb, 24, 0).reshape(steps, nb)
    out = []
    for use_graph in (True, False):
        bs = g.BatchState(model, nb)
        try:
            bs.set_graph(use_graph)
            toks = np.stack([bs.step(tokens[i]) for i in range(steps)])
            out.append((toks, np.stack([bs.logits(s) for s in range(nb)]), bs.save_stream_state(3)[0]))
        finally:
            bs.free()
    assert (out[0][0] == out[1][0]).all()
    assert same_bits(out[0][1], out[1][1]) and same_bits(out[0][2], out[1][2])
    bs = g.BatchState(model, nb)
    try:
        am, inner, outer = bs.teacher_forced(tokens)
        assert (am == out[0][0]).all()
        assert (inner > 0).all() and (outer >= inner * 0.5).all()
        with pytest.raises(g.GDNError):
            bs.step(np.full(nb, model.config.vocab_size))
    finally:
        bs.free()


def test_random_one_layer_against_exact_product_oracle(orc):
    """One layer, four streams, three steps against ORC_BF16X (LIBM): the
    remaining difference is the summation order of the projections."""
    m = g.Model.synth(num_layers=1, seed=3, std=0.02, bf16=True)
    hdr = orc.header_from(m.config)
    nb, steps = 4, 3
    tokens = g.synth_tokens(steps * nb, 25, 0).reshape(steps, nb)
    bs = g.BatchState(m, nb)
    try:
        st = [np.zeros(8 * 256 * 256, np.float32) for _ in range(nb)]
        cv = [np.zeros(3 * 3 * 2048, np.float32) for _ in range(nb)]
        for i in range(steps):
            got = bs.step(tokens[i])
            for s in range(nb):
                ot, ol, _ = orc.decode_step(orc.BF16X, hdr, m.blob, st[s], cv[s], int(tokens[i, s]), orc.LIBM)
                lg = bs.logits(s)
                err = np.abs(lg - ol).max()
                assert err <= LOGIT_TOL, (i, s, err)
                assert check_argmax(ol, ot, got[s], err)
        for s in range(nb):
            r, c = bs.save_stream_state(s)
            assert np.linalg.norm(r - st[s]) <= STATE_TOL * np.linalg.norm(st[s])
            assert np.linalg.norm(c - cv[s]) <= STATE_TOL * np.linalg.norm(cv[s])
    finally:
        bs.free()
        m.free()


# ------------------------------------------------------------------ prefill

def stepped_reference(m, prompt):
    """One stream stepped token by token through the multi-stream engine."""
    bs = g.BatchState(m, 1)
    try:
        for t in prompt:
            last = int(bs.step([t])[0])
        return last, bs.logits(0), bs.final_hidden(0), bs.save_stream_state(0)
    finally:
        bs.free()


@pytest.mark.parametrize("n", [1, 2, 64, 65, 128, 150])
def test_prefill_equals_steps(model, n):
    """Prefill of n tokens (chunks of 64; n < 3 exercises the conv tails
    alone, 64 / 65 / 128 the chunk edges) equals n single-stream steps bit
    for bit, and leaves the other streams' states alone."""
    prompt = g.synth_tokens(n, 40 + n, 0)
    seed_ref, logits_ref, hidden_ref, (rec_ref, conv_ref) = stepped_reference(model, prompt)
    bs = g.BatchState(model, 3)
    try:
        seed = bs.prefill(1, prompt)
        assert seed == seed_ref
        assert same_bits(bs.logits(1), logits_ref) and same_bits(bs.final_hidden(1), hidden_ref)
        rec, conv = bs.save_stream_state(1)
        assert same_bits(rec, rec_ref) and same_bits(conv, conv_ref)
        for other in (0, 2):
            r, c = bs.save_stream_state(other)
            assert not r.any() and not c.any()
        # decoding continues from the prefilled state like the stepped stream
        nxt = bs.step([0, seed, 0])
        ref = g.BatchState(model, 1)
        try:
            for t in prompt:
                ref.step([t])
            assert int(ref.step([seed])[0]) == nxt[1]
            assert same_bits(ref.logits(0), bs.logits(1))
        finally:
            ref.free()
    finally:
        bs.free()


@pytest.mark.parametrize("n", [4096, 4200])
def test_prefill_long_segment_equals_steps(n):
    """A 4096-token segment, where the engine runs the q/k/v/g and down
    projections on k_pgemm_a (its grid fills the CUs only from 1024 and 4096
    tokens), equals n single-stream steps bit for bit (2 layers); at 4200
    the 104-token second segment runs them on k_pgemm, from the first
    segment's state."""
    m = g.Model.synth(num_layers=2, seed=4, std=0.02, bf16=True)
    try:
        prompt = g.synth_tokens(n, 44, 0)
        seed_ref, logits_ref, hidden_ref, (rec_ref, conv_ref) = stepped_reference(m, prompt)
        bs = g.BatchState(m, 1)
        try:
            assert bs.prefill(0, prompt) == seed_ref
            assert same_bits(bs.logits(0), logits_ref) and same_bits(bs.final_hidden(0), hidden_ref)
            rec, conv = bs.save_stream_state(0)
            assert same_bits(rec, rec_ref) and same_bits(conv, conv_ref)
        finally:
            bs.free()
    finally:
        m.free()


def test_prefill_continues_a_decoded_stream(model):
    """A prefill on a stream that has already decoded tokens continues from
    its state and conv tails: 5 steps then a 70-token prefill equal 75
    steps bit for bit."""
    head = g.synth_tokens(5, 47, 0)
    prompt = g.synth_tokens(70, 48, 0)
    seed_ref, logits_ref, hidden_ref, (rec_ref, conv_ref) = stepped_reference(model, np.concatenate([head, prompt]))
    bs = g.BatchState(model, 2)
    try:
        for t in head:
            bs.step([0, t])
        assert bs.prefill(1, prompt) == seed_ref
        assert same_bits(bs.logits(1), logits_ref) and same_bits(bs.final_hidden(1), hidden_ref)
        rec, conv = bs.save_stream_state(1)
        assert same_bits(rec, rec_ref) and same_bits(conv, conv_ref)
    finally:
        bs.free()


def test_prefill_one_hot_matches_batch1(onehot):
    """On the one-hot model the prefill equals batch-1 decode steps
    (BF16W_FP32S) too: state, conv tails, seed token and last logits."""
    m = onehot
    prompt = g.synth_tokens(70, 41, 0)
    rs = g.RunState(m, g.CONTRACT_BF16W_FP32S)
    try:
        for t in prompt:
            seed_ref = rs.decode_step(int(t))
        logits_ref = rs.logits()
        rec_ref, conv_ref = rs.save_state()
    finally:
        rs.free()
    bs = g.BatchState(m, 2)
    try:
        assert bs.prefill(0, prompt) == seed_ref
        assert equal_values(bs.logits(0), logits_ref)
        rec, conv = bs.save_stream_state(0)
        assert equal_values(rec, rec_ref) and equal_values(conv, conv_ref)
    finally:
        bs.free()


def test_load_rejects_non_bf16_tails(model):
    """The device keeps each stream's conv tails as BF16: a tail value that
    is not BF16-exact is refused before anything (tails or state) is
    written."""
    bs = g.BatchState(model, 2)
    try:
        rec0, conv0 = bs.save_stream_state(1)
        conv = g.bf16_round(g.synth_normal(conv0.size, 41, 0, std=0.5))
        conv[5] = np.float32(1.0 + 2.0 ** -10)  # needs 10 mantissa bits
        with pytest.raises(g.GDNError):
            bs.load_stream_state(1, rec0 + 1.0, conv)
        rec, cv = bs.save_stream_state(1)
        assert equal_values(rec, rec0) and equal_values(cv, conv0)
        conv[5] = np.float32(1.0)
        bs.load_stream_state(1, None, conv)
        assert equal_values(bs.save_stream_state(1)[1], conv)
    finally:
        bs.free()


def test_prefill_rejects_bad_tokens(model):
    bs = g.BatchState(model, 1)
    try:
        with pytest.raises(g.GDNError):
            bs.prefill(0, [1, model.config.vocab_size])
        with pytest.raises(g.GDNError):
            bs.prefill(0, [])
    finally:
        bs.free()


def test_random_24_layers_16_steps_against_exact_product_oracle(orc, model):
    """The multi-stream engine over the full 24-layer random model for 16
    steps, four streams, against ORC_BF16X (the same arithmetic with the
    projections' products exact, summed in the reference's order): what
    remains is the projections' summation order, amplified by the BF16
    rounding points.  Measured on MI355X: logits max-abs 0.147, state
    relative L2 2.6e-2, argmax equal on 60 of 64 stream-steps and a near tie
    on the rest.  Bounds: logits max-abs <= 0.25, state relative L2 <= 5e-2,
    argmax equal or a near tie on every stream-step."""
    m = model
    hdr = orc.header_from(m.config)
    nb, steps = 4, 16
    tokens = g.synth_tokens(steps * nb, 31, 0).reshape(steps, nb)
    st = [np.zeros(24 * 8 * 256 * 256, np.float32) for _ in range(nb)]
    cv = [np.zeros(24 * 3 * 3 * 2048, np.float32) for _ in range(nb)]
    worst, agree, near = 0.0, 0, 0
    bs = g.BatchState(m, nb)
    try:
        for i in range(steps):
            got = bs.step(tokens[i])
            for s in range(nb):
                ot, ol, _ = orc.decode_step(orc.BF16X, hdr, m.blob, st[s], cv[s], int(tokens[i, s]), orc.LIBM)
                err = float(np.abs(bs.logits(s) - ol).max())
                worst = max(worst, err)
                agree += int(ot == got[s])
                near += int(check_argmax(ol, ot, got[s], err))
        rel = max(float(np.linalg.norm(bs.save_stream_state(s)[0] - st[s]) / np.linalg.norm(st[s]))
                  for s in range(nb))
    finally:
        bs.free()
    print(f"[batch] 24 layers x {steps} steps x {nb} streams vs ORC_BF16X: logits max-abs {worst:.3e}, "
          f"state rel-L2 {rel:.3e}, argmax equal {agree}/{steps * nb}, equal or near tie {near}/{steps * nb}",
          flush=True)
    assert worst <= 0.25 and rel <= 5e-2 and near == steps * nb


def test_prefill_one_hot_matches_oracle(orc, onehot):
    """A 70-token prefill (two chunks) on the one-hot model, where every
    projection sum has one term, equals the oracle (BF16W_FP32S, glibc
    transcendentals) stepped token by token: seed token, last logits and
    hidden vector, recurrent state and conv tails."""
    m = onehot
    hdr = orc.header_from(m.config)
    prompt = g.synth_tokens(70, 49, 0)
    st = np.zeros(24 * 8 * 256 * 256, np.float32)
    cv = np.zeros(24 * 3 * 3 * 2048, np.float32)
    for t in prompt:
        seed_ref, logits_ref, hidden_ref = orc.decode_step(1, hdr, m.blob, st, cv, int(t), orc.LIBM)
    bs = g.BatchState(m, 2)
    try:
        assert bs.prefill(1, prompt) == seed_ref
        assert equal_values(bs.logits(1), logits_ref) and equal_values(bs.final_hidden(1), hidden_ref)
        rec, conv = bs.save_stream_state(1)
        assert equal_values(rec, st) and equal_values(conv, cv)
    finally:
        bs.free()


def test_prefill_random_model_against_exact_product_oracle(orc):
    """A 70-token prefill on a random 2-layer model against ORC_BF16X
    stepped token by token: the summation order of the projections is the
    only difference.  Measured on MI355X: last logits max-abs 1.0e-2, state
    relative L2 3.2e-3.  Bounds: last logits within LOGIT_TOL (2e-2), the
    seed equal or a near tie, state and conv tails within 1e-2 relative L2."""
    m = g.Model.synth(num_layers=2, seed=4, std=0.02, bf16=True)
    hdr = orc.header_from(m.config)
    prompt = g.synth_tokens(70, 50, 0)
    st = np.zeros(2 * 8 * 256 * 256, np.float32)
    cv = np.zeros(2 * 3 * 3 * 2048, np.float32)
    for t in prompt:
        seed_ref, logits_ref, _ = orc.decode_step(orc.BF16X, hdr, m.blob, st, cv, int(t), orc.LIBM)
    bs = g.BatchState(m, 1)
    try:
        seed = bs.prefill(0, prompt)
        err = float(np.abs(bs.logits(0) - logits_ref).max())
        rec, conv = bs.save_stream_state(0)
    finally:
        bs.free()
        m.free()
    rel = float(np.linalg.norm(rec - st) / np.linalg.norm(st))
    print(f"[prefill] 2 layers x 70 tokens vs ORC_BF16X: logits max-abs {err:.3e}, state rel-L2 {rel:.3e}",
          flush=True)
    assert err <= LOGIT_TOL and check_argmax(logits_ref, seed_ref, seed, err)
    assert rel <= 1e-2 and np.linalg.norm(conv - cv) <= 1e-2 * np.linalg.norm(cv)


# ---------------------------------------------------------- chunked prefill

def _rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(np.asarray(b, np.float64)))


@pytest.mark.parametrize("n", [1, 8, 64, 150])
def test_prefill_chunked_recurrence_precision(n):
    """The chunk-parallel (WY) recurrence against the token-order scan where
    nothing else differs: after one layer the two modes have the same q, k,
    v, beta and decay, so the state differs only by the FP32
    re-association of the recurrence's sums (measured 1.1e-6 relative L2 at
    n = 64).  Bound: 1e-5."""
    m = g.Model.synth(num_layers=1, seed=0, std=0.02, bf16=True)
    prompt = g.synth_tokens(n, 61, 0)
    bs = g.BatchState(m, 2)
    try:
        bs.prefill(0, prompt)
        rec_scan, conv_scan = bs.save_stream_state(0)
        bs.set_prefill_mode(g.PREFILL_CHUNKED)
        bs.prefill(1, prompt)
        rec, conv = bs.save_stream_state(1)
    finally:
        bs.free()
        m.free()
    rel = _rel(rec, rec_scan)
    print(f"[prefill chunked] 1 layer, n={n}: state rel-L2 vs scan {rel:.3e}", flush=True)
    assert rel <= 1e-5 and same_bits(conv, conv_scan)


def test_prefill_chunked_from_a_loaded_state_leaves_other_streams():
    """The chunked recurrence from a nonzero state (N(0, 0.01) per element,
    BF16 conv tails), on the middle stream of three: against the scan from
    the same state, one layer, 100 tokens (a full chunk then a partial
    one), state relative L2 <= 1e-5; the other two streams' states and
    tails stay bit for bit."""
    m = g.Model.synth(num_layers=1, seed=2, std=0.02, bf16=True)
    rng = np.random.default_rng(9)
    n_rec, n_conv = 8 * 256 * 256, 3 * 3 * 2048
    states = [rng.normal(0.0, 0.01, n_rec).astype(np.float32) for _ in range(3)]
    tails = [g.bf16_round(rng.normal(0.0, 1.0, n_conv).astype(np.float32)) for _ in range(3)]
    prompt = g.synth_tokens(100, 63, 0)
    out = {}
    for mode in (g.PREFILL_SCAN, g.PREFILL_CHUNKED):
        bs = g.BatchState(m, 3)
        try:
            bs.set_prefill_mode(mode)
            for sidx in range(3):
                bs.load_stream_state(sidx, states[sidx], tails[sidx])
            bs.prefill(1, prompt)
            out[mode] = [bs.save_stream_state(sidx) for sidx in range(3)]
        finally:
            bs.free()
    m.free()
    rel = _rel(out[g.PREFILL_CHUNKED][1][0], out[g.PREFILL_SCAN][1][0])
    print(f"[prefill chunked] from a loaded state, 1 layer x 100 tokens vs scan: state rel-L2 {rel:.3e}", flush=True)
    assert rel <= 1e-5 and same_bits(out[g.PREFILL_CHUNKED][1][1], out[g.PREFILL_SCAN][1][1])
    for sidx in (0, 2):
        rec, conv = out[g.PREFILL_CHUNKED][sidx]
        assert same_bits(rec, states[sidx]) and same_bits(conv, tails[sidx])


@pytest.mark.parametrize("n", [64, 150])
def test_prefill_chunked_full_model_against_scan(model, n):
    """Over the 24-layer random model the re-association flips occasional
    BF16 roundings of o, which the later layers amplify, as for the
    multi-stream projections' summation order.  Measured at n = 64: last
    logits max-abs 0.125, state relative L2 3.0e-2.  Bounds: logits max-abs
    <= 0.25, state relative L2 <= 5e-2, seed equal or a near tie."""
    prompt = g.synth_tokens(n, 61, 0)
    bs = g.BatchState(model, 2)
    try:
        seed_scan = bs.prefill(0, prompt)
        logits_scan = bs.logits(0)
        rec_scan, _ = bs.save_stream_state(0)
        bs.set_prefill_mode(g.PREFILL_CHUNKED)
        seed = bs.prefill(1, prompt)
        logits = bs.logits(1)
        rec, _ = bs.save_stream_state(1)
    finally:
        bs.free()
    err = float(np.abs(logits - logits_scan).max())
    rel = _rel(rec, rec_scan)
    print(f"[prefill chunked] 24 layers, n={n} vs scan: logits max-abs {err:.3e}, state rel-L2 {rel:.3e}, "
          f"seed {seed} vs {seed_scan}", flush=True)
    assert err <= 0.25 and rel <= 5e-2 and check_argmax(logits_scan, seed_scan, seed, err)


def test_prefill_chunked_against_exact_product_oracle(orc):
    """The chunked prefill on a random 2-layer model against ORC_BF16X
    stepped token by token (70 tokens, two chunks): the projections' and the
    recurrence's summation orders are the differences.  Bounds: last logits
    max-abs <= 5e-2 (seed equal or a near tie), state and conv tails within
    1e-2 relative L2."""
    m = g.Model.synth(num_layers=2, seed=4, std=0.02, bf16=True)
    hdr = orc.header_from(m.config)
    prompt = g.synth_tokens(70, 50, 0)
    st = np.zeros(2 * 8 * 256 * 256, np.float32)
    cv = np.zeros(2 * 3 * 3 * 2048, np.float32)
    for t in prompt:
        seed_ref, logits_ref, _ = orc.decode_step(orc.BF16X, hdr, m.blob, st, cv, int(t), orc.LIBM)
    bs = g.BatchState(m, 1)
    try:
        bs.set_prefill_mode(g.PREFILL_CHUNKED)
        seed = bs.prefill(0, prompt)
        err = float(np.abs(bs.logits(0) - logits_ref).max())
        rec, conv = bs.save_stream_state(0)
    finally:
        bs.free()
        m.free()
    rel = _rel(rec, st)
    print(f"[prefill chunked] 2 layers x 70 tokens vs ORC_BF16X: logits max-abs {err:.3e}, "
          f"state rel-L2 {rel:.3e}", flush=True)
    assert err <= 5e-2 and check_argmax(logits_ref, seed_ref, seed, err)
    assert rel <= 1e-2 and _rel(conv, cv) <= 1e-2


def test_prefill_mode_rejects_unknown(model):
    bs = g.BatchState(model, 1)
    try:
        with pytest.raises(g.GDNError):
            bs.set_prefill_mode(7)
        for bad in (0, 64, 200, 32768 + 128):
            with pytest.raises(g.GDNError):
                bs.set_prefill_segment(bad)
    finally:
        bs.free()


@pytest.mark.parametrize("mode", ["scan", "chunked"])
def test_prefill_segments(model, mode):
    """A 300-token prompt run as segments of 128 tokens (128 + 128 + 44: the
    conv window and the state cross segment edges, the last segment is a
    partial token tile) gives the results of one segment bit for bit, in
    both recurrence modes; in scan mode both equal 300 steps."""
    prompt = g.synth_tokens(300, 49, 0)
    out = []
    for seg in (None, 128):
        bs = g.BatchState(model, 2)
        try:
            bs.set_prefill_mode(g.PREFILL_SCAN if mode == "scan" else g.PREFILL_CHUNKED)
            if seg:
                bs.set_prefill_segment(seg)
            seed = bs.prefill(1, prompt)
            out.append((seed, bs.logits(1), bs.final_hidden(1), *bs.save_stream_state(1)))
        finally:
            bs.free()
    one, segs = out
    assert one[0] == segs[0]
    assert all(same_bits(a, b) for a, b in zip(one[1:], segs[1:]))
    if mode == "scan":
        seed_ref, logits_ref, hidden_ref, (rec_ref, conv_ref) = stepped_reference(model, prompt)
        assert one[0] == seed_ref
        assert same_bits(one[1], logits_ref) and same_bits(one[2], hidden_ref)
        assert same_bits(one[3], rec_ref) and same_bits(one[4], conv_ref)
