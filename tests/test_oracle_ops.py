"""Closed-form and special-case pins of the oracle's operators.

Each expected value below is derived by hand from the mathematics (noted in
the comment), and the inputs are chosen so that a plausible mistake -- a
different association, a dropped rounding point, a swapped bank, a wrong tap
orientation -- changes the result.
"""
import numpy as np
import pytest

F = np.float32
TWO24 = F(2.0 ** 24)


def bf(x):
    """RNE to BF16 for finite values (the definition, via integers)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)


# ---------------------------------------------------------------- trees

def test_tree16_association(orc):
    # balanced: (2^24 + 1) -> 2^24 (tie to even), (-2^24 + 1) exact,
    # (1 + 1) = 2 twice: (2^24 + 2) + (-2^24 + 1 + 2) = 16777218 - 16777213 = 5.
    # A left-to-right sum gives 3; pairing (p0+p2) would give 4 or 6.
    p = np.zeros(16, F)
    p[0], p[1], p[2], p[3] = TWO24, 1, 1, 1
    p[4], p[5], p[6], p[7] = -TWO24, 1, 1, 1
    assert orc.tree16(p) == 5.0
    # integers sum exactly
    q = np.arange(16, dtype=F)
    assert orc.tree16(q) == 120.0


def test_tree256_association(orc):
    a = np.zeros(256, F)
    a[0], a[1], a[128] = TWO24, 1, 1
    # l128[0] = 2^24 + 1 -> 2^24; the 1 at index 128 joins at the top: 2^24 + 1 -> 2^24
    assert orc.tree256(a) == float(TWO24)
    a = np.zeros(256, F)
    a[0], a[2], a[1] = TWO24, -TWO24, 1
    # (2^24 + 1) -> 2^24, then + (-2^24) = 0: the 1 is lost.  A sequential
    # sum would also lose it, a (0,2)-first pairing would keep it.
    assert orc.tree256(a) == 0.0
    assert orc.tree256(np.ones(256, F)) == 256.0


# ----------------------------------------------------------------- GEMV

@pytest.mark.parametrize("contract", [0, 2])
def test_gemv_one_hot_selects_column(orc, contract):
    rng = np.random.default_rng(3)
    W = bf(rng.normal(0, 0.02, (64, 2048)).astype(F))
    for k in (0, 17, 1023, 2047):
        x = np.zeros(2048, F)
        x[k] = 1.0
        y = orc.gemv(contract, W, x)
        assert (y == W[:, k]).all()


@pytest.mark.parametrize("K", [2048, 5632])
def test_gemv_integer_exact(orc, K):
    rng = np.random.default_rng(4)
    W = rng.integers(-8, 9, (32, K)).astype(F)
    x = rng.integers(-8, 9, K).astype(F)
    want = (W.astype(np.int64) @ x.astype(np.int64)).astype(F)
    for contract in (0, 2):
        assert (orc.gemv(contract, W, x) == want).all()


def test_gemv_bank_order(orc):
    # x = 1; the row holds 2^24 at beat 0, -2^24 at beat 4 (both even/lower)
    # and a 1 at beat 1 (odd/lower) and a 1 at beat 2 lane 16 (even/upper).
    # Banks: even_lo = (2^24) + (-2^24) = 0, even_hi = 1, odd_lo = 1:
    # y = (0 + 1) + (1 + 0) = 2.  One running sum over all beats gives 0 or 1;
    # merging halves per beat before banking gives 1.
    W = np.zeros((8, 2048), F)
    W[0, 0] = TWO24
    W[0, 4 * 32] = -TWO24
    W[0, 1 * 32] = 1.0
    W[0, 2 * 32 + 16] = 1.0
    x = np.ones(2048, F)
    for contract in (0, 2):
        assert orc.gemv(contract, W, x)[0] == 2.0


def test_gemv_native_rounding_point(orc):
    # each product (1 + 2^-7)^2 = 1 + 2^-6 + 2^-14 rounds to 1 + 2^-6 in the
    # native contract (BF16 products) but not in the FP32 control arm.
    w = F(1 + 2.0 ** -7)
    W = np.full((8, 2048), w, F)
    x = np.full(2048, w, F)
    y_ref = orc.gemv(0, W, x)[0]
    y_f32 = orc.gemv(2, W, x)[0]
    assert y_ref == F(2048 * (1 + 2.0 ** -6))
    assert y_f32 != y_ref


def _literal_gemv_row(products):
    """The GEMV contract written out as plain loops over float32 values:
    tree16 = balanced pairs over each 16-product half-beat, four banks
    (lower/upper x even/odd beat) accumulated in beat order from +0.0, then
    (even_lo + even_hi) + (odd_lo + odd_hi)."""
    def tree16(v):
        v = list(v)
        while len(v) > 1:
            v = [F(v[2 * i] + v[2 * i + 1]) for i in range(len(v) // 2)]
        return v[0]
    banks = [F(0.0)] * 4
    for b in range(len(products) // 32):
        lo = tree16(products[32 * b:32 * b + 16])
        hi = tree16(products[32 * b + 16:32 * b + 32])
        e = 2 * (b & 1)
        banks[e] = F(banks[e] + lo)
        banks[e + 1] = F(banks[e + 1] + hi)
    return F(F(banks[0] + banks[1]) + F(banks[2] + banks[3]))


@pytest.mark.parametrize("K", [64, 128, 2048])
def test_gemv_brute_force_literal_loop(orc, K):
    """orc_gemv against the literal loop above on random BF16 operands with
    zeros, subnormals and a wide exponent range; the native products come
    from orc_native_product_bits (exhaustively pinned in
    test_oracle_bf16.py), the FP32 arm's from float32 multiplication."""
    rng = np.random.default_rng(K)
    M = 6
    W = bf(rng.normal(0, 1, (M, K)).astype(F) * np.exp2(rng.integers(-20, 20, (M, K))).astype(F))
    x = bf(rng.normal(0, 1, K).astype(F) * np.exp2(rng.integers(-20, 20, K)).astype(F))
    W[0, ::7] = 0.0
    x[::11] = 0.0
    W[1, 3] = np.uint32(0x00010000).view(F)   # a subnormal weight (DAZ)
    x[5] = np.uint32(0x80020000).view(F)      # a subnormal activation
    wb = (W.view(np.uint32) >> 16).astype(np.uint16)
    xb = (x.view(np.uint32) >> 16).astype(np.uint16)
    for contract in (0, 2):
        got = orc.gemv(contract, W, x, threads=False)
        for r in range(M):
            if contract == 0:
                p = orc.native_product_array(wb[r], xb).astype(np.uint32) << 16
                prod = p.view(F)
            else:
                prod = (W[r] * x).astype(F)
            want = _literal_gemv_row(prod)
            assert got[r].view(np.uint32) == want.view(np.uint32), (contract, r)


def test_gemv_tiny_order(orc):
    # acc = (acc + lo) + hi per beat: (0 + 2^24) + 1 -> 2^24; then
    # (2^24 + -2^24) + 0 = 0.  Separate lo/hi banks would give 1.
    W = np.zeros((1, 2048), F)
    W[0, 0] = TWO24
    W[0, 16] = 1.0
    W[0, 32] = -TWO24
    x = np.ones(2048, F)
    assert orc.gemv_tiny(W, x)[0] == 0.0


# ----------------------------------------------------------------- norms

def test_rmsnorm_constant(orc):
    # x = 1: sum = 2048, 1/sqrtf(1 + 1e-6f) = 0.99999952 -> BF16 1.0
    out = orc.rmsnorm(0, np.ones(2048, F), np.ones(2048, F))
    assert (out == 1.0).all()
    # x = 2, w = 0.5: scale ~ 1/2 -> 2 * scale * 0.5 ~ 0.5
    out = orc.rmsnorm(0, np.full(2048, 2.0, F), np.full(2048, 0.5, F))
    assert (out == 0.5).all()
    # FP32 arm keeps the unrounded value
    out = orc.rmsnorm(2, np.ones(2048, F), np.ones(2048, F))
    assert (out == F(1.0) / np.sqrt(F(1.0) + F(1e-6))).all()


def test_rmsnorm_scale_invariance(orc):
    rng = np.random.default_rng(5)
    x = bf(rng.normal(0, 1, 2048).astype(F))
    w = bf(rng.normal(1, 0.1, 2048).astype(F))
    a = orc.rmsnorm(2, x, w)
    b = orc.rmsnorm(2, x * F(4), w)
    np.testing.assert_allclose(a, b, rtol=1e-5)


def test_residual_rmsnorm(orc):
    x = np.full(2048, 1.0, F)
    y = np.full(2048, 2.0 ** -9, F)  # 1 + 2^-9 is a tie -> BF16 1.0
    xo, out = orc.residual_rmsnorm(0, x, y, np.ones(2048, F))
    assert (xo == 1.0).all() and (out == 1.0).all()
    xo, _ = orc.residual_rmsnorm(2, x, y, np.ones(2048, F))
    assert (xo == F(1 + 2.0 ** -9)).all()


def test_output_norm_gate(orc):
    # a = 1 per head -> normalised ~1; g = 0 -> gate g*sigmoid(g) = 0
    o = np.ones(2048, F)
    out = orc.output_norm_gate(0, o, np.zeros(2048, F), np.ones(256, F), 8, 256)
    assert (out == 0).all()
    # heads normalise independently: head h scaled by (h+1) gives the same row
    o = np.concatenate([np.full(256, h + 1, F) for h in range(8)])
    g = np.full(2048, 4.0, F)
    out = orc.output_norm_gate(2, o, g, np.ones(256, F), 8, 256)
    s = F(4.0) / (F(1) + np.exp(F(-4.0)))
    np.testing.assert_allclose(out, np.full(2048, s, F), rtol=2e-6)


def _rms_scale(total, n):
    # 1 / sqrtf(total / n + 1e-6f) in float32
    return F(1.0) / np.sqrt(F(total) / F(n) + F(1e-6))


def test_rmsnorm_sum_is_chunked_then_sequential(orc):
    # gdn_model.cpp:1432-1450: sixteen-value chunks summed in lane order from
    # 0, the 128 chunk sums then added in order.  x^2 values:
    #  (a) chunk 0 = [2^24, 1 x 15], chunk 1 = sixteen 1s: the chunk sums are
    #      2^24 (each +1 is a tie that rounds back to 2^24) and 16, total
    #      2^24 + 16 exactly; one flat sequential sum over all 2048 squares
    #      stays at 2^24.
    #  (b) chunk 0 = [2^24], chunks 1..127 = [1]: chunk sums added in order
    #      stay at 2^24; a balanced tree over the chunk sums (127 first) gives
    #      2^24 + 128.
    # Expected outputs from the closed-form totals (FP32 arm: no rounding).
    x = np.zeros(2048, F)
    x[0] = 4096.0
    x[1:32] = 1.0
    w = np.ones(2048, F)
    out = orc.rmsnorm(2, x, w)
    want = x * _rms_scale(2.0 ** 24 + 16, 2048)
    assert (out.view(np.uint32) == want.view(np.uint32)).all()
    assert not (out == x * _rms_scale(2.0 ** 24, 2048)).all()
    x = np.zeros(2048, F)
    x[0] = 4096.0
    x[16::16] = 1.0
    out = orc.rmsnorm(2, x, w)
    want = x * _rms_scale(2.0 ** 24, 2048)
    assert (out.view(np.uint32) == want.view(np.uint32)).all()
    assert not (out == x * _rms_scale(2.0 ** 24 + 128, 2048)).all()


def test_output_norm_sum_is_chunked_per_head(orc):
    # The same association per 256-value head (16 chunks of 16): head 0 holds
    # [4096, 1 x 31] (chunk sums 2^24 and 16 -> 2^24 + 16), head 1 holds 4096
    # then a 1 in each later chunk (sums in order stay 2^24).  Gate g = 2^7
    # with sigmoid(2^7) = 1 in float32, so out = x * scale * 128.
    o = np.zeros(2048, F)
    o[0], o[1:32] = 4096.0, 1.0
    o[256], o[256 + 16:512:16] = 4096.0, 1.0
    g = np.full(2048, 128.0, F)
    out = orc.output_norm_gate(2, o, g, np.ones(256, F), 8, 256)
    s0 = _rms_scale(2.0 ** 24 + 16, 256)
    s1 = _rms_scale(2.0 ** 24, 256)
    assert (out[:256] == o[:256] * s0 * F(128)).all()
    assert (out[256:512] == o[256:512] * s1 * F(128)).all()
    assert s0 != s1


# ----------------------------------------------------------------- conv

def test_conv_taps_and_shift(orc):
    C = 2048
    rng = np.random.default_rng(6)
    raw = bf(rng.normal(0, 1, C).astype(F))
    tails = bf(rng.normal(0, 1, (3, C)).astype(F))
    # tap 3 applies to the newest input
    w = np.zeros((C, 4), F)
    w[:, 3] = 1.0
    out, t2 = orc.conv_silu(0, raw, w, tails, orc.CR)
    want = bf(np.array([orc.lib().orc_silu(float(v), orc.CR) for v in raw], F))
    assert (out == want).all()
    # the tail shifts by one row and appends the raw (pre-conv) input
    assert (t2[0] == tails[1]).all() and (t2[1] == tails[2]).all() and (t2[2] == raw).all()
    # tap 0 applies to the oldest row
    w = np.zeros((C, 4), F)
    w[:, 0] = 1.0
    out, _ = orc.conv_silu(0, raw, w, tails, orc.CR)
    want = bf(np.array([orc.lib().orc_silu(float(v), orc.CR) for v in tails[0]], F))
    assert (out == want).all()
    # zero tails and zero weights give silu(0) = 0
    out, _ = orc.conv_silu(0, raw, np.zeros((C, 4), F), np.zeros((3, C), F))
    assert (out == 0).all()


def test_conv_sum_is_left_associated(orc):
    # s = ((t0 w0 + t1 w1) + t2 w2) + x w3 (gdn_model.cpp:1646-1650) with
    # products 2^24, 1, 1, 1: every +1 onto 2^24 is a tie that rounds back,
    # so s = 2^24 and silu(s) = 2^24.  Any pairing of the last three terms
    # first (1 + 1 = 2, or 1 + 1 + 1 = 3 -> 2^24 + 2 or + 4) differs.
    C = 2048
    tails = np.ones((3, C), F)
    tails[0] = 4096.0
    w = np.zeros((C, 4), F)
    w[:, 0] = 4096.0
    w[:, 1:] = 1.0
    out, _ = orc.conv_silu(2, np.ones(C, F), w, tails, orc.CR)
    assert (out == TWO24).all()
    # the newest term alone large: ((1 + 1) + 1) + 2^24 = 2^24 + 3 -> 2^24 + 4
    tails = np.ones((3, C), F)
    w = np.ones((C, 4), F)
    w[:, 3] = TWO24
    out, _ = orc.conv_silu(2, np.ones(C, F), w, tails, orc.CR)
    assert (out == F(2.0 ** 24 + 4)).all()


# ----------------------------------------------------------------- recurrence

def _unit(v):
    return v / np.sqrt((v.astype(np.float64) ** 2).sum())


def test_recurrence_beta_zero(orc):
    rng = np.random.default_rng(7)
    S = rng.normal(0, 0.01, (256, 256)).astype(F)
    q, k, v = (rng.normal(0, 1, 256).astype(F) for _ in range(3))
    o, S2 = orc.recurrence_head_scalars(2, q, k, v, 0.0, 0.5, S)
    # beta = 0: S' = decay * S exactly (k * 0 adds +-0)
    assert (S2 == F(0.5) * S).all()
    qn = _unit(q.astype(np.float64))
    np.testing.assert_allclose(o, 0.0625 * 0.5 * (S.astype(np.float64).T @ qn), rtol=2e-5, atol=1e-7)


def test_recurrence_one_hot_key_overwrites_row(orc):
    # decay = 1, beta = 1, k = e_j: S'[j] = v, other rows unchanged.
    rng = np.random.default_rng(8)
    S = rng.integers(-4, 5, (256, 256)).astype(F)
    v = rng.integers(-4, 5, 256).astype(F)
    k = np.zeros(256, F)
    k[37] = 3.0  # normalised to 1 (up to the 1e-6 guard): use a power of two scale
    q = rng.normal(0, 1, 256).astype(F)
    o, S2 = orc.recurrence_head_scalars(2, q, k, v, 1.0, 1.0, S)
    knorm = F(3.0) * (F(1.0) / np.sqrt(F(9.0) + F(1e-6)))
    # row j: S + kn * (v - kn * S_j) ; with kn != 1 exactly, compare to fp64
    want = S.astype(np.float64).copy()
    want[37] = S[37] + float(knorm) * (v - float(knorm) * S[37])
    np.testing.assert_allclose(S2, want, rtol=1e-6, atol=1e-6)
    others = np.ones(256, bool)
    others[37] = False
    assert (S2[others] == S[others]).all()


def test_recurrence_plain_ieee_case(orc):
    # decay = 1 and beta = 0.5 leave only exactly-rounded FP32 arithmetic
    # (the reference's own cosim setting, slr2_region_cosim/README.md:8-12):
    # compare to the textbook recurrence in fp64.
    rng = np.random.default_rng(9)
    S = rng.normal(0, 0.01, (256, 256)).astype(F)
    q, k, v = (rng.normal(0, 1, 256).astype(F) for _ in range(3))
    o, S2 = orc.recurrence_head_scalars(2, q, k, v, 0.5, 1.0, S)
    qn, kn = _unit(q.astype(np.float64)), _unit(k.astype(np.float64))
    S64 = S.astype(np.float64)
    # textbook (chunk.py:688-718): S_t = a S (I - b k k^T) + b v k^T in [V][K];
    # in [K][V]: S_t = a S + b k (v - a S^T k)^T ; o = S_t^T q / sqrt(dk)
    St = S64 + np.outer(kn, 0.5 * (v - S64.T @ kn))
    np.testing.assert_allclose(S2, St, rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(o, St.T @ qn / 16.0, rtol=1e-4, atol=1e-6)


def test_recurrence_gated_against_fp64(orc):
    rng = np.random.default_rng(10)
    S = rng.normal(0, 0.01, (256, 256)).astype(F)
    for step in range(4):
        q, k, v = (rng.normal(0, 1, 256).astype(F) for _ in range(3))
        a, b = float(rng.normal()), float(rng.normal())
        a_log = float(rng.uniform(0, np.log(16)))
        o, S2 = orc.recurrence_head(2, q, k, v, a, b, a_log, 0.0, S, orc.CR)
        beta = 1 / (1 + np.exp(-b))
        decay = np.exp(-np.exp(a_log) * np.log1p(np.exp(a)))
        qn, kn = _unit(q.astype(np.float64)), _unit(k.astype(np.float64))
        S64 = S.astype(np.float64)
        St = decay * S64 + np.outer(kn, beta * (v - decay * (S64.T @ kn)))
        np.testing.assert_allclose(S2, St, rtol=1e-4, atol=1e-7)
        np.testing.assert_allclose(o, St.T @ qn / 16.0, rtol=1e-4, atol=1e-7)
        S = S2


def test_recurrence_ref_rounds_state(orc):
    rng = np.random.default_rng(11)
    S = bf(rng.normal(0, 0.01, (256, 256)).astype(F))
    q, k, v = (bf(rng.normal(0, 1, 256).astype(F)) for _ in range(3))
    o, S2 = orc.recurrence_head(0, q, k, v, 0.1, 0.2, 0.3, 0.0, S)
    assert ((S2.view(np.uint32) & 0xFFFF) == 0).all()
    assert ((o.view(np.uint32) & 0xFFFF) == 0).all()
    o1, S1 = orc.recurrence_head(1, q, k, v, 0.1, 0.2, 0.3, 0.0, S)
    assert (o1 == o).all()          # same pass; only the stored state differs
    assert (bf(S1) == S2).all()


def test_head_scalars_closed_form(orc):
    beta, decay = orc.head_scalars(0.0, 0.0, 0.0, 0.0, orc.CR)
    assert beta == 0.5
    assert decay == F(np.exp(-np.log(2.0)))  # exp(-1 * softplus(0)) = 1/2
    beta, decay = orc.head_scalars(25.0, -30.0, 0.0, 0.0, orc.CR)
    assert decay == F(np.exp(np.float32(-25.0)))  # softplus(x > 20) = x


# ----------------------------------------------------------------- misc

def test_swiglu(orc):
    g = np.array([0.0, 1.0, -1.0, 4.0], F)
    u = np.array([5.0, 2.0, 2.0, 0.5], F)
    h = orc.swiglu(2, g, u, orc.CR)
    want = g / (1 + np.exp(-g.astype(np.float64))) * u
    np.testing.assert_allclose(h, want, rtol=1e-6)
    assert orc.swiglu(0, g, u, orc.CR)[0] == 0.0


def test_argmax_rules(orc):
    assert orc.argmax(np.array([1, 3, 3, 2], F)) == 1              # lowest index wins ties
    assert orc.argmax(np.array([np.nan, 1, np.nan, 2], F)) == 3     # NaN never wins
    assert orc.argmax(np.full(5, -np.inf, F)) == 0                  # nothing beats -FLT_MAX
    assert orc.argmax(np.array([-3.402823466e38, -3.402823466e38], F)) == 0
    assert orc.argmax(np.array([0, np.inf, np.inf], F)) == 1


# ------------------------------------------- order-sensitive association pins
#
# Each test below feeds inputs whose float32 result changes under any other
# grouping, FMA contraction or summation direction of the same terms, and
# asserts the exact bits the reference's expression gives.  The expected bits
# are derived in the comments; where a result is computed in numpy, the test
# also asserts that the plausible alternative groupings disagree with it on
# these inputs, so a regrouped oracle fails.

HALF_KEYS = (0, 1, 100, 101)


def _keys_at(rows):
    # 2^19 at four rows: the sum of squares is 2^40 in any order and
    # 2^40 + 1e-6f == 2^40, so 1/sqrtf(.) = 2^-20 and kn = 1/2 exactly there.
    assert len(rows) == 4
    k = np.zeros(256, F)
    k[list(rows)] = 2.0 ** 19
    return k


@pytest.mark.parametrize("contract", [0, 2])
def test_recurrence_chains_are_sequential_over_rows(orc, contract):
    # gdn_model.cpp:2612-2615: r_i = r_i + S[j][i]*kn_j and p_i likewise,
    # row j = 0..255 in order.  kn = qn = 1/2 at rows 0, 1, 100, 101
    # (alpha = 4 * 1/4 = 1) and S = 2^25, 2, 2, 2 there, so the terms are
    # 2^24, 1, 1, 1.  In order every +1 onto 2^24 is a tie that rounds back:
    # r = p = 2^24.  A tree (the 1s at rows 100, 101 paired first), 64-row
    # blocks summed in order, or a reversed sum give 2^24 + 2, 2^24 + 2 and
    # 2^24 + 4.  With beta = decay = 1 and v = 2^24 + 8:
    #   delta = v - r = 8 (6 or 4 for the alternatives)
    #   o = (1/16)(p + alpha*delta) = (2^24 + 8)/16 = 2^20 + 1/2
    #   S'[j] = S[j] + kn_j*delta: 2^25 + 4 at row 0, 6 at rows 1, 100, 101.
    k = _keys_at(HALF_KEYS)
    S = np.zeros((256, 256), F)
    S[0], S[1], S[100], S[101] = 2.0 ** 25, 2.0, 2.0, 2.0
    v = np.full(256, 2.0 ** 24 + 8, F)
    o, S2 = orc.recurrence_head_scalars(contract, k, k, v, 1.0, 1.0, S)
    if contract == 2:
        assert (o == F(2.0 ** 20 + 0.5)).all()
        assert (S2[0] == F(2.0 ** 25 + 4)).all()
    else:  # outputs and state rounded to BF16 (8 significant bits)
        assert (o == F(2.0 ** 20)).all()
        assert (S2[0] == F(2.0 ** 25)).all()
    for j in (1, 100, 101):
        assert (S2[j] == 6.0).all()          # delta = 8: the sum in row order
    rest = np.ones(256, bool)
    rest[list(HALF_KEYS)] = False
    assert (S2[rest] == 0).all()


# decay = 1 - 2^-24 (the float below 1) and a state entry 1 + 2^-23 at row 0:
# the exact product decay * (0.5 + 2^-24) = 0.5 + 2^-25 - 2^-48 lies just
# below the midpoint of 0.5 and its successor, so the rounded product is
# 0.5, while a fused multiply-add keeps the 2^-25 - 2^-48.
DECAY_BELOW_1 = float(np.nextafter(F(1), F(0)))
S_ROW0 = 1.0 + 2.0 ** -23


def _delta_case(orc, v, beta):
    k = _keys_at((0, 1, 2, 3))              # kn = qn = 1/2 at rows 0..3
    S = np.zeros((256, 256), F)
    S[0] = S_ROW0                           # r = p = (1 + 2^-23)/2 = 0.5 + 2^-24
    return orc.recurrence_head_scalars(2, k, k, np.full(256, v, F), beta, DECAY_BELOW_1, S)


def test_delta_and_output_round_each_product(orc):
    # gdn_model.cpp:2671-2673, delta = beta*(v - decay*r) and
    # o = q_scale*(decay*p + alpha*delta), every product rounded before the
    # add (no FMA); round(decay*r) = round(decay*p) = 0.5.
    # v = 0, beta = 1: delta = -0.5; o = (0.5 + 1*(-0.5))/16 = 0 (an FMA gives
    # (2^-25 - 2^-48)/16); S'[0] = round(decay*(1 + 2^-23)) + (1/2)(-1/2)
    # = 1 - 0.25 = 0.75 (an FMA in the update gives 0.75 + 2^-24).
    o, S2 = _delta_case(orc, 0.0, 1.0)
    assert (o == 0).all()
    assert (S2[0] == F(0.75)).all() and (S2[1] == F(-0.25)).all()
    # v = 0.5, beta = 1: delta = 0.5 - 0.5 = 0 (an FMA gives -(2^-25 - 2^-48),
    # visible in S'[1] = 0 + (1/2) delta); o = (0.5 + 0)/16 = 1/32.
    o, S2 = _delta_case(orc, 0.5, 1.0)
    assert (S2[1] == 0).all() and (S2[0] == 1.0).all()
    assert (o == F(1.0 / 32)).all()


def test_delta_scales_the_difference(orc):
    # beta*(v - decay*r) with v = 0.5 + 2^-24: v - round(decay*r) = 2^-24
    # exactly, so delta = f32(1/3) * 2^-24 exactly and S'[1] = delta/2 =
    # f32(1/3) * 2^-25.  Distributing beta (beta*v - beta*(decay*r)) rounds
    # beta*v up by one ulp of 1/6 and gives delta = 2^-26, S'[1] = 2^-27.
    third = float(F(1.0 / 3.0))
    _, S2 = _delta_case(orc, 0.5 + 2.0 ** -24, third)
    assert (S2[1] == F(third * 2.0 ** -25)).all()
    assert F(third * 2.0 ** -25) != F(2.0 ** -27)


def _sig(orc, x, tmode):
    f = orc.lib().orc_sigmoid
    return np.array([f(float(v), tmode) for v in x], F)


@pytest.mark.parametrize("contract", [0, 2])
def test_swiglu_association(orc, contract):
    # gdn_model.cpp:4763: h = R(silu(g) * u) with silu(g) = g * sigmoid(g)
    # (gdn_model.cpp:1318), i.e. R((g*s)*u), on gate/up values already at the
    # BF16 point.  sigmoid itself is pinned against glibc (test_libm.py).
    rng = np.random.default_rng(21)
    g = bf(rng.normal(0, 2, 4096).astype(F))
    u = bf(rng.normal(0, 2, 4096).astype(F))
    s = _sig(orc, g, orc.LIBM)
    rnd = bf if contract == 0 else (lambda x: x)
    want = rnd(F(g * s) * u)
    h = orc.swiglu(contract, g, u)
    assert (h.view(np.uint32) == want.view(np.uint32)).all()
    # the same terms grouped otherwise differ on a share of these inputs in
    # the FP32 arm (the oracle runs one grouping for every contract; in the
    # BF16 arm a one-ulp FP32 difference shows only next to a BF16 tie)
    if contract == 2:
        for alt in (g * F(s * u), F(g * u) * s):
            assert (alt != want).mean() > 0.2


@pytest.mark.parametrize("contract", [0, 2])
def test_output_gate_association(orc, contract):
    # gdn_model.cpp:5808-5810: normalized = (a * scale) * w, then
    # out = R((normalized * g) * sigmoid(g)).  Integer head values make the
    # sum of squares exact in any order (the chunked order is pinned by
    # test_output_norm_sum_is_chunked_per_head), so
    # scale = 1/sqrtf(sum/256 + 1e-6f) is computed here in float32.
    rng = np.random.default_rng(22)
    a = rng.integers(1, 4, 2048).astype(F) * rng.choice([-1, 1], 2048).astype(F)
    w = bf(rng.normal(1, 0.3, 256).astype(F))
    g = bf(rng.normal(0, 2, 2048).astype(F))
    out = orc.output_norm_gate(contract, a, g, w, 8, 256)
    rnd = bf if contract == 0 else (lambda x: x)
    s = _sig(orc, g, orc.LIBM)
    want = np.empty(2048, F)
    alts = [np.empty(2048, F) for _ in range(4)]
    for h in range(8):
        sl = slice(256 * h, 256 * (h + 1))
        total = F((a[sl].astype(np.float64) ** 2).sum())
        scale = F(1) / np.sqrt(total / F(256) + F(1e-6))
        nrm = F(a[sl] * scale) * w
        want[sl] = rnd(F(nrm * g[sl]) * s[sl])
        alts[0][sl] = rnd(F(nrm * F(g[sl] * s[sl])))               # normalized * silu(g)
        alts[1][sl] = rnd(F(F(a[sl] * F(scale * w)) * g[sl]) * s[sl])  # a * (scale * w)
        alts[2][sl] = rnd(F(nrm * s[sl]) * g[sl])                  # sigmoid before g
        alts[3][sl] = rnd(F(F(a[sl] * scale) * F(w * g[sl])) * s[sl])  # w * g first
    assert (out.view(np.uint32) == want.view(np.uint32)).all()
    if contract == 2:  # one grouping for every contract (see test_swiglu_association)
        for alt in alts:
            assert (alt != want).mean() > 0.05
