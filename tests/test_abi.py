"""The C-ABI boundary (include/gdn_amd.h) without a GPU: the library loads,
exports every declared entry point, keeps the reference's struct and
workspace layouts (gdn_model.h:30-75), and its host-side helpers (formats,
validation, synthetic generator, native product, scalar LM head) behave like
the reference's.  No call here touches the device."""
import ctypes
import os
import re

import numpy as np
import pytest

import gateddeltanet_amd as g
from gateddeltanet_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gdn_amd.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(gdn_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 34
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_struct_and_workspace_layout():
    assert ctypes.sizeof(_lib.GDNWeightHeader) == 60
    # gdn_model.h:54-75 values
    assert _lib.WS_OFF_X_NORM == 2048 and _lib.WS_OFF_Q == 4096
    assert _lib.WS_OFF_A == 10240 and _lib.WS_OFF_B == 10256 and _lib.WS_OFF_GATE == 10272
    assert _lib.WS_OFF_ATTN == 12320 and _lib.WS_OFF_TMP_HIDDEN == 14368
    assert _lib.WS_OFF_MLP_GATE == 16416 and _lib.WS_OFF_MLP_UP == 22048
    assert _lib.WS_OFF_REC_STATE == 27680 and _lib.WS_OFF_HEAD_BUF == 12610592
    assert _lib.WS_OFF_LOGITS == 13052960 and _lib.WS_FLOATS == 13084960
    text = open(HEADER).read()
    for name in ("GDN_WSF_STATE   12582912u", "GDN_WSF_HEADBUF 442368u", "GDN_WSF_LOGITS  32000u"):
        assert name in text


def test_default_config_and_sizes():
    c = g.default_config(24)
    assert bytes(c.magic)[:6] == b"GDNWv1" and c.version == 1
    assert (c.vocab_size, c.hidden_size, c.num_layers, c.num_heads) == (32000, 2048, 24, 8)
    assert (c.head_dim, c.intermediate_size, c.conv_size) == (256, 5632, 4)
    assert np.float32(c.norm_eps).view(np.uint32) == 0x358637BD
    n = _lib.load().gdn_total_weight_floats(ctypes.byref(c))
    # 1,399,324,672 dense params (architecture.md:280-283) + embeddings + aux
    dense = 24 * (4 * 2048 * 2048 + 2048 * 2048 + 3 * 5632 * 2048) + 32000 * 2048
    aux = 24 * (2048 + 8 + 8 + 2 * 8 * 2048 + 3 * 2048 * 4 + 256 + 2048) + 2048
    assert dense == 1399324672
    assert n == dense + aux + 32000 * 2048


def test_synth_is_deterministic_and_seeded():
    a = g.synth_normal(10001, 0, 5)
    b = g.synth_normal(10001, 0, 5)
    c = g.synth_normal(10001, 1, 5)
    assert (a == b).all() and not (a == c).all()
    assert abs(a.mean()) < 0.05 and abs(a.std() - 1) < 0.05
    # element i does not depend on how many are drawn
    assert (g.synth_normal(17, 0, 5) == a[:17]).all()
    u = g.synth_uniform(10000, 3, 1, 2.0, 4.0)
    assert u.min() >= 2.0 and u.max() < 4.0
    t = g.synth_tokens(10000, 0, 0, 32000)
    assert t.min() >= 0 and t.max() < 32000
    r = g.synth_normal(1000, 0, 2, bf16=True)
    assert ((r.view(np.uint32) & 0xFFFF) == 0).all()


def small(layers=1, vocab=256, bf16=True):
    cfg = g.default_config(layers)
    cfg.vocab_size = vocab
    return g.Model.synth(config=cfg, seed=0, bf16=bf16)


def test_gdnw_round_trip(tmp_path):
    m = small()
    p = str(tmp_path / "m.gdnw")
    m.save(p)
    assert os.path.getsize(p) == 60 + 4 * m.total_floats
    m2 = g.Model.load(p)
    assert (m2.blob == m.blob).all()
    assert (m2.layer(0)["o_norm"] == 1.0).all()
    assert (m2.final_norm == 1.0).all()


def test_gdnw_rejects_non_bf16_and_bad_magic(tmp_path):
    m = small(bf16=False)
    p = str(tmp_path / "f32.gdnw")
    m.save(p)
    with pytest.raises(g.GDNError):
        g.Model.load(p)
    assert (g.Model.load(p, fp32=True).blob == m.blob).all()
    raw = bytearray(open(p, "rb").read(200))
    raw[0:6] = b"XXXXXX"
    bad = str(tmp_path / "bad.gdnw")
    open(bad, "wb").write(bytes(raw))
    with pytest.raises(g.GDNError):
        g.Model.load(bad)


def test_validate_bf16_exact():
    m = small()
    lib = _lib.load()
    c = m.config
    assert lib.gdn_validate_bf16_exact_weights(m.blob.ctypes.data_as(_lib.FP), ctypes.byref(c)) == 0
    m.blob[123] = np.float32(0.1)
    assert lib.gdn_validate_bf16_exact_weights(m.blob.ctypes.data_as(_lib.FP), ctypes.byref(c)) == -1


def test_host_native_product_and_rne_hooks(orc):
    lib = _lib.load()
    rng = np.random.default_rng(14)
    for w, x in rng.integers(0, 1 << 16, (2000, 2)):
        want = orc.lib().orc_native_product_bits(int(w), int(x)) << 16
        got = np.float32(lib.gdn_native_bf16_mul_to_fp32(int(w), int(x))).view(np.uint32)
        assert got == want or (np.isnan(np.uint32(want).view(np.float32)) and np.isnan(got.view(np.float32)))
    for b in rng.integers(0, 1 << 32, 2000, dtype=np.uint64):
        assert lib.gdn_test_fp32_to_bf16_rne_bits(int(b)) == orc.lib().orc_rne_bits(int(b))
    assert lib.gdn_test_bf16_to_fp32_bits(0x3F80) == 0x3F800000


def test_host_compute_logits_matches_oracle(orc):
    m = small(vocab=512)
    h = g.bf16_round(np.random.default_rng(15).normal(0, 1, 2048).astype(np.float32))
    ours = m.compute_logits(h)
    ref = orc.compute_logits(orc.header_from(m.config), m.blob, h)
    assert (ours.view(np.uint32) == ref.view(np.uint32)).all()


@pytest.mark.parametrize("rows,k,rt", [(32, 64, 2), (64, 96, 4), (16, 32, 1)])
def test_mfma_tiling_layout(rows, k, rt):
    """The multi-stream GEMM's A-operand tiling (v_mfma_f32_16x16x32_bf16:
    lane l holds row l % 16, columns 8 (l / 16) .. + 7 of a 16 x 32 tile),
    checked element by element against the layout rule; every source value
    lands exactly once."""
    src = np.arange(rows * k, dtype=np.uint32).astype(np.uint16).reshape(rows, k)
    dst = np.empty(rows * k, np.uint16)
    _lib.load().gdn_test_tile_bf16(src.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), rows, k, rt,
                                   dst.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)))
    kt_n = k // 32
    for blk in range(rows // (16 * rt)):
        for kt in range(kt_n):
            for r in range(rt):
                base = (((blk * kt_n + kt) * rt + r) * 64) * 8
                for lane in range(64):
                    row = blk * 16 * rt + r * 16 + lane % 16
                    c0 = kt * 32 + 8 * (lane // 16)
                    assert (dst[base + lane * 8: base + lane * 8 + 8] == src[row, c0:c0 + 8]).all()
    assert sorted(dst.tolist()) == sorted(src.ravel().tolist())


# ---- the remaining gdn_model.h calls of the reference's gdn_eval.cpp ----

def bf16_value(bits):
    return np.uint32(bits << 16).view(np.float32)


def test_run_state_struct_prefix_is_the_reference_layout():
    """GDNRunState keeps gdn_model.h:153-160's fields in order (workspace,
    x, recurrent_state, head_buffer, 32 weight shards, aux image) with the
    engine pointer appended after them."""
    names = [f[0] for f in _lib.GDNRunState._fields_]
    assert names == ["workspace", "x", "recurrent_state", "head_buffer", "weight_shards", "aux_weights", "engine"]
    ptr = ctypes.sizeof(ctypes.c_void_p)
    assert _lib.GDNRunState.weight_shards.offset == 4 * ptr
    assert _lib.GDNRunState.aux_weights.offset == (4 + 32) * ptr
    assert _lib.GDNRunState.engine.offset == (5 + 32) * ptr
    assert ctypes.sizeof(_lib.Beat512) == 64
    text = open(HEADER).read()
    for name in ("#define GEMV_CHANNELS 32", "#define GDN_RECURRENT_STATE_PORTS       4",
                 "#define GDN_RECURRENT_STATE_FIRST_PORT 28"):
        assert name in text


def test_weight_shards_hold_no_weight_beats():
    c = g.default_config(24)
    lib = _lib.load()
    assert lib.gdn_weight_shard_beats(ctypes.byref(c)) == 0
    assert lib.gdn_weight_shard_bytes(ctypes.byref(c)) == 0


def test_beat_lane_accessors():
    """FP32 lane i = bytes 4i..4i+3, BF16 lane i = bytes 2i..2i+1
    (little-endian; gdn_model.cpp:225-272)."""
    lib = _lib.load()
    beat = _lib.Beat512()
    lib.gdn_test_set_fp32_lane_bits(ctypes.byref(beat), 3, 0x11223344)
    assert bytes(beat.bytes)[12:16] == bytes([0x44, 0x33, 0x22, 0x11])
    assert lib.gdn_test_get_fp32_lane_bits(ctypes.byref(beat), 3) == 0x11223344
    lib.gdn_test_set_bf16_lane_bits(ctypes.byref(beat), 31, 0xABCD)
    assert bytes(beat.bytes)[62:64] == bytes([0xCD, 0xAB])
    assert lib.gdn_test_get_bf16_lane_bits(ctypes.byref(beat), 6) == 0x3344  # low half of FP32 lane 3
    assert lib.gdn_test_get_bf16_lane_bits(ctypes.byref(beat), 7) == 0x1122  # high half
    assert lib.gdn_test_get_bf16_lane_bits(ctypes.byref(beat), 31) == 0xABCD


def test_state_scatter_and_conv_pack_layouts():
    """The reference's layout test (all_bf16_layout_test.cpp:27-107) restated:
    3 rows of BF16 values 0x3f00 | (i & 0x7f) scattered over four stripes
    are found at (port = island + 2 high_half, beat = 2 row + pair, lane =
    16 subhalf + lane16) for value high_half*128 + pair*64 + subhalf*32 +
    island*16 + lane16; the conv tails 0x3e80 | (i & 0x7f) land in the first
    GDN_CONV_TAIL_BF16_BEATS_PER_STRIPE beats of each stripe reservation and
    the rest stays zero."""
    lib = _lib.load()
    rows = 3
    rec = np.array([bf16_value(0x3F00 | (i & 0x7F)) for i in range(rows * 256)], np.float32)
    stripes = [(_lib.Beat512 * (rows * 2))() for _ in range(4)]
    arr = (ctypes.POINTER(_lib.Beat512) * 4)(*[ctypes.cast(s, ctypes.POINTER(_lib.Beat512)) for s in stripes])
    assert lib.gdn_scatter_recurrent_state(arr, rec.ctypes.data_as(_lib.FP), rec.size) == 0
    for row in range(rows):
        for port in range(4):
            island, high_half = port & 1, port >> 1
            for pair in range(2):
                beat = stripes[port][row * 2 + pair]
                for subhalf in range(2):
                    for lane in range(16):
                        v = high_half * 128 + pair * 64 + subhalf * 32 + island * 16 + lane
                        src = row * 256 + v
                        got = lib.gdn_test_get_bf16_lane_bits(ctypes.byref(beat), subhalf * 16 + lane)
                        assert got == (0x3F00 | (src & 0x7F)), (row, port, pair, subhalf, lane)
    bad = rec.copy()
    bad[5] = np.float32(0.1)
    assert lib.gdn_scatter_recurrent_state(arr, bad.ctypes.data_as(_lib.FP), bad.size) == -1
    assert lib.gdn_scatter_recurrent_state(arr, rec.ctypes.data_as(_lib.FP), 255) == -1

    n = _lib.WSF_HEADBUF
    conv = ((np.arange(n) & 0x7F) | 0x3E80).astype(np.uint32) << 16
    conv = conv.view(np.float32)
    packed = (_lib.Beat512 * (n // 16))()
    for i in range(0, n // 16, 7):
        packed[i].bytes[0] = 0xFF  # stale content the packer must clear
    assert lib.gdn_pack_conv_tails_bf16(packed, conv.ctypes.data_as(_lib.FP), n) == 0
    raw = np.frombuffer(packed, np.uint16).reshape(72, 384, 32)
    per = n // 72
    want = ((np.arange(n) & 0x7F) | 0x3E80).astype(np.uint16).reshape(72, per)
    assert (raw[:, :192, :].reshape(72, per) == want).all()
    assert (raw[:, 192:, :] == 0).all()
    assert lib.gdn_pack_conv_tails_bf16(packed, conv.ctypes.data_as(_lib.FP), n - 1) == -1


def test_mixed_mul_stats_count_host_products():
    """gdn_native_bf16_mul_to_fp32 counts each outcome as the reference's
    native multiplier does (gdn_model.cpp:401-462): every call; NaN, infinity
    and zero-exponent inputs as special, subnormal ones also as flushed
    inputs; magnitudes below 0x007fc000 or rounding to a zero exponent as
    flushed outputs; infinite results as overflows."""
    lib = _lib.load()
    cases = [  # (w, x, special, flushed_in, flushed_out, overflow)
        (0x3F80, 0x4000, 0, 0, 0, 0),   # 1 * 2
        (0x0000, 0x4000, 1, 0, 0, 0),   # zero input
        (0x0001, 0x4000, 1, 1, 0, 0),   # subnormal input (DAZ)
        (0x7F80, 0x4000, 1, 0, 0, 0),   # infinity
        (0x7FC1, 0x0005, 1, 1, 0, 0),   # NaN and a subnormal: one special pair
        (0x0080, 0x0080, 0, 0, 1, 0),   # 2^-126 * 2^-126: flushed
        (0x7F00, 0x7F00, 0, 0, 0, 1),   # 2^127 * 2^127: overflow
        (0x3F80, 0x0080, 0, 0, 0, 0),   # 1 * 2^-126: the smallest normal survives
        (0x3F7F, 0x0080, 0, 0, 1, 0),   # (1 - 2^-8) * 2^-126 = 0x007f8000 < 0x007fc000
        (0x7F7F, 0x3FFF, 0, 0, 0, 1),   # rounds up to infinity
    ]
    lib.gdn_reset_mixed_mul_stats()
    try:
        for w, x, *_ in cases:
            lib.gdn_native_bf16_mul_to_fp32(w, x)
        st = lib.gdn_get_mixed_mul_stats()
        want = np.array([c[2:] for c in cases]).sum(axis=0)
        assert st.calls == len(cases)
        assert (st.special_inputs, st.flushed_inputs, st.flushed_outputs, st.overflows) == tuple(want)
        # the scalar LM head counts its V x H products
        m = small(vocab=64)
        h = np.zeros(2048, np.float32)
        h[::2] = 1.0
        lib.gdn_reset_mixed_mul_stats()
        m.compute_logits(h)
        st = lib.gdn_get_mixed_mul_stats()
        assert st.calls == 64 * 2048 and st.special_inputs == 64 * 1024
        assert st.flushed_inputs == 0 and st.overflows == 0
    finally:
        lib.gdn_stop_mixed_mul_stats()


def test_run_state_init_rejects_shapes_before_any_device_call():
    """A vocabulary that is no multiple of the LM head's 8-row block, and
    max_tokens outside 1..max_seq_len, fail in gdn_run_state_init before the
    device is touched (so this runs without a GPU)."""
    m = small(vocab=260)
    with pytest.raises(g.GDNError):
        g.RunState(m, g.CONTRACT_BF16W_FP32S)
    m2 = small()
    lib = _lib.load()
    st = _lib.GDNRunState()
    assert lib.gdn_run_state_init(ctypes.byref(st), m2.ptr, 0) == -1
    assert lib.gdn_run_state_init(ctypes.byref(st), m2.ptr, m2.config.max_seq_len + 1) == -1
    assert st.engine is None
