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
