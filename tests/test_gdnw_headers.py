"""Malformed .gdnw files through gdn_model_load / gdn_model_load_fp32 (host
only, no device call): every truncation and header corruption either loads a
model whose payload matches its header or is refused with -1 and a message,
never a crash.  Header checks that 32-bit arithmetic would get wrong are
pinned with hand-made headers: a num_heads x head_dim product that wraps, a
payload size that wraps size_t, and zero dimensions (the conv tails are sized
by conv_size - 1).  The reference's loader (gdn_model.cpp:1161-1229) reads
the header and then the payload it describes."""
import ctypes
import random
import struct

import pytest

import gateddeltanet_amd as g
from gateddeltanet_amd import _lib

HDR = 60  # sizeof(GDNWeightHeader)
# field offsets in the header: magic[8], then u32 fields in declaration order
FIELDS = ["version", "vocab_size", "hidden_size", "num_layers", "num_heads", "num_v_heads", "head_dim",
          "intermediate_size", "conv_size", "max_seq_len", "bos_token_id", "eos_token_id"]


def tiny_file(tmp_path):
    cfg = g.default_config(1)
    cfg.vocab_size, cfg.hidden_size, cfg.num_heads, cfg.num_v_heads = 64, 64, 1, 1
    cfg.head_dim, cfg.intermediate_size = 64, 128
    m = g.Model.synth(config=cfg, seed=1)
    p = tmp_path / "tiny.gdnw"
    m.save(str(p))
    m.free()
    return p, p.read_bytes()


def with_fields(raw, **vals):
    b = bytearray(raw)
    for k, v in vals.items():
        off = 8 + 4 * FIELDS.index(k)
        b[off:off + 4] = struct.pack("<I", v)
    return bytes(b)


def try_load(path, fp32=False):
    lib = _lib.load()
    m = _lib.GDNModel()
    rc = (lib.gdn_model_load_fp32 if fp32 else lib.gdn_model_load)(ctypes.byref(m), str(path).encode())
    if rc == 0:
        total = lib.gdn_total_weight_floats(ctypes.byref(m.config))
        lib.gdn_model_free(ctypes.byref(m))
        return rc, total
    return rc, None


def test_header_layout_matches_field_table():
    assert ctypes.sizeof(_lib.GDNWeightHeader) == HDR
    for k in FIELDS:
        assert getattr(_lib.GDNWeightHeader, k).offset == 8 + 4 * FIELDS.index(k)


def test_truncations_and_header_stomps_never_crash(tmp_path):
    p, raw = tiny_file(tmp_path)
    n_payload = len(raw) - HDR
    cases = [raw[:cut] for cut in (0, 1, 7, HDR - 1, HDR, HDR + 1, HDR + 4, len(raw) // 2, len(raw) - 1)]
    for k in FIELDS:
        for v in (0, 1, 3, 0x10000, 0x7fffffff, 0x80000000, 0xffffffff):
            cases.append(with_fields(raw, **{k: v}))
    rng = random.Random(7)
    for _ in range(150):
        b = bytearray(raw)
        for _ in range(rng.randint(1, 4)):
            b[rng.randrange(HDR)] = rng.randrange(256)
        cases.append(bytes(b))
    loaded = 0
    bad = tmp_path / "bad.gdnw"
    for data in cases:
        bad.write_bytes(data)
        for fp32 in (False, True):
            rc, total = try_load(bad, fp32)
            assert rc in (0, -1)
            if rc == 0:
                # a model only loads when the file holds the payload its header describes
                assert 4 * total <= len(data) - HDR
                loaded += 1
    assert loaded > 0  # fields that do not size the payload (max_seq_len, token ids) still load
    assert try_load(p) == (0, n_payload // 4)
    # trailing bytes after the payload are ignored, as the reference's sequential read does
    bad.write_bytes(raw + b"\0" * 8)
    assert try_load(bad) == (0, n_payload // 4)


def test_wrapped_head_product_is_refused(tmp_path, capfd):
    _, raw = tiny_file(tmp_path)
    # 2 x 0x80000020 = 64 modulo 2^32
    bad = tmp_path / "wrap.gdnw"
    bad.write_bytes(with_fields(raw, num_heads=2, num_v_heads=2, head_dim=0x80000020))
    assert try_load(bad)[0] == -1
    assert "differs from num_heads" in capfd.readouterr().err


def test_payload_size_that_wraps_size_t_is_refused(tmp_path, capfd):
    _, raw = tiny_file(tmp_path)
    # hidden = 2^23 x 2^8 = 2^31, vocab 2^32 - 1: the embedding and LM head alone
    # are about 2^64 floats
    bad = tmp_path / "huge.gdnw"
    bad.write_bytes(with_fields(raw, hidden_size=1 << 31, num_heads=1 << 23, num_v_heads=1 << 23,
                                head_dim=1 << 8, vocab_size=0xffffffff))
    assert try_load(bad)[0] == -1
    assert "more payload than this process can address" in capfd.readouterr().err


@pytest.mark.parametrize("field", ["vocab_size", "intermediate_size", "conv_size"])
def test_zero_dimensions_are_refused(tmp_path, capfd, field):
    _, raw = tiny_file(tmp_path)
    bad = tmp_path / "zero.gdnw"
    bad.write_bytes(with_fields(raw, **{field: 0}))
    assert try_load(bad)[0] == -1
    assert "zero dimension" in capfd.readouterr().err


def test_zero_hidden_is_refused(tmp_path, capfd):
    _, raw = tiny_file(tmp_path)
    bad = tmp_path / "zero_h.gdnw"
    bad.write_bytes(with_fields(raw, hidden_size=0, num_heads=0, num_v_heads=0))
    assert try_load(bad)[0] == -1
    assert "zero dimension" in capfd.readouterr().err


def test_synth_refuses_the_same_headers():
    cfg = g.default_config(1)
    cfg.conv_size = 0
    with pytest.raises(g.GDNError):
        g.Model.synth(config=cfg)
