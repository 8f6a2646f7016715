"""Malformed .gdnw files through gdn_model_load / gdn_model_load_fp32 (host
only, no device call): every truncation and header corruption either loads a
model whose payload matches its header or is refused with -1 and a message,
never a crash.  Header checks that 32-bit arithmetic would get wrong are
pinned with hand-made headers: a num_heads x head_dim product that wraps, a
payload size that wraps size_t, and zero dimensions (the conv tails are sized
by conv_size - 1).  The reference's loader (gdn_model.cpp:1161-1229) reads
the header and then the payload it describes.  The .gdnstate reader
(gdn_eval.cpp:196-267) is held to the same rule: every dimension that sizes a
section, the value dimension included, must match the model before a buffer
is sized from it."""
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


def write_gdnstate(path, cfg, version=1, dv=None, prompt=(), payload=True):
    """A .gdnstate in the reference's layout (export_gdn_state.py:340-362)."""
    hd = cfg.head_dim
    v = [version, cfg.num_layers, cfg.num_heads, hd, hd if dv is None else dv, cfg.hidden_size,
         cfg.conv_size, len(prompt), 0]
    rec = cfg.num_layers * cfg.num_heads * hd * hd
    conv = cfg.num_layers * 3 * (cfg.conv_size - 1) * cfg.hidden_size
    with open(path, "wb") as f:
        f.write(b"GDNSTAT1" + struct.pack("<9I", *v) + struct.pack(f"<{len(prompt)}i", *prompt))
        if payload:
            f.write(b"\0" * 4 * (rec + conv))


@pytest.mark.parametrize("case", ["dv_huge", "dv_small", "version", "layers", "short"])
def test_gdnstate_header_checked_before_any_allocation(tmp_path, capfd, case):
    """gdn_load_gdnstate refuses a header that disagrees with the model
    before it sizes a buffer from it.  Without a GPU the run state has no
    engine, so a file that passes the header checks stops at the first
    device upload instead ("not initialised")."""
    cfg = g.default_config(1)
    cfg.vocab_size, cfg.hidden_size, cfg.num_heads, cfg.num_v_heads = 64, 64, 1, 1
    cfg.head_dim, cfg.intermediate_size = 64, 128
    m = g.Model.synth(config=cfg, seed=1)
    lib = _lib.load()
    p = tmp_path / "s.gdnstate"
    expect = {"dv_huge": "x 64 x 4294967295", "dv_small": "x 64 x 32", "version": "version 2",
              "layers": "2 layers", "short": "ends inside its recurrent-state section"}[case]
    if case == "dv_huge":
        write_gdnstate(p, cfg, dv=0xffffffff)   # about 2^38 floats if sized from the file
    elif case == "dv_small":
        write_gdnstate(p, cfg, dv=32)
    elif case == "version":
        write_gdnstate(p, cfg, version=2)
    elif case == "layers":
        c2 = g.default_config(2)
        for k in ("vocab_size", "hidden_size", "num_heads", "num_v_heads", "head_dim", "intermediate_size"):
            setattr(c2, k, getattr(cfg, k))
        write_gdnstate(p, c2)
    else:
        write_gdnstate(p, cfg, prompt=[1, 2, 3], payload=False)
    capfd.readouterr()
    rs = _lib.GDNRunState()
    plen, seed = ctypes.c_uint32(), ctypes.c_int32()
    rc = lib.gdn_load_gdnstate(ctypes.byref(rs), m.ptr, str(p).encode(), ctypes.byref(plen), ctypes.byref(seed))
    assert rc == -1
    assert expect in capfd.readouterr().err
    # the well-formed file passes the header and stops only at the missing engine
    write_gdnstate(p, cfg, prompt=[5, 6])
    rc = lib.gdn_load_gdnstate(ctypes.byref(rs), m.ptr, str(p).encode(), ctypes.byref(plen), ctypes.byref(seed))
    assert rc == -1 and "not initialised" in capfd.readouterr().err
    m.free()
