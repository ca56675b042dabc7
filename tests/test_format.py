"""The .dfssm format: byte layout and sizes (training/export_dfssm.py:104-193), header extension,
validation of malformed files, bit packing known answers."""
import struct
import warnings

import numpy as np
import pytest

from dfssm.format import (DFSSMConfig, DFSSMFormatError, EMB_F16, EMB_I8, HEADER_FMT, NORM_F16,
                          expected_size, layer_bytes, layer_tensor_specs, pack_sign_bits, parse_header,
                          read_dfssm, unpack_sign_bits, write_dfssm)
from dfssm.synth import config_1p3b, config_2p7b, config_tiny, make_weights


def test_sizes_match_exporter_layout():
    # per-layer bytes of the 1.3B shape, summing the write_tensor calls of export_dfssm.py:135-185
    D, DI, N, H, R = 2048, 4096, 128, 64, 16
    IPO, C = 2 * DI + 2 * N + H, DI + 2 * N
    by_hand = (IPO * D // 8 + 2 * IPO + IPO * R + 2 * IPO + R * D + 2 * R
               + D * DI // 8 + 2 * D + D * R + 2 * D + R * DI + 2 * R
               + C * 4 * 2 + C * 2 + 3 * H * 4 + DI * 4 + D * 4)
    assert layer_bytes(config_1p3b()) == by_hand == 3_606_080
    assert expected_size(config_1p3b(EMB_F16)) == 64 + 50288 * 2048 * 2 + 48 * by_hand + 2048 * 4
    assert expected_size(config_1p3b(EMB_F16)) == 379_079_744
    assert expected_size(config_1p3b(EMB_I8)) == 276_190_496
    assert layer_bytes(config_2p7b()) == 5_493_824
    assert [n for n, _, _ in layer_tensor_specs(config_1p3b())][:3] == ["in_packed", "in_scale", "in_lA"]


def test_header_is_the_exporter_struct():
    c = config_1p3b()
    h = c.header_bytes()
    assert len(h) == 64
    magic, L, D, DI, N, H, hd, ng, V, kw, reserved = struct.unpack(HEADER_FMT, h)
    assert (magic, L, D, DI, N, H, hd, ng, V, kw) == (b"DFSSM001", 48, 2048, 4096, 128, 64, 64, 1, 50288, 4)
    assert reserved[0] == EMB_I8 and reserved[1] == 0 and not any(reserved[2:])
    assert parse_header(h) == c


@pytest.mark.parametrize("emb_code", [EMB_I8, EMB_F16])
def test_roundtrip(tmp_path, emb_code):
    w = make_weights(config_tiny(n_layer=2, emb_code=emb_code), seed=3)
    p = tmp_path / "m.dfssm"
    n = write_dfssm(str(p), w)
    assert n == p.stat().st_size == expected_size(w.cfg)
    r = read_dfssm(str(p))
    assert r.cfg == w.cfg
    assert np.array_equal(r.emb, w.emb)
    for a, b in zip(r.layers, w.layers):
        for k in a:
            assert np.array_equal(a[k], b[k]), k
    assert np.array_equal(r.norm_f, w.norm_f)


def test_fp16_norm_variant(tmp_path):
    c = config_tiny(n_layer=1)
    c16 = DFSSMConfig(**{**c.__dict__, "norm_code": NORM_F16})
    w = make_weights(c16, seed=1)
    assert w.layers[0]["norm_w"].dtype == np.float16
    p = tmp_path / "n16.dfssm"
    write_dfssm(str(p), w)
    assert read_dfssm(str(p)).layers[0]["ln_w"].dtype == np.float16


def test_rejects_truncated_and_oversized(tmp_path):
    w = make_weights(config_tiny(n_layer=1), seed=0)
    p = tmp_path / "m.dfssm"
    write_dfssm(str(p), w)
    raw = p.read_bytes()
    (tmp_path / "short.dfssm").write_bytes(raw[:-1])
    (tmp_path / "long.dfssm").write_bytes(raw + b"\0")
    for name in ("short.dfssm", "long.dfssm"):
        with pytest.raises(DFSSMFormatError, match="does not match"):
            read_dfssm(str(tmp_path / name))


def test_rejects_bad_magic_reserved_and_dims(tmp_path):
    w = make_weights(config_tiny(n_layer=1), seed=0)
    p = tmp_path / "m.dfssm"
    write_dfssm(str(p), w)
    raw = bytearray(p.read_bytes())
    bad = bytearray(raw); bad[:8] = b"DFSSM002"
    with pytest.raises(DFSSMFormatError, match="magic"):
        parse_header(bytes(bad))
    bad = bytearray(raw); bad[44 + 5] = 1
    with pytest.raises(DFSSMFormatError, match="reserved"):
        parse_header(bytes(bad))
    bad = bytearray(raw); bad[44] = 7
    with pytest.raises(DFSSMFormatError, match="embedding code"):
        parse_header(bytes(bad))
    bad = bytearray(raw); struct.pack_into("<I", bad, 8 + 4 * 4, 7)   # nheads = 7 does not divide d_inner
    with pytest.raises(DFSSMFormatError):
        parse_header(bytes(bad))
    with pytest.raises(DFSSMFormatError):
        parse_header(b"DFSSM001")


def test_headdim_mismatch_warns(tmp_path):
    # the reference exporter writes headdim=32 for a 64-wide head (export_dfssm.py:24,114)
    c = config_tiny(n_layer=1)
    c32 = DFSSMConfig(**{**c.__dict__, "headdim": 32})
    w = make_weights(c32, seed=0)
    p = tmp_path / "h.dfssm"
    write_dfssm(str(p), w)
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        r = read_dfssm(str(p))
    assert any("headdim" in str(x.message) for x in rec)
    assert r.cfg.p == c.d_inner // c.nheads


def test_bit_order_known_answers():
    # export_dfssm.py:34-42: word j bit b <- column 32j + b; bit 1 -> +1 (sign >= 0), 0 -> -1
    row = np.zeros(64, np.uint8)
    row[0] = 1
    row[31] = 1
    row[33] = 1
    p = pack_sign_bits(row[None, :])
    assert p.dtype == np.uint32 and p.shape == (1, 2)
    assert p[0, 0] == 0x80000001 and p[0, 1] == 0x2
    u = unpack_sign_bits(p)[0]
    assert u[0] == 1 and u[31] == 1 and u[33] == 1 and u[1] == -1 and u[32] == -1
    assert np.array_equal(unpack_sign_bits(np.array([[0x1]], np.uint32))[0], np.r_[1, -np.ones(31)].astype(np.int8))


def test_pack_unpack_roundtrip():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2, (37, 256)).astype(np.uint8)
    assert np.array_equal((unpack_sign_bits(pack_sign_bits(bits)) + 1) // 2, bits)
