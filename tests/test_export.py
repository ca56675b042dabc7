"""Exporter (row f2): float student weights -> .dfssm, as training/export_dfssm.py converts them.

Pinned by known answers of each conversion (sign bits including exact zeros, mean |w| scale,
per-row int8 quantization with round-half-even and the 1e-8 floor, LoRA scaling folded into A),
by the byte layout (file size from the header, header fields), and by a round trip: a synthetic
student state dict exported, read back, unpacked and run through the oracle.
"""
import struct
import warnings

import numpy as np
import pytest
import torch

from dfssm.export import (export_dfssm, lora_factors, quantize_rows_int8, scaffold_bits_and_scale,
                          weights_from_state_dict)
from dfssm.format import EMB_F16, EMB_I8, HEADER_FMT, expected_size, read_dfssm, unpack_sign_bits


def test_sign_bits_known_answers():
    w = -np.ones((2, 64), np.float32)
    w[0, 0] = 0.3          # word 0, bit 0
    w[0, 33] = 2.0         # word 1, bit 1
    w[1, 31] = 1e-30       # word 0, bit 31 (any positive value)
    w[1, 5] = 0.0          # exact zero: (sign(0) + 1) // 2 = 0 -> -1
    w[1, 6] = -0.0
    packed, _ = scaffold_bits_and_scale(w)
    assert packed.dtype == np.uint32 and packed.shape == (2, 2)
    assert packed[0].tolist() == [1, 2]
    assert packed[1].tolist() == [1 << 31, 0]
    signs = unpack_sign_bits(packed)
    np.testing.assert_array_equal(signs, np.where(w > 0, 1, -1))


def test_scale_is_fp16_of_mean_abs():
    w = np.array([[1.0, -3.0, 0.0, 4.0] * 8, [0.5] * 32], np.float32)
    _, s = scaffold_bits_and_scale(w)
    assert s.dtype == np.float16
    assert s.tolist() == [2.0, 0.5]
    rng = np.random.default_rng(0)
    w = rng.normal(0, 0.02, (64, 512)).astype(np.float32)
    _, s = scaffold_bits_and_scale(w)
    ref = np.abs(w.astype(np.float64)).mean(axis=1)
    # fp32 mean then fp16: within one fp16 ulp of the exact mean
    assert np.all(np.abs(s.astype(np.float64) - ref) <= np.spacing(s.astype(np.float16)).astype(np.float64))


def test_quantize_rows_int8_known_answers():
    w = np.array([[127.0, -63.5, 0.5, 1.5, 2.5, -127.0, 0.0, 64.5],
                  [0.0] * 8,
                  [-254.0, 1.0, 3.0, 5.0, 0.0, 0.0, 0.0, 0.0]], np.float32)
    q, s = quantize_rows_int8(w)
    assert q.dtype == np.int8 and s.dtype == np.float16
    # row 0: s = 1; round half to even: -63.5 -> -64, 0.5 -> 0, 1.5 -> 2, 2.5 -> 2, 64.5 -> 64
    assert q[0].tolist() == [127, -64, 0, 2, 2, -127, 0, 64]
    assert float(s[0]) == 1.0
    # row 1: all zero -> s = 1e-8 (fp16 0, as the reference stores it), q = 0
    assert q[1].tolist() == [0] * 8 and float(s[1]) == float(np.float16(1e-8))
    # row 2: s = 2: 1 / 2 = 0.5 -> 0, 3 / 2 = 1.5 -> 2, 5 / 2 = 2.5 -> 2
    assert q[2].tolist() == [-127, 0, 2, 2, 0, 0, 0, 0] and float(s[2]) == 2.0


def test_lora_scaling_folded_into_A():
    rng = np.random.default_rng(1)
    A = rng.normal(0, 0.01, (32, 16)).astype(np.float32)
    B = rng.normal(0, 0.01, (16, 64)).astype(np.float32)
    qa, sa, qb, sb = lora_factors(A, B, 1.0 / 16)
    qa2, sa2 = quantize_rows_int8(A * np.float32(1.0 / 16))
    np.testing.assert_array_equal(qa, qa2)
    np.testing.assert_array_equal(sa, sa2)
    # the largest |entry| of every row maps to +-127
    assert np.all(np.abs(qa.astype(int)).max(axis=1) == 127)
    assert np.all(np.abs(qb.astype(int)).max(axis=1) == 127)
    # dequantized within half a step of the input
    step = (np.abs(A / 16).max(axis=1) / 127)[:, None]
    assert np.all(np.abs(qa * step - A / 16) <= 0.5 * step * (1 + 1e-5))


def _student_sd(n_layer=2, D=512, DI=1024, H=16, N=128, V=1000, seed=0):
    """A synthetic state dict with the student's names and shapes; the frozen scaffold weights sit
    on the 17 density levels of Kw = 4 (df_ssm_dfw_lora.py:56-61), so exact zeros occur."""
    g = torch.Generator().manual_seed(seed)
    IPO, C = 2 * DI + 2 * N + H, DI + 2 * N
    sd = {"embedding.weight": torch.randn(V, D, generator=g) * 0.05, "norm_f.weight": 1 + 0.1 * torch.randn(D, generator=g)}

    def frozen(o, i):
        lv = torch.randint(0, 17, (o, i), generator=g).float() / 16 * 2 - 1
        return lv * (0.01 + 0.04 * torch.rand(o, 1, generator=g))

    for l in range(n_layer):
        p = f"layers.{l}.mixer."
        sd[p + "in_proj.frozen_weight"] = frozen(IPO, D)
        sd[p + "in_proj.lora_A"] = torch.randn(IPO, 16, generator=g) * 0.01
        sd[p + "in_proj.lora_B"] = torch.randn(16, D, generator=g) * 0.01
        sd[p + "out_proj.frozen_weight"] = frozen(D, DI)
        sd[p + "out_proj.lora_A"] = torch.randn(D, 16, generator=g) * 0.01
        sd[p + "out_proj.lora_B"] = torch.randn(16, DI, generator=g) * 0.01
        sd[p + "conv1d.weight"] = torch.randn(C, 1, 4, generator=g) * 0.5
        sd[p + "conv1d.bias"] = torch.randn(C, generator=g) * 0.1
        sd[p + "A_log"] = torch.rand(H, generator=g) * np.log(16)
        sd[p + "D"] = torch.ones(H)
        sd[p + "dt_bias"] = torch.randn(H, generator=g) - 3
        sd[p + "norm.weight"] = 1 + 0.1 * torch.randn(DI, generator=g)
        sd[f"layers.{l}.norm.weight"] = 1 + 0.1 * torch.randn(D, generator=g)
    return sd


def test_roundtrip_student(tmp_path):
    sd = _student_sd()
    path = str(tmp_path / "student.dfssm")
    n = export_dfssm(sd, path)
    w = read_dfssm(path)
    c = w.cfg
    assert n == expected_size(c) and (c.n_layer, c.d_model, c.d_inner, c.nheads, c.vocab_size) == (2, 512, 1024, 16, 1000)
    assert c.headdim == 64 and c.emb_code == EMB_F16
    raw = open(path, "rb").read(64)
    magic, L, D, DI, N, H, P, G, V, kw, res = struct.unpack(HEADER_FMT, raw)
    assert (magic, L, D, DI, N, H, P, G, V, kw) == (b"DFSSM001", 2, 512, 1024, 128, 16, 64, 1, 1000, 4)
    assert res == b"\x00" * 20  # an fp16-table export leaves every reserved byte zero, as the reference
    for l in range(2):
        p = f"layers.{l}.mixer."
        L = w.layers[l]
        for pre in ("in", "out"):
            fw = sd[p + f"{pre}_proj.frozen_weight"].numpy()
            assert (fw == 0).any()
            np.testing.assert_array_equal(unpack_sign_bits(L[f"{pre}_packed"]), np.where(fw > 0, 1, -1))
            np.testing.assert_array_equal(L[f"{pre}_scale"], np.abs(fw).mean(axis=1).astype(np.float16))
        np.testing.assert_array_equal(L["conv_w"], sd[p + "conv1d.weight"].squeeze(1).numpy().astype(np.float16))
        np.testing.assert_array_equal(L["A_log"], sd[p + "A_log"].numpy())
        np.testing.assert_array_equal(L["ln_w"], sd[f"layers.{l}.norm.weight"].numpy())
    np.testing.assert_array_equal(w.emb, sd["embedding.weight"].numpy().astype(np.float16))
    # the exported model runs through the oracle
    from dfssm.synth import make_prompts
    from oracle import oracle as O
    toks, _ = O.OracleModel(w, 2).generate(make_prompts(2, c.vocab_size, 3), 3)
    assert toks.shape == (2, 3) and (toks >= 0).all() and (toks < c.vocab_size).all()


def test_export_options(tmp_path):
    sd = _student_sd(n_layer=1)
    path = str(tmp_path / "ref_header.dfssm")
    export_dfssm(sd, path, headdim_field=32, emb_code=EMB_I8, lora_alpha=2.0)
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        w = read_dfssm(path)
    assert w.cfg.headdim == 32 and w.cfg.p == 64 and any("headdim" in str(r.message) for r in rec)
    assert w.cfg.emb_code == EMB_I8 and w.emb.dtype == np.int8 and w.emb_scale.dtype == np.float16
    qa, sa, _, _ = lora_factors(sd["layers.0.mixer.in_proj.lora_A"], sd["layers.0.mixer.in_proj.lora_B"], 2.0 / 16)
    np.testing.assert_array_equal(w.layers[0]["in_lA"], qa)
    with pytest.raises(ValueError):
        weights_from_state_dict(sd, lora_rank=8)
