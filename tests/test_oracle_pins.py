"""Pins of the oracle (oracle/dfssm_oracle.c) that do not need the reference build: exhaustive fp16
conversion, bit order, exact integer scaffold against brute force, the fp16 rounding points of
the reference's PyTorch expressions evaluated by torch on the CPU, closed forms of the SSM, the
head/argmax rule, and the accuracy of the oracle's own exp/log1p against fp64."""
import ctypes

import numpy as np
import pytest
import torch

from dfssm.format import pack_sign_bits, unpack_sign_bits
from oracle import oracle as O


def _arr(fn, x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    getattr(O.lib(), fn)(O._p(x), O._p(out), ctypes.c_long(x.size))
    return out


# ------------------------------------------------------------------ fp16 conversion
def test_f2h_exhaustive_halves_roundtrip():
    h = np.arange(65536, dtype=np.uint16).view(np.float16)
    f = h.astype(np.float32)
    back = O.f2h(f)
    finite = np.isfinite(f)
    assert np.array_equal(back.view(np.uint16)[finite], h.view(np.uint16)[finite])
    assert np.all(np.isnan(back[np.isnan(f)]))


def test_f2h_random_and_ties_match_numpy():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.normal(0, 1, 200000), rng.normal(0, 3e4, 20000), rng.normal(0, 1e-5, 20000),
                        np.array([65504, 65519.99, 2 ** -24, 2 ** -25, 3 * 2 ** -26, -2 ** -25])]
                       ).astype(np.float32)
    # exact ties: halfway between consecutive halves
    h = rng.integers(0x0400, 0x7bff, 10000).astype(np.uint16).view(np.float16)
    mid = (h.astype(np.float64) + np.nextafter(h, np.float16(np.inf)).astype(np.float64)) / 2
    x = np.concatenate([x, mid.astype(np.float32)])
    assert np.array_equal(O.f2h(x).view(np.uint16), x.astype(np.float16).view(np.uint16))
    # overflow: RNE rounds to infinity from 65520 up
    big = O.f2h(np.float32([65520, 1e6, -1e6, np.inf]))
    assert np.isposinf(big[0]) and np.isposinf(big[1]) and np.isneginf(big[2]) and np.isposinf(big[3])


# ------------------------------------------------------------------ bits + scaffold
def test_unpack_matches_format_module():
    rng = np.random.default_rng(1)
    p = rng.integers(0, 2 ** 32, (17, 8), dtype=np.uint32)
    assert np.array_equal(O.unpack_bits(p), unpack_sign_bits(p))


@pytest.mark.parametrize("M,N,K", [(1, 8512, 2048), (4, 200, 4096), (3, 64, 512)])
def test_scaffold_acc_brute_force(M, N, K):
    rng = np.random.default_rng([M, N, K])
    bits = rng.integers(0, 2 ** 32, (N, K // 32), dtype=np.uint32)
    q = rng.integers(-128, 128, (M, K)).astype(np.int8)
    ref = q.astype(np.int64) @ unpack_sign_bits(bits).astype(np.int64).T
    assert np.array_equal(O.scaffold_acc(bits, q), ref)


def test_scaffold_extremes():
    K = 2048
    bits = np.stack([np.full(K // 32, 0xFFFFFFFF, np.uint32), np.zeros(K // 32, np.uint32)])
    q = np.stack([np.full(K, 127, np.int8), np.full(K, -128, np.int8)])
    acc = O.scaffold_acc(bits, q)
    assert acc.tolist() == [[127 * K, -127 * K], [-128 * K, 128 * K]]


# ------------------------------------------------------------------ fp16 rounding points vs torch (CPU)
def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


def test_quantize_given_scale_matches_torch():
    """(x / scale).round().clamp(-128, 127).to(int8) of df_ssm_inference.py:151, evaluated by torch
    in fp16 on the CPU (tensor/tensor division: IEEE fp32, rounded to fp16, then round-half-even)."""
    rng = np.random.default_rng(2)
    xn = (rng.normal(0, 1, (8, 2048)) * rng.uniform(0.01, 50, (8, 1))).astype(np.float16)
    q, s = O.quantize(xn)
    tq = (_t(xn) / _t(s)[:, None]).round().clamp(-128, 127).to(torch.int8).numpy()
    assert np.array_equal(q, tq)


def test_quantize_scale_rule():
    """scale = fp16(fp16(max(amax, 1e-4)) * fp32(1/127)) (df_ssm_inference.py:150): ATen's GPU kernel
    divides a tensor by a scalar by multiplying with the scalar's fp32 reciprocal; checked on every
    positive fp16 amax. True fp32 division gives the same fp16 scale for every one of them, so the
    scale does not depend on which of the two the reference's build uses."""
    amax = np.arange(0x0001, 0x7c00, dtype=np.uint16).view(np.float16)
    x = np.zeros((amax.size, 64), np.float16)
    x[:, 0] = amax
    _, s = O.quantize(x)
    c = np.maximum(amax.astype(np.float32), np.float32(1e-4)).astype(np.float16).astype(np.float32)
    want = (c * np.float32(1.0 / 127.0)).astype(np.float16)
    assert np.array_equal(s.view(np.uint16), want.view(np.uint16))
    div = (c / np.float32(127.0)).astype(np.float16)
    assert np.array_equal(div.view(np.uint16), want.view(np.uint16))
    # all-zero row: amax clamps to fp16(1e-4); outputs are 0
    q0, s0 = O.quantize(np.zeros((1, 512), np.float16))
    assert not q0.any() and float(s0[0]) == float(np.float16(np.float16(1e-4).astype(np.float32) / 127))


def test_rmsnorm_matches_torch_expression():
    """_rms_norm (df_ssm_inference.py:141-145) in torch on the CPU, then copy_ into fp16."""
    rng = np.random.default_rng(3)
    x = (rng.normal(0, 1, (16, 2048)) * rng.uniform(0.1, 30, (16, 1))).astype(np.float16)
    w = (1 + rng.uniform(-0.1, 0.1, 2048)).astype(np.float32)
    tx = _t(x)
    var = tx.float().pow(2).mean(dim=-1, keepdim=True)
    ref = ((tx * torch.rsqrt(var + 1e-5)) * _t(w)).half().numpy()
    got = O.rmsnorm(x, w)
    d = np.abs(got.view(np.uint16).astype(np.int32) - ref.view(np.uint16).astype(np.int32))
    # the sum of squares is order dependent (torch: fp32 vector lanes; oracle: fp64); rsqrt's
    # last bit may differ, which moves an element by at most one fp16 ulp, rarely
    assert d.max() <= 1 and (d > 0).mean() < 1e-3


def test_gate_matches_torch_expression():
    """silu_z = z * sigmoid(z); gated = y * silu_z in fp16 (df_ssm_inference.py:194-195)."""
    rng = np.random.default_rng(4)
    z = rng.normal(0, 3, (4, 4096)).astype(np.float16)
    y = rng.normal(0, 2, (4, 4096)).astype(np.float16)
    tz = _t(z)
    ref = (_t(y) * (tz * torch.sigmoid(tz))).numpy()
    got = O.gate(y, z)
    d = np.abs(got.view(np.uint16).astype(np.int32) - ref.view(np.uint16).astype(np.int32))
    # sigmoid uses a different exp (1 ulp) before rounding to fp16: rare 1-ulp differences
    assert d.max() <= 1 and (d > 0).mean() < 2e-3


def test_lora_matches_torch_fp16_gemms():
    """proj.addmm_(x_norm @ B16.T, A16.T) with B16/A16 the load-time fp16 dequant
    (df_ssm_inference.py:82-83,173), evaluated by torch on the CPU."""
    rng = np.random.default_rng(5)
    K, N, M = 2048, 512, 3
    xn = rng.normal(0, 1, (M, K)).astype(np.float16)
    lA = np.clip(np.rint(rng.normal(0, 20, (N, 16))), -127, 127).astype(np.int8)
    lB = np.clip(np.rint(rng.normal(0, 20, (16, K))), -127, 127).astype(np.int8)
    lAs = (1.7e-3 * rng.uniform(0.5, 1.5, N)).astype(np.float16)
    lBs = (rng.uniform(0.5, 1.5, 16) / (20 * np.sqrt(K))).astype(np.float16)
    A16 = (_t(lA).float() * _t(lAs).float().unsqueeze(1)).half()
    B16 = (_t(lB).float() * _t(lBs).float().unsqueeze(1)).half()
    h16 = (_t(xn) @ B16.T)
    h = O.lora_h(xn, lB, lBs)
    dh = np.abs(h.astype(np.float32) - h16.float().numpy())
    assert dh.max() <= 2 * np.abs(h16.float().numpy()).max() * 2 ** -11
    # epilogue: y + h16 @ A16^T with y = 0 (acc 0) checks the A-side dequant and the sum
    acc = np.zeros((M, N), np.int32)
    out = O.dequant_lora(acc, np.ones(M, np.float16), np.ones(N, np.float16), h, lA, lAs)
    ref = (torch.from_numpy(h.astype(np.float32)) @ A16.float().T).numpy()
    assert np.abs(out.astype(np.float32) - ref).max() <= np.abs(ref).max() * 2 ** -10


def test_dequant_rounding_chain():
    """y = fp16(fp16(fp16(acc) * s_x) * s_w): int32 -> fp16 then two fp16 tensor products
    (df_ssm_inference.py:158); acc beyond 2048 loses integer precision as in the reference."""
    acc = np.array([[0, 1, 2047, 2049, 4097, -65504, 70000]], np.int32)
    xs = np.array([0.03], np.float16)
    ws = np.linspace(0.01, 0.05, acc.shape[1]).astype(np.float16)
    out = O.dequant_lora(acc, xs, ws, np.zeros((1, 16), np.float16), np.zeros((acc.shape[1], 16), np.int8),
                         np.zeros(acc.shape[1], np.float16))
    ref = ((_t(acc).half() * _t(xs)[:, None]) * _t(ws)[None, :]).numpy()
    assert np.array_equal(out.view(np.uint16), ref.view(np.uint16))


# ------------------------------------------------------------------ SSM closed forms
def _ssm_inputs(M=2, H=4, P=16, N=128, seed=6):
    rng = np.random.default_rng(seed)
    xbc = rng.normal(0, 1, (M, H * P + 2 * N)).astype(np.float16)
    dt = rng.normal(-1, 1, (M, H)).astype(np.float16)
    return rng, xbc, dt, np.zeros(H, np.float32), rng.uniform(0, np.log(16), H).astype(np.float32)


def test_ssm_decay_without_input():
    """B = 0: h_t = Abar^t h_0 with Abar = exp(dt * -exp(A_log)) in (0, 1)."""
    M, H, P, N = 2, 4, 16, 128
    rng, xbc, dt, dtb, A_log = _ssm_inputs(M, H, P, N)
    xbc[:, H * P:H * P + N] = 0                      # B = 0
    h0 = rng.normal(0, 1, (M, H, P, N)).astype(np.float32)
    h = h0.copy()
    O.ssm_step(h, xbc, dt, dtb, A_log, np.ones(H, np.float32))
    sp = np.log1p(np.exp(dt.astype(np.float64) + dtb))
    abar = np.exp(sp * -np.exp(A_log.astype(np.float64)))
    assert np.all((abar > 0) & (abar < 1))
    np.testing.assert_allclose(h, h0 * abar[:, :, None, None], rtol=1e-6)


def test_ssm_readout_and_skip():
    """From h = 0: h1 = (x dt) B (outer product) and y = C.h1 + D x."""
    M, H, P, N = 1, 2, 16, 128
    rng, xbc, dt, dtb, A_log = _ssm_inputs(M, H, P, N, seed=7)
    Dp = rng.uniform(0.5, 1.5, H).astype(np.float32)
    h = np.zeros((M, H, P, N), np.float32)
    y = O.ssm_step(h, xbc, dt, dtb, A_log, Dp)
    x = xbc[0, :H * P].astype(np.float64).reshape(H, P)
    Bv, Cv = xbc[0, H * P:H * P + N].astype(np.float64), xbc[0, H * P + N:].astype(np.float64)
    sp = np.log1p(np.exp(dt[0].astype(np.float64)))
    h1 = (x * sp[:, None])[:, :, None] * Bv[None, None, :]
    np.testing.assert_allclose(h[0], h1, rtol=2e-6, atol=1e-7)
    ych = (h1 * Cv).sum(-1) + x * Dp[:, None]
    np.testing.assert_allclose(y[0].astype(np.float64).reshape(H, P), ych, rtol=2e-3, atol=2e-3)


def test_conv_shift_register():
    """state <- (s1, s2, x); out = silu(s0 w0 + s1 w1 + s2 w2 + x w3 + b) (df_ssm_kernels.cu:39-46)."""
    rng = np.random.default_rng(8)
    M, C = 2, 64
    st = rng.normal(0, 1, (M, C, 3)).astype(np.float16)
    x = rng.normal(0, 1, (M, C)).astype(np.float16)
    w = rng.normal(0, 0.5, (C, 4)).astype(np.float16)
    b = rng.normal(0, 0.1, C).astype(np.float16)
    st0, x0 = st.copy(), x.copy()
    O.conv_step(st, x, w, b)
    assert np.array_equal(st[:, :, :2], st0[:, :, 1:]) and np.array_equal(st[:, :, 2], x0)
    o = (st0[:, :, 0].astype(np.float64) * w[:, 0] + st0[:, :, 1] * w[:, 1].astype(np.float64)
         + st0[:, :, 2] * w[:, 2].astype(np.float64) + x0 * w[:, 3].astype(np.float64) + b)
    np.testing.assert_allclose(x.astype(np.float64), o / (1 + np.exp(-o)), rtol=2e-3, atol=2e-3)


# ------------------------------------------------------------------ head + argmax
def test_lm_head_exact_and_first_index_ties():
    from dfssm.synth import config_tiny, make_weights
    w = make_weights(config_tiny(n_layer=1), seed=9)
    rng = np.random.default_rng(9)
    xf = rng.normal(0, 1, (3, w.cfg.d_model)).astype(np.float16)
    logits, nxt = O.lm_head(w, xf)
    exact = xf.astype(np.float64) @ w.emb.astype(np.float64).T     # exact: fp16 x int8 in fp64
    ref = (exact.astype(np.float32) * w.emb_scale.astype(np.float32)).astype(np.float16)
    assert np.array_equal(logits.view(np.uint16), ref.view(np.uint16))
    assert np.array_equal(nxt, np.argmax(logits.astype(np.float32), axis=1))
    # a tie: duplicate the winning row further down -> the first index wins
    w.emb[-1] = w.emb[nxt[0]]
    w.emb_scale[-1] = w.emb_scale[nxt[0]]
    _, nxt2 = O.lm_head(w, xf[:1])
    assert nxt2[0] == nxt[0]


# ------------------------------------------------------------------ own exp / log1p
def test_exp_accuracy_and_specials():
    x = np.concatenate([np.linspace(-86, 88.7, 400001, dtype=np.float32), np.float32([0, -0.0, 1e-30, 0.5])])
    e = _arr("or_expf_array", x)
    ref = np.exp(x.astype(np.float64))
    ulp = np.abs(e - ref) / np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert ulp.max() <= 1.0
    sp = _arr("or_expf_array", np.float32([-86.5, -1000, 89.5, 1e30, np.nan]))
    assert sp[0] == 0 and sp[1] == 0 and np.isinf(sp[2]) and np.isinf(sp[3]) and np.isnan(sp[4])


def test_log1p_accuracy_and_specials():
    y = np.concatenate([np.exp(np.linspace(-86, 88, 400001)).astype(np.float32), np.float32([1e-45, 1, 2, 3e38])])
    l = _arr("or_log1pf_array", y)
    ref = np.log1p(y.astype(np.float64))
    ulp = np.abs(l - ref) / np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert ulp.max() <= 3.0
    sp = _arr("or_log1pf_array", np.float32([0, np.inf, np.nan]))
    assert sp[0] == 0 and np.isinf(sp[1]) and np.isnan(sp[2])
