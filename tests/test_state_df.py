"""Pins of the oracle's density-field state quantization (or_state_df), CPU only.

Row f4 restates df_ssd_scan's chunk-boundary quantization (training/df_ssm_mamba2_distill_dfw.py:
139-165), SprayBank.quantize (:88-91) and _quantize_error (:105-110). Checks:
  * against a float64 NumPy evaluation of the reference's formula (torch.std unbiased,
    searchsorted side='left', round half to even): identical quantization levels wherever the
    value is clear of every threshold, dequantized state and error within fp32 rounding;
  * closed forms: a constant row (std clamped to 1e-8) and a row of +-a;
  * the count is numpy.searchsorted(side='left') including values exactly on a threshold;
  * the error is a multiple of 2^-(bits-1) in [-1, 1], and exact hc - q with bits >= 32.
"""
import numpy as np
import pytest

from oracle import oracle as O


def _ref64(h, R, e=None, bits=8):
    """df_ssd_scan's boundary step in float64 (torch semantics)."""
    h = h.astype(np.float64)
    mean = h.mean(axis=1, keepdims=True)
    std = np.maximum(h.std(axis=1, ddof=1, keepdims=True), 1e-8)
    lo = mean - 3.0 * std
    rng = np.maximum(6.0 * std, 1e-8)
    hs = np.clip((h - lo) / rng, 0, 1)
    hc = hs if e is None else np.clip(hs + e.astype(np.float64), 0, 1)
    cnt = np.searchsorted(R.astype(np.float64), hc, side="left")
    q = cnt / R.size
    err = None
    if e is not None:
        err = np.clip(hc - q, -1, 1)
        if bits < 32:
            err = np.round(err * 2 ** (bits - 1)) / 2 ** (bits - 1)
    return q * rng + lo, err, cnt, hc


def _rows(n, seed):
    rng = np.random.default_rng(seed)
    scale = 10.0 ** rng.uniform(-4, 2, (n, 1))
    return (rng.normal(0, 1, (n, 128)) * scale + rng.normal(0, 1, (n, 1)) * scale).astype(np.float32)


@pytest.mark.parametrize("kk,sd,bits", [(64, False, 8), (64, True, 8), (16, True, 8), (64, True, 32)])
def test_matches_reference_formula(kk, sd, bits):
    rng = np.random.default_rng(kk + bits)
    h = _rows(512, kk)
    R = np.sort(rng.random(kk).astype(np.float32))
    e = (np.round(rng.uniform(-0.02, 0.02, h.shape) * 128) / 128).astype(np.float32) if sd else None
    got, gerr = O.state_density_field(h, R, e, bits)
    ref, rerr, cnt, hc = _ref64(h, R, e, bits)
    clear = np.min(np.abs(hc[..., None] - R.astype(np.float64)), axis=-1) > 1e-5
    assert clear.mean() > 0.99
    # same level where clear of the thresholds: the dequantized state agrees to fp32 rounding
    rngw = (np.maximum(6 * h.astype(np.float64).std(axis=1, ddof=1), 1e-8))[:, None]
    lo = (h.astype(np.float64).mean(axis=1, keepdims=True) - rngw / 2)
    qg = np.rint((got.astype(np.float64) - lo) / rngw * kk)
    np.testing.assert_array_equal(qg[clear], cnt[clear])
    assert np.all(np.abs(got - ref)[clear] <= 1e-5 * (rngw + np.abs(lo)).repeat(128, 1)[clear])
    if sd:
        tol = 2.0 ** -(bits - 1) if bits < 32 else 1e-6
        assert np.all(np.abs(gerr - rerr)[clear] <= 1e-6 + (0 if bits >= 32 else 0))
        assert np.max(np.abs(gerr)) <= 1.0 and tol > 0


def test_constant_row_and_pm_row():
    R = np.array([0.25, 0.75], np.float32)
    h = np.zeros((1, 128), np.float32)
    got, _ = O.state_density_field(h, R)
    # std 0 -> 1e-8: hs = 3e-8 / 6e-8 = 0.5 -> one threshold below -> q = 0.5 -> h = 0.5 * 6e-8 - 3e-8 = 0
    assert np.all(got == 0.0)
    h = np.where(np.arange(128) % 2 == 0, 2.0, -2.0).astype(np.float32)[None]
    R = ((np.arange(64) + 0.5) / 64).astype(np.float32)
    got, _ = O.state_density_field(h, R)
    std = 2.0 * np.sqrt(128 / 127)
    for v in (2.0, -2.0):
        hs = (v + 3 * std) / (6 * std)
        q = np.searchsorted(R.astype(np.float64), hs) / 64
        assert np.allclose(got[0][h[0] == v], q * 6 * std - 3 * std, rtol=0, atol=1e-6)


def test_count_is_searchsorted_left():
    R = np.array([0.1, 0.2, 0.2, 0.5, 0.9], np.float32)
    # rows whose scaled values land exactly on thresholds: h = lo + v * range needs exact fp32
    # arithmetic, so check the count rule through tiny rows with known hs instead: a row of 64
    # zeros and 64 copies of c has mean c/2 and hs in {a, 1 - a}; sweep c and compare
    for c in (1.0, 3.0, 0.5):
        h = np.concatenate([np.zeros(64), np.full(64, c)]).astype(np.float32)[None]
        got, _ = O.state_density_field(h, R, None, 8)
        ref, _, cnt, _ = _ref64(h, R)
        np.testing.assert_allclose(got, ref, rtol=0, atol=1e-6)
    # exact threshold hits: an outlier (hs clamped to 1) with sigma-delta input e = R[j] - 1 has
    # hc = 1 + (R[j] - 1) = R[j] exactly; the threshold itself is not counted (strict <)
    R = np.array([0.5, 0.75], np.float32)
    h = np.zeros((1, 128), np.float32)
    h[0, 0] = 1000.0
    for j, want in ((1, 1), (0, 0)):
        e = np.zeros((1, 128), np.float32)
        e[0, 0] = R[j] - np.float32(1.0)
        got, err = O.state_density_field(h, R, e, 32)
        std = np.float32(np.sqrt(np.float64(np.float32(np.sum((h[0] - np.float32(1000.0 / 128)) ** 2, dtype=np.float64) / 127))))
        q = want / 2
        assert err[0, 0] == np.float32(R[j] - np.float32(q))
        assert np.isfinite(std)


def test_error_grid():
    rng = np.random.default_rng(5)
    h = _rows(64, 9)
    R = np.sort(rng.random(64).astype(np.float32))
    e = np.zeros_like(h)
    for _ in range(3):
        h, e = O.state_density_field(h, R, e, 8)
        assert np.all(np.abs(e) <= 1.0)
        np.testing.assert_array_equal(e * 128, np.round(e * 128))
