"""Pins of the oracle's sampling definition (or_sample), CPU only.

The sampler replaces torch.sort / cumsum / multinomial (eval/gen_test.py:54-95,
training/df_ssm_mamba2_distill_dfw.py:1066-1078) with a deterministic definition; these checks
tie that definition to the reference's rules:
  * top_p = 0 keeps only the most probable token: the draw is the argmax of the penalized logits;
  * the two penalty orders against their closed forms (seen tokens divided by r after the
    temperature; per occurrence, positive / r and others * r, before it);
  * the kept set against a float64 NumPy evaluation of the reference's drop rule
    `(cumsum(sorted p) - p) > top_p`, on logits whose probability masses are far from the cut;
  * the draw frequencies against softmax over the kept set (chi-square), and the inverse-CDF
    draw against a Python-integer restatement.
"""
import numpy as np
import pytest

from oracle import oracle as O


def _draw(logits, counts=None, T=1.0, top_p=1.0, r=1.0, mode=0, seed=0, steps=1, want_kept=False):
    lg = np.ascontiguousarray(np.atleast_2d(logits).astype(np.float16))
    M, V = lg.shape
    cn = np.zeros((M, V), np.int32) if counts is None else np.ascontiguousarray(counts, np.int32).reshape(M, V).copy()
    st = np.zeros(M, np.uint32)
    out = []
    kept = None
    for _ in range(steps):
        res = O.sample(lg, cn, st, T, top_p, r, mode, seed, want_kept=want_kept)
        if want_kept:
            res, kept = res
        out.append(res.copy())
    return np.stack(out, 1), cn, st, kept


def test_top_p_zero_is_argmax():
    rng = np.random.default_rng(0)
    lg = rng.normal(0, 3, (4, 3000)).astype(np.float16)
    toks, cn, st, _ = _draw(lg, top_p=0.0, steps=3, T=0.7)
    np.testing.assert_array_equal(toks[:, 0], lg.astype(np.float32).argmax(axis=1))
    # every draw of the same logits repeats it, and the counts / steps advance
    assert (toks == toks[:, :1]).all()
    assert (st == 3).all() and (cn.sum(axis=1) == 3).all()
    # first index on ties
    tie = np.zeros((1, 64), np.float16)
    tie[0, [5, 9, 40]] = 2.0
    assert _draw(tie, top_p=0.0)[0][0, 0] == 5


def test_penalty_orders():
    # mode 0 (gen_test): z = (l / T) / r for seen tokens: 2/1.2 = 1.67 < 1.9 -> token 1
    lg = np.array([[2.0, 1.9, -5.0, -5.0]], np.float16)
    cnt = np.array([[1, 0, 0, 0]], np.int32)
    assert _draw(lg, cnt, top_p=0.0, r=1.2, mode=0)[0][0, 0] == 1
    assert _draw(lg, cnt, top_p=0.0, r=1.0, mode=0)[0][0, 0] == 0
    # negative logits: mode 0 divides (-1 / 1.2 = -0.83 > -0.9 -> token 0 wins),
    # mode 1 multiplies (-1 * 1.2 = -1.2 < -1.1 -> token 1 wins)
    lg = np.array([[-1.0, -0.9, -5.0, -5.0]], np.float16)
    lg[0, 1] = -1.1
    assert _draw(lg, cnt, top_p=0.0, r=1.2, mode=0)[0][0, 0] == 0
    assert _draw(lg, cnt, top_p=0.0, r=1.2, mode=1)[0][0, 0] == 1
    # mode 1 applies once per occurrence: 3 occurrences -> 3 / 1.2^3 = 1.74 < 1.8
    lg = np.array([[3.0, 1.8, -5.0, -5.0]], np.float16)
    assert _draw(lg, np.array([[2, 0, 0, 0]]), top_p=0.0, r=1.2, mode=1)[0][0, 0] == 0
    assert _draw(lg, np.array([[3, 0, 0, 0]]), top_p=0.0, r=1.2, mode=1)[0][0, 0] == 1


def _reference_kept(lg32, T, top_p):
    """gen_test.py:76-80 in float64: sort descending, drop when cumsum - p > top_p."""
    z = lg32.astype(np.float64) / T
    p = np.exp(z - z.max())
    p /= p.sum()
    order = np.argsort(-p, kind="stable")
    sp = p[order]
    drop = (np.cumsum(sp) - sp) > top_p
    kept = np.zeros(lg32.shape[0], bool)
    kept[order[~drop]] = True
    return kept, np.cumsum(sp) - sp


@pytest.mark.parametrize("top_p", [0.3, 0.6, 0.9, 0.99])
def test_kept_set_matches_reference_rule(top_p):
    rng = np.random.default_rng(int(top_p * 100))
    checked = 0
    for trial in range(60):
        lg = rng.normal(0, 2.5, 2000).astype(np.float16)
        kept_ref, excl = _reference_kept(lg.astype(np.float32), 0.8, top_p)
        # only logits whose cut is clear by far more than the fp32 exp / 2^-40 rounding
        if np.min(np.abs(excl - top_p)) < 1e-5:
            continue
        _, _, _, kept = _draw(lg[None], T=0.8, top_p=top_p, want_kept=True)
        np.testing.assert_array_equal(kept[0], kept_ref)
        checked += 1
    assert checked >= 20


def test_draw_frequencies():
    lg = np.array([[1.0, 0.5, 0.0, -0.5, 2.0, -3.0, 1.5, 0.25]], np.float16)
    n = 4000
    for top_p in (1.0, 0.7):
        toks, _, _, kept = _draw(lg, top_p=top_p, steps=n, seed=123, want_kept=True)
        k = kept[0]
        p = np.exp(lg[0].astype(np.float64))
        p = np.where(k, p, 0.0)
        p /= p.sum()
        freq = np.bincount(toks[0], minlength=8)
        assert freq[~k].sum() == 0
        exp = n * p[k]
        chi2 = ((freq[k] - exp) ** 2 / exp).sum()
        # chi-square with (kept - 1) degrees of freedom; 0.999 quantile of df <= 7 is < 25
        assert chi2 < 25, (top_p, freq, exp)
    # other seeds give other streams
    a = _draw(lg, steps=50, seed=1)[0]
    b = _draw(lg, steps=50, seed=2)[0]
    assert (a != b).any()


def _splitmix64(x):
    m = (1 << 64) - 1
    x = (x + 0x9E3779B97F4A7C15) & m
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & m
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & m
    return x ^ (x >> 31)


def test_inverse_cdf_draw():
    """The draw restated in Python integers: R = floor(h S / 2^64) with h = splitmix64 of
    (seed, sequence, step), the first kept index (index order) whose cumulative kept mass E
    exceeds R; masses E = floor(exp(z - max) 2^40) from the oracle's exp."""
    from oracle import oracle as OO
    rng = np.random.default_rng(9)
    lg = rng.normal(0, 2, (2, 300)).astype(np.float16)
    seed = 987654321
    toks, _, _, kept = _draw(lg, top_p=0.8, seed=seed, want_kept=True, T=0.9)
    for b in range(2):
        z = lg[b].astype(np.float32) / np.float32(0.9)
        e = OO.lib()  # the oracle's own exp, element by element
        import ctypes
        f = e.or_expf
        f.argtypes = [ctypes.c_float]
        f.restype = ctypes.c_float
        m = z.max()
        E = [int(np.float32(f(float(np.float32(zi - m)))) * np.float32(2.0 ** 40)) for zi in z]
        S = sum(E[i] for i in range(300) if kept[b, i])
        h = _splitmix64(seed ^ ((b << 40) | (0 << 17) | 0x1FFFF))
        R = (h * S) >> 64
        acc, tok = 0, None
        for i in range(300):
            if kept[b, i]:
                acc += E[i]
                if acc > R:
                    tok = i
                    break
        assert toks[b, 0] == tok
