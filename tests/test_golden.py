"""The oracle against fixtures written by the reference's own compiled CPU kernels
(tests/golden/make_golden.py); runs where the reference itself cannot be built or run."""
import os
import sys

import numpy as np

from oracle import oracle as O

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_golden as G  # noqa: E402

from dfssm.synth import make_prompts, make_weights  # noqa: E402

FIX = np.load(G.OUT)


def test_int32_accumulators_match_reference_fixture():
    bits, _, q = G.scaffold_case()
    acc = O.scaffold_acc(bits, q[None, :])[0]
    assert np.array_equal(acc, FIX["acc_in"])


def test_cpu_numerics_decode_matches_reference_fixture():
    w = make_weights(G.golden_config(), seed=11)
    prompt = make_prompts(1, w.cfg.vocab_size, 8)[0]
    assert np.array_equal(prompt, FIX["prompt"])
    m = O.OracleCPUModel(w)
    for i, t in enumerate(prompt):
        lo, _ = m.step(int(t))
        lr = FIX["logits"][i]
        assert np.abs(lo - lr).max() <= 1e-5 * np.abs(lr).max()
        assert int(np.argmax(lo)) == int(np.argmax(lr))
    h = m.h.astype(np.float64)
    np.testing.assert_allclose(h.sum(axis=(2, 3)), FIX["h_sum"], rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose((h * h).sum(axis=(2, 3)), FIX["h_sq"], rtol=1e-5)
    c = m.conv.astype(np.float64)
    np.testing.assert_allclose(c.sum(axis=(1, 2)), FIX["conv_sum"], rtol=1e-5, atol=1e-3)
    np.testing.assert_allclose((c * c).sum(axis=(1, 2)), FIX["conv_sq"], rtol=1e-5)
