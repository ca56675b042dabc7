"""Density-field state (row f4) on the GPU against the oracle (or_state_df).

dfssm_state_density_field must reproduce the oracle bit for bit (state and sigma-delta error) on
random rows of many scales, constant rows and 1.3B-sized state, for power-of-two and other
threshold counts, with and without sigma-delta, through repeated boundaries; bad arguments are
rejected. End to end, greedy generation with the density-field state (quantization after every
block_len tokens, prompt included) gives the oracle's tokens.
"""
import numpy as np
import pytest
import torch

from df_ssm_inference import DFSSMModel, StateDensityField
from dfssm import _C
from dfssm.synth import config_tiny, make_prompts, make_weights
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _gpu_df(h, R, e, bits):
    hg = torch.from_numpy(h.copy()).to(DEV)
    eg = None if e is None else torch.from_numpy(e.copy()).to(DEV)
    Rg = torch.from_numpy(np.ascontiguousarray(R, np.float32)).to(DEV)
    _C.check(_C.lib().dfssm_state_density_field(hg.data_ptr(), None if eg is None else eg.data_ptr(),
                                                 h.shape[0], 128, Rg.data_ptr(), R.size, bits, _C.stream()),
             "state_density_field")
    torch.cuda.synchronize()
    return hg.cpu().numpy(), None if eg is None else eg.cpu().numpy()


def _rows(n, seed):
    rng = np.random.default_rng(seed)
    scale = 10.0 ** rng.uniform(-6, 3, (n, 1))
    h = (rng.normal(0, 1, (n, 128)) * scale + rng.normal(0, 1, (n, 1)) * scale).astype(np.float32)
    h[0] = 0.0
    h[1] = 3.5
    h[2, ::2] = -1.0
    h[2, 1::2] = 1.0
    h[3, 0] = 1e4
    return h


@pytest.mark.parametrize("kk,sd,bits", [(64, True, 8), (64, False, 8), (16, True, 8), (1000, True, 8),
                                         (64, True, 32), (9, True, 4)])
def test_kernel_vs_oracle(kk, sd, bits):
    print(f"state df kk={kk} sd={sd} bits={bits}", flush=True)
    rng = np.random.default_rng(kk * 7 + bits)
    h = _rows(8192, kk)
    e = np.zeros_like(h) if sd else None
    for it in range(3):
        R = np.sort(rng.random(kk).astype(np.float32))
        ho, eo = O.state_density_field(h, R, e, bits)
        hg, eg = _gpu_df(h, R, e, bits)
        np.testing.assert_array_equal(hg.view(np.uint32), ho.view(np.uint32), err_msg=f"boundary {it}")
        if sd:
            np.testing.assert_array_equal(eg.view(np.uint32), eo.view(np.uint32))
        h, e = ho, eo


def test_full_size_state():
    """The 1.3B state at batch 1 (48 x 64 x 64 rows) in one call."""
    rng = np.random.default_rng(1)
    h = (rng.normal(0, 1, (48 * 64 * 64, 128)) * 10.0 ** rng.uniform(-3, 1, (48 * 64 * 64, 1))).astype(np.float32)
    e = np.zeros_like(h)
    R = np.sort(rng.random(64).astype(np.float32))
    ho, eo = O.state_density_field(h, R, e, 8)
    hg, eg = _gpu_df(h, R, e, 8)
    np.testing.assert_array_equal(hg.view(np.uint32), ho.view(np.uint32))
    np.testing.assert_array_equal(eg.view(np.uint32), eo.view(np.uint32))


def test_rejects_bad_args():
    lib = _C.lib()
    h = torch.zeros(4, 128, device=DEV)
    R = torch.rand(64, device=DEV)
    assert lib.dfssm_state_density_field(h.data_ptr(), None, 4, 64, R.data_ptr(), 64, 8, _C.stream()) == -2
    assert lib.dfssm_state_density_field(h.data_ptr(), None, 4, 128, R.data_ptr(), 0, 8, _C.stream()) == -5
    assert lib.dfssm_state_density_field(h.data_ptr(), None, 4, 128, R.data_ptr(), 1025, 8, _C.stream()) == -5
    assert lib.dfssm_state_density_field(h.data_ptr() + 4, None, 3, 128, R.data_ptr(), 64, 8, _C.stream()) == -4
    assert lib.dfssm_state_density_field(None, None, 4, 128, R.data_ptr(), 64, 8, _C.stream()) == -1


@pytest.mark.parametrize("B,Tp,sd", [(1, 20, True), (3, 70, True), (2, 5, False)])
def test_generate_state_df_vs_oracle(B, Tp, sd):
    w = make_weights(config_tiny(n_layer=2), seed=21)
    df = StateDensityField.random(K=4, num_banks=8, seed=B, block_len=32, sigma_delta=sd)
    prompts = make_prompts(B, w.cfg.vocab_size, Tp)
    n = 80
    print(f"state df generate B={B} Tp={Tp} sd={sd}", flush=True)
    orc = O.OracleModel(w, B)
    err = np.zeros_like(orc.h) if sd else None
    pos = 0

    def boundary():
        nonlocal err
        if pos % df.block_len == 0:
            c = pos // df.block_len - 1
            h2, e2 = O.state_density_field(orc.h.reshape(-1, 128), df.thresholds[c % df.thresholds.shape[0]],
                                           None if err is None else err.reshape(-1, 128), df.sd_bits)
            orc.h[...] = h2.reshape(orc.h.shape)
            if err is not None:
                err = e2.reshape(orc.h.shape)

    for t in range(Tp - 1):
        orc.step(prompts[:, t])
        pos += 1
        boundary()
    tok = prompts[:, -1]
    ref = []
    for i in range(n):
        _, tok = orc.step(tok)
        pos += 1
        boundary()
        ref.append(tok.copy())
    ref = np.stack(ref, 1)
    gpu = DFSSMModel.from_weights(w, device=DEV, batch_size=B)
    got = gpu.generate(n_tokens=n, prompt=torch.from_numpy(prompts), return_tokens=True, verbose=False,
                       state_df=df).cpu().numpy()
    np.testing.assert_array_equal(got, ref)
    gh = gpu.h_state.cpu().numpy()
    print(f"state bit-equal: {np.array_equal(gh.view(np.uint32), orc.h.view(np.uint32))}, "
          f"max rel {np.abs(gh - orc.h).max() / max(np.abs(orc.h).max(), 1e-30):.3e}")
    assert np.abs(gh - orc.h).max() <= 1e-3 * np.abs(orc.h).max()
    assert gpu.error_flag() == 0
