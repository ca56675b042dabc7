"""Sampling head (dfssm_sample) on the GPU against the oracle's definition (or_sample).

The draw is deterministic for a seed, so the GPU must reproduce the oracle's tokens, occurrence
counts and step counters exactly: per kernel call on random logits (vocabularies from 7 to the
largest, 65536, every parameter combination, several steps) and end to end (sampled generation of a tiny
model against the oracle's decode step followed by or_sample). top_p = 0 must give the greedy
tokens.
"""
import ctypes

import numpy as np
import pytest
import torch

from df_ssm_inference import DFSSMModel
from dfssm import _C
from dfssm.format import DFSSMConfig
from dfssm.synth import config_tiny, make_prompts, make_weights
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

PARAMS = [(0.7, 0.9, 1.2, 0), (1.3, 0.5, 1.0, 1), (1.0, 1.0, 1.0, 0), (0.8, 0.0, 1.2, 1), (0.6, 0.95, 1.5, 1)]


def _model(V, B):
    c = DFSSMConfig(n_layer=1, d_model=512, d_inner=1024, d_state=128, nheads=16, headdim=64, ngroups=1,
                    vocab_size=V, kw=4)
    return DFSSMModel.from_weights(make_weights(c, seed=3), device=DEV, batch_size=B)


# V = 7: one slice workgroup; 513: two ragged slices; 65536: the largest vocabulary (64 slices of
# 1024 tokens); B = 32: a decode batch
@pytest.mark.parametrize("V,B", [(7, 2), (513, 3), (1000, 1), (1000, 5), (50288, 3), (50288, 32), (65536, 2)])
def test_sample_kernel_vs_oracle(V, B):
    print(f"sampler V={V} B={B}", flush=True)
    m = _model(V, B)
    rng = np.random.default_rng(V + B)
    for (T, top_p, r, mode) in PARAMS:
        seed = int(rng.integers(0, 2**62))
        counts = rng.integers(0, 3, (B, V)).astype(np.int32) * (rng.random((B, V)) < 0.01)
        counts = np.ascontiguousarray(counts, np.int32)
        step = np.zeros(B, np.uint32)
        cg = torch.from_numpy(counts.copy()).to(DEV)
        sg = torch.zeros(B, dtype=torch.int32, device=DEV)
        nxt = torch.zeros(B, dtype=torch.int64, device=DEV)
        p = _C.SampleParams(T, top_p, r, mode, seed)
        for it in range(4):
            lg = (rng.normal(0, 3, (B, V))).astype(np.float16)
            lgd = torch.from_numpy(lg.view(np.int16)).to(DEV)
            _C.check(_C.lib().dfssm_sample(m._model, lgd.data_ptr(), cg.data_ptr(), sg.data_ptr(), ctypes.byref(p),
                                           nxt.data_ptr(), None, m.workspace.data_ptr(), _C.stream()), "sample")
            ref = O.sample(lg, counts, step, T, top_p, r, mode, seed)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(nxt.cpu().numpy(), ref, err_msg=f"{(T, top_p, r, mode)} step {it}")
            np.testing.assert_array_equal(cg.cpu().numpy(), counts)
            np.testing.assert_array_equal(sg.cpu().numpy().view(np.uint32), step)


def _oracle_sampled(w, prompts, n, T, top_p, r, mode, seed):
    B, Tp = prompts.shape
    orc = O.OracleModel(w, B)
    V = w.cfg.vocab_size
    counts = np.zeros((B, V), np.int32)
    for b in range(B):
        np.add.at(counts[b], prompts[b], 1)
    step = np.zeros(B, np.uint32)
    for t in range(Tp - 1):
        orc.step(prompts[:, t])
    tok = prompts[:, -1]
    out = []
    for _ in range(n):
        logits, _ = orc.step(tok)
        tok = O.sample(np.ascontiguousarray(logits), counts, step, T, top_p, r, mode, seed)
        out.append(tok.copy())
    return np.stack(out, 1)


@pytest.mark.parametrize("B,mode", [(1, 0), (3, 1), (6, 0)])
def test_generate_sampled_vs_oracle(B, mode):
    w = make_weights(config_tiny(n_layer=2), seed=11)
    prompts = make_prompts(B, w.cfg.vocab_size, 5)
    T, top_p, r, seed, n = 0.8, 0.9, 1.2, 77, 12
    print(f"sampled generate B={B} mode={mode}", flush=True)
    ref = _oracle_sampled(w, prompts, n, T, top_p, r, mode, seed)
    gpu = DFSSMModel.from_weights(w, device=DEV, batch_size=B)
    got = gpu.generate(n_tokens=n, prompt=torch.from_numpy(prompts), return_tokens=True, verbose=False,
                       temperature=T, top_p=top_p, repetition_penalty=r, penalty_mode=mode, seed=seed)
    np.testing.assert_array_equal(got.cpu().numpy(), ref)
    # the same call again (graphs reused, counts and counters reset) gives the same tokens
    again = gpu.generate(n_tokens=n, prompt=torch.from_numpy(prompts), return_tokens=True, verbose=False,
                         temperature=T, top_p=top_p, repetition_penalty=r, penalty_mode=mode, seed=seed)
    assert torch.equal(got, again)
    assert gpu.error_flag() == 0


def test_top_p_zero_is_greedy():
    w = make_weights(config_tiny(n_layer=2), seed=12)
    B = 4
    prompts = torch.from_numpy(make_prompts(B, w.cfg.vocab_size, 4))
    gpu = DFSSMModel.from_weights(w, device=DEV, batch_size=B)
    greedy = gpu.generate(n_tokens=10, prompt=prompts, return_tokens=True, verbose=False)
    samp = gpu.generate(n_tokens=10, prompt=prompts, return_tokens=True, verbose=False, temperature=1.0, top_p=0.0)
    assert torch.equal(greedy, samp)


def test_sample_rejects_bad_params():
    m = _model(1000, 1)
    lg = torch.zeros(1, 1000, dtype=torch.float16, device=DEV)
    cg = torch.zeros(1, 1000, dtype=torch.int32, device=DEV)
    sg = torch.zeros(1, dtype=torch.int32, device=DEV)
    nxt = torch.zeros(1, dtype=torch.int64, device=DEV)
    for bad in (_C.SampleParams(0.0, 0.9, 1.0, 0, 1), _C.SampleParams(1.0, -0.1, 1.0, 0, 1),
                _C.SampleParams(1.0, 0.9, 0.0, 0, 1), _C.SampleParams(1.0, 0.9, 1.0, 2, 1)):
        rc = _C.lib().dfssm_sample(m._model, lg.data_ptr(), cg.data_ptr(), sg.data_ptr(), ctypes.byref(bad),
                                   nxt.data_ptr(), None, m.workspace.data_ptr(), _C.stream())
        assert rc == -5
