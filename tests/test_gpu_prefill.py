"""Prompt prefill (dfssm_prefill) against step-by-step ingestion and the oracle.

The layer-major prefill must give, bit for bit, what T decode steps give: the fp32 SSM state,
the conv state, the residual row handed to the next step, the greedy token and the logits of the
last prompt token. Covered: batch 1 (one-launch decode layer) and >= 5 (matrix-core path),
prompt lengths below, at and across the kernel's 16-token staging rounds, prompts split into
several chunks, head dimensions 16 / 32 / 64 (one, two and four 16-row state blocks per scan
workgroup), the 1.3B shape and the 2.7B layer shapes.
"""
import numpy as np
import pytest
import torch

from df_ssm_inference import DFSSMModel
from dfssm.format import DFSSMConfig
from dfssm.synth import config_1p3b, config_tiny, make_prompts, make_weights
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _twins(w, B):
    return (DFSSMModel.from_weights(w, device=DEV, batch_size=B),
            DFSSMModel.from_weights(w, device=DEV, batch_size=B))


def _assert_same(a: DFSSMModel, b: DFSSMModel, la, lb):
    torch.cuda.synchronize()
    assert torch.equal(a.h_state, b.h_state), "SSM state differs"
    assert torch.equal(a.conv_state.view(torch.int16), b.conv_state.view(torch.int16)), "conv state differs"
    assert torch.equal(a.x.view(torch.int16), b.x.view(torch.int16)), "next-step input differs"
    assert torch.equal(a._next, b._next), "greedy token differs"
    if la is not None:
        assert torch.equal(la.view(torch.int16), lb.view(torch.int16)), "logits differ"
    assert a.error_flag() == 0 and b.error_flag() == 0


def _prefill_vs_steps(w, B, T, max_rows=None, steps_first=0):
    prompts = torch.from_numpy(make_prompts(B, w.cfg.vocab_size, T + steps_first))
    pf, st = _twins(w, B)
    if max_rows is not None:
        pf.PREFILL_MAX_ROWS = max_rows
    if steps_first:  # a state that is not zero when the prefill starts
        pf.ingest(prompts[:, :steps_first], step_by_step=True)
        st.ingest(prompts[:, :steps_first], step_by_step=True)
    lp = pf.prefill(prompts[:, steps_first:], want_logits=True)
    if T > 1:
        st.ingest(prompts[:, steps_first:-1], step_by_step=True)
    # the last prompt token through forward(): logits, greedy token and its embedding in x
    ls = st.forward(prompts[:, -1].to(DEV))
    _assert_same(pf, st, lp, ls)
    # continuing from both: the same greedy tokens
    gp = pf.decode(5)
    gs = st.decode(5)
    assert torch.equal(gp, gs)


@pytest.fixture(scope="module")
def tiny_weights():
    return make_weights(config_tiny(n_layer=3), seed=0)


@pytest.mark.parametrize("B,T", [(1, 1), (1, 17), (3, 40), (5, 16), (16, 9), (64, 3), (5, 61), (64, 9)])
def test_prefill_equals_steps_tiny(tiny_weights, B, T):
    print(f"prefill tiny B={B} T={T}", flush=True)
    _prefill_vs_steps(tiny_weights, B, T)


@pytest.mark.parametrize("B,T,rows", [(2, 37, 2 * 5), (8, 20, 8 * 7), (5, 33, 5 * 16)])
def test_prefill_chunks(tiny_weights, B, T, rows):
    """Prompts longer than one chunk (chunks of rows / B tokens), from a non-zero state."""
    print(f"prefill chunks B={B} T={T} rows={rows}", flush=True)
    _prefill_vs_steps(tiny_weights, B, T, max_rows=rows, steps_first=3)


@pytest.mark.parametrize("nheads,headdim", [(32, 32), (64, 16)])
def test_prefill_headdims(nheads, headdim):
    """Head dimensions 32 and 16 (two and one 16-row state blocks per scan workgroup), against
    step-by-step ingestion and the oracle's greedy tokens."""
    c = DFSSMConfig(n_layer=2, d_model=512, d_inner=1024, d_state=128, nheads=nheads, headdim=headdim,
                    ngroups=1, vocab_size=1000, kw=4)
    w = make_weights(c, seed=7)
    print(f"prefill heads {nheads} x {headdim}", flush=True)
    _prefill_vs_steps(w, 6, 21)
    B, T, n = 6, 21, 4
    prompts = make_prompts(B, c.vocab_size, T)
    ref, _ = O.OracleModel(w, B).generate(prompts, n)
    gpu = DFSSMModel.from_weights(w, device=DEV, batch_size=B)
    got = gpu.generate(n_tokens=n, prompt=torch.from_numpy(prompts), return_tokens=True, verbose=False)
    np.testing.assert_array_equal(got.cpu().numpy(), ref)


def test_prefill_1p3b():
    """1.3B shape, batch 4, 32-token prompts: prefill == 32 decode steps."""
    w = make_weights(config_1p3b(), seed=0)
    print("prefill 1.3B B=4 T=32", flush=True)
    _prefill_vs_steps(w, 4, 32)


def test_prefill_2p7b_layer_shapes():
    """Config 4's layer shapes (d_model 2560, d_inner 5120, 80 heads) at batch 64, 4 layers."""
    c = DFSSMConfig(n_layer=4, d_model=2560, d_inner=5120, d_state=128, nheads=80, headdim=64, ngroups=1,
                    vocab_size=4096, kw=4)
    w = make_weights(c, seed=5)
    print("prefill 2.7B layers B=64 T=20", flush=True)
    _prefill_vs_steps(w, 64, 20)


def test_prefill_rejects_bad_prompts(tiny_weights):
    gpu = DFSSMModel.from_weights(tiny_weights, device=DEV, batch_size=2)
    with pytest.raises(ValueError):
        gpu.prefill(torch.zeros(3, 4, dtype=torch.int64))
    with pytest.raises(IndexError):
        gpu.prefill(torch.full((2, 4), tiny_weights.cfg.vocab_size, dtype=torch.int64))
