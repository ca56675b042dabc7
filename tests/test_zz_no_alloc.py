"""dfssm_decode_step_static (the decode step whose workspace is the library's static device array,
for callers that cannot allocate) against dfssm_decode_step with a caller-allocated workspace:
from identical states and tokens, logits, greedy tokens, the next-step input x and both states
must be bit-identical, step after step. Two calls in a row with different inputs, the second
smaller (batch 4, then batch 1, then the 1.3B shape at batch 1; at batch >= 5, where the array
also holds the per-workgroup launch counts and tagged words of the fused SSM and out_proj
launches and the batched head's digit planes: batch 17, then 5, then the 1.3B shape at batch
32), so that the array is reused and re-cleared when the dimensions change; the error flag
reported through error_out is 0.
"""
import ctypes

import numpy as np
import pytest
import torch

from df_ssm_inference import DFSSMModel
from dfssm import _C
from dfssm.synth import config_1p3b, config_tiny, make_prompts, make_weights

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _clone_state(m):
    return m.h_state.clone(), m.conv_state.clone(), m.x.clone()


def _run_pair(m: DFSSMModel, steps: int, seed: int):
    """`steps` decode steps through both entry points from the same state; compare every output."""
    lib = _C.lib()
    B, V = m.batch_size, m.cfg.vocab_size
    prompts = make_prompts(B, V, steps, base_seed=seed)
    m.ingest(torch.from_numpy(make_prompts(B, V, 3, base_seed=seed + 7)))  # a non-zero state
    torch.cuda.synchronize()
    h0, c0, x0 = _clone_state(m)
    # twin state tensors for the static path
    h1, c1, x1 = h0.clone(), c0.clone(), x0.clone()
    st1 = _C.State(h1.data_ptr(), c1.data_ptr())
    logits0 = torch.empty_like(m.logits)
    logits1 = torch.empty_like(m.logits)
    next0 = torch.empty(B, dtype=torch.int64, device=DEV)
    next1 = torch.empty(B, dtype=torch.int64, device=DEV)
    err = torch.full((1,), -1, dtype=torch.int32, device=DEV)
    for t in range(steps):
        tok = torch.from_numpy(prompts[:, t]).to(DEV)
        _C.check(lib.dfssm_decode_step(m._model, tok.data_ptr(), m.x.data_ptr(), m._state, m.workspace.data_ptr(),
                                       logits0.data_ptr(), next0.data_ptr(), 1, _C.stream()), "decode_step")
        _C.check(lib.dfssm_decode_step_static(m._model, tok.data_ptr(), x1.data_ptr(), ctypes.byref(st1),
                                              logits1.data_ptr(), next1.data_ptr(), 1, err.data_ptr(),
                                              _C.stream()), "decode_step_static")
        torch.cuda.synchronize()
        assert int(err.item()) == 0, f"step {t}: static path error flag {int(err.item())}"
        assert torch.equal(logits0.view(torch.int16), logits1.view(torch.int16)), f"step {t}: logits differ"
        assert torch.equal(next0, next1), f"step {t}: tokens differ"
        assert torch.equal(m.x.view(torch.int16), x1.view(torch.int16)), f"step {t}: next-step input differs"
        assert torch.equal(m.h_state, h1), f"step {t}: SSM state differs"
        assert torch.equal(m.conv_state.view(torch.int16), c1.view(torch.int16)), f"step {t}: conv state differs"
    assert m.error_flag() == 0


@pytest.fixture(scope="module")
def w13():
    return make_weights(config_1p3b(), seed=0)


def test_static_decode_matches_workspace_decode(w13):
    w = make_weights(config_tiny(n_layer=3), seed=0)
    print("static decode: tiny model, batch 4", flush=True)
    _run_pair(DFSSMModel.from_weights(w, device=DEV, batch_size=4), steps=5, seed=3000)
    print("static decode: tiny model, batch 1 (smaller, after batch 4)", flush=True)
    _run_pair(DFSSMModel.from_weights(w, device=DEV, batch_size=1), steps=5, seed=3100)
    print("static decode: 1.3B shape, batch 1", flush=True)
    _run_pair(DFSSMModel.from_weights(w13, device=DEV, batch_size=1), steps=3, seed=3200)


def test_static_decode_batched_launches(w13):
    w = make_weights(config_tiny(n_layer=3), seed=1)
    print("static decode: tiny model, batch 17", flush=True)
    _run_pair(DFSSMModel.from_weights(w, device=DEV, batch_size=17), steps=4, seed=3300)
    print("static decode: tiny model, batch 5 (smaller, after batch 17)", flush=True)
    _run_pair(DFSSMModel.from_weights(w, device=DEV, batch_size=5), steps=4, seed=3400)
    print("static decode: 1.3B shape, batch 32", flush=True)
    _run_pair(DFSSMModel.from_weights(w13, device=DEV, batch_size=32), steps=3, seed=3500)


def test_static_decode_rejects_oversized_dims():
    """Dimensions whose workspace exceeds the static array are refused before any launch."""
    w = make_weights(config_tiny(n_layer=1), seed=0)
    m = DFSSMModel.from_weights(w, device=DEV, batch_size=1)
    big = _C.Dims(*[getattr(m.dims, f) for f, _ in _C.Dims._fields_])
    big.batch, big.d_model, big.d_inner, big.nheads, big.vocab_size = 64, 5120, 5120, 80, 65536
    assert _C.lib().dfssm_workspace_bytes(big) > (24 << 20)
    model = _C.Model(big, m._descs, m.embedding_tiled.data_ptr(), m.embedding_scale.data_ptr(),
                     m.norm_f_weight.data_ptr())
    rc = _C.lib().dfssm_decode_step_static(model, None, m.x.data_ptr(), m._state, None, m._next.data_ptr(), 0,
                                           None, _C.stream())
    assert rc == -6, rc
    assert "static workspace" in _C.lib().dfssm_error_string(rc).decode()
