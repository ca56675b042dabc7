"""Host-side logic of the drop-in API, checked without a GPU: the one-launch layer's residency
rule (dfssm_one_launch_plan), the decoding of the workspace error flag, and token range checks that
must fire before any kernel reads the ids."""
import numpy as np
import pytest
import torch

from dfssm import _C
from dfssm.synth import config_tiny
import df_ssm_inference as dfi


def _dims(**kw):
    base = dict(n_layer=48, d_model=2048, d_inner=4096, d_state=128, nheads=64, headdim=64, ngroups=1,
                vocab_size=50288, batch=1, emb_code=1)
    base.update(kw)
    return _C.Dims(*[base[f] for f, _ in _C.Dims._fields_])


@pytest.mark.parametrize("kw,cus,per_cu,grid", [
    ({}, 256, 1, 256),                 # MI355X: one 1024-thread workgroup per CU
    ({}, 256, 2, 256),
    ({}, 256, 0, 0),                   # the instantiation does not fit a CU: five kernels
    ({"batch": 4}, 256, 1, 256),
    ({"batch": 5}, 256, 1, 0),         # batch >= 5 always runs five kernels
    ({}, 140, 1, 0),                   # 133 in_proj groups + 16 LoRA workgroups do not fit
    ({}, 2048, 1, 256),                # item-organised layer: one workgroup per SSM item
    ({"d_model": 2560, "d_inner": 5120, "nheads": 80}, 256, 1, 256),
    ({"batch": 65}, 256, 1, 0),
])
def test_one_launch_plan(kw, cus, per_cu, grid):
    assert _C.lib().dfssm_one_launch_plan(_dims(**kw), cus, per_cu) == grid


@pytest.mark.parametrize("kw,cus,per_cu,grid", [
    ({}, 256, 1, 256),                 # 1.3B shape on MI355X: 8 XCDs x 32 CUs
    ({"batch": 4}, 256, 1, 256),
    ({}, 256, 0, 0),                   # the instantiation does not fit a CU
    ({}, 304, 1, 0),                   # not 8 x 32 CUs
    ({"batch": 5}, 256, 1, 0),         # batch >= 5: five kernels
    ({"d_model": 2560, "d_inner": 5120, "nheads": 80}, 256, 1, 256),   # 2.7B: 26 phase-A groups per XCD
    ({"d_model": 512, "d_inner": 1024, "nheads": 16}, 256, 1, 256),    # the tests' tiny model
    ({"d_model": 4096, "d_inner": 4096}, 256, 1, 256),                 # 16 out_proj groups per XCD
    ({"d_model": 512, "d_inner": 1024, "nheads": 32}, 256, 1, 256),    # 4 heads x 32 rows per XCD: 2 row groups
    ({"d_model": 5120, "d_inner": 5120, "nheads": 80}, 256, 1, 256),   # 20 out_proj groups = 2 x 10 z groups
    ({"d_model": 4096, "d_inner": 2048, "nheads": 32}, 256, 1, 0),     # 16 out_proj groups > 2 x 4 z groups
])
def test_xcd_layer_plan(kw, cus, per_cu, grid):
    assert _C.lib().dfssm_xcd_layer_plan(_dims(**kw), cus, per_cu) == grid


def test_describe_error_flag():
    assert dfi.describe_error_flag(0) == ""
    assert "token id out of range" in dfi.describe_error_flag(dfi.ERR_TOKEN_RANGE)
    assert "timed out" in dfi.describe_error_flag(dfi.ERR_WAIT_TIMEOUT)
    both = dfi.describe_error_flag(dfi.ERR_TOKEN_RANGE | dfi.ERR_WAIT_TIMEOUT | 16)
    assert "out of range" in both and "timed out" in both and "0x10" in both


def _hostless_model(B=2):
    """A DFSSMModel shell with no device state: any kernel launch or device access would fail
    with AttributeError, so a test that expects IndexError shows the check ran first."""
    m = dfi.DFSSMModel.__new__(dfi.DFSSMModel)
    m.batch_size = B
    m.cfg = config_tiny(n_layer=1)
    return m


@pytest.mark.parametrize("bad", [-1, "V"])
def test_generate_checks_prompt_range_before_launch(bad):
    m = _hostless_model()
    V = m.cfg.vocab_size
    tok = V if bad == "V" else bad
    prompt = torch.tensor([[1, 2], [3, tok]])
    with pytest.raises(IndexError):
        m.generate(n_tokens=4, prompt=prompt, verbose=False)
    with pytest.raises(IndexError):
        m.generate(n_tokens=4, prompt=prompt, temperature=0.7, verbose=False)
    with pytest.raises(IndexError):
        m.ingest(prompt)
    with pytest.raises(IndexError):
        m.prefill(prompt)
    with pytest.raises(IndexError):
        m.forward(torch.tensor([0, tok]))


def test_generate_checks_prompt_shape():
    m = _hostless_model(B=2)
    with pytest.raises(ValueError):
        m.generate(n_tokens=4, prompt=torch.zeros(3, 2, dtype=torch.int64), verbose=False)
