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
    ({}, 2048, 1, 1024),               # one workgroup per CU, at most 1024
    ({"d_model": 2560, "d_inner": 5120, "nheads": 80}, 256, 1, 256),
    ({"batch": 65}, 256, 1, 0),
])
def test_one_launch_plan(kw, cus, per_cu, grid):
    assert _C.lib().dfssm_one_launch_plan(_dims(**kw), cus, per_cu) == grid


def test_describe_error_flag():
    """Every bit names its own source (the launch whose bounded wait gave up), as include/dfssm.h
    defines them."""
    assert dfi.describe_error_flag(0) == ""
    assert (dfi.ERR_TOKEN_RANGE, dfi.ERR_WAIT_LAYER, dfi.ERR_WAIT_SSM_PROLOGUE, dfi.ERR_WAIT_OUT_PROLOGUE) == \
        (1, 4, 8, 16)
    assert "token id out of range" in dfi.describe_error_flag(dfi.ERR_TOKEN_RANGE)
    layer = dfi.describe_error_flag(dfi.ERR_WAIT_LAYER)
    ssm = dfi.describe_error_flag(dfi.ERR_WAIT_SSM_PROLOGUE)
    out = dfi.describe_error_flag(dfi.ERR_WAIT_OUT_PROLOGUE)
    assert "one-launch layer" in layer and "timed out" in layer
    assert "SSM" in ssm and "timed out" in ssm and "one-launch" not in ssm
    assert "out_proj" in out and "timed out" in out and "one-launch" not in out
    assert len({layer, ssm, out}) == 3
    every = dfi.describe_error_flag(1 | 4 | 8 | 16 | 64)
    assert all(x in every for x in ("out of range", layer, ssm, out, "0x40"))


def test_error_bits_match_header():
    """The Python constants are the C header's DFSSM_ERR_* values."""
    import os
    import re
    hdr = open(os.path.join(os.path.dirname(__file__), "..", "include", "dfssm.h")).read()
    vals = dict(re.findall(r"#define DFSSM_ERR_(\w+) (\d+)", hdr))
    assert {k: int(v) for k, v in vals.items()} == {
        "TOKEN_RANGE": dfi.ERR_TOKEN_RANGE, "WAIT_LAYER": dfi.ERR_WAIT_LAYER,
        "WAIT_SSM_PROLOGUE": dfi.ERR_WAIT_SSM_PROLOGUE, "WAIT_OUT_PROLOGUE": dfi.ERR_WAIT_OUT_PROLOGUE}


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
