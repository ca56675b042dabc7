"""The drop-in's API behaviour on the GPU, as the reference's callers use it.

- The reference's decode loop (inference/gpu/df_ssm_inference.py:234-236:
  `logits = self.forward(tokens); tokens = logits.argmax(dim=-1)`) on device token ids runs without
  a host synchronization per step -- torch's sync debug mode raises on any -- and yields the
  oracle's greedy tokens.
- A device token id out of range does not raise inside forward() (that would need a host
  round trip); it sets ERR_TOKEN_RANGE, which check_errors() reports.
- The reference's LayerWeights attributes (:32-44, built at :70-98): in_w_T / out_w_T (the +-1
  matrices, pre-transposed) and the fp16-dequantized LoRA factors, against the file's contents.
"""
import numpy as np
import pytest
import torch

import df_ssm_inference as dfi
from df_ssm_inference import DFSSMModel
from dfssm import _C
from dfssm.format import unpack_sign_bits
from dfssm.synth import config_tiny, make_weights
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def tiny_weights():
    return make_weights(config_tiny(n_layer=3), seed=3)


@pytest.mark.parametrize("B", [1, 2, 8])
def test_reference_loop_no_sync(tiny_weights, B):
    w = tiny_weights
    print(f"reference decode loop B={B}", flush=True)
    gpu = DFSSMModel.from_weights(w, device=DEV, batch_size=B)
    tokens = torch.zeros(B, dtype=torch.long, device=DEV)
    gpu.forward(tokens)  # the first call captures the graph (a capture synchronizes)
    gpu.reset_state()
    torch.cuda.synchronize()
    seen = []
    torch.cuda.set_sync_debug_mode("error")
    try:
        for _ in range(32):
            logits = gpu.forward(tokens)
            tokens = logits.argmax(dim=-1)
            seen.append(tokens)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    got = torch.stack(seen, 1).cpu().numpy()
    orc = O.OracleModel(w, B)
    tok = np.zeros(B, np.int64)
    ref = []
    for _ in range(32):
        _, tok = orc.step(tok)
        ref.append(tok)
    np.testing.assert_array_equal(got, np.stack(ref, 1))
    gpu.check_errors()


def test_device_token_out_of_range_is_deferred(tiny_weights):
    gpu = DFSSMModel.from_weights(tiny_weights, device=DEV, batch_size=2)
    V = tiny_weights.cfg.vocab_size
    gpu.forward(torch.tensor([1, 2], device=DEV))
    gpu.check_errors()
    gpu.forward(torch.tensor([V, 2], device=DEV))  # no exception here
    assert gpu.error_flag() & dfi.ERR_TOKEN_RANGE
    with pytest.raises(_C.DFSSMError, match="out of range"):
        gpu.check_errors()
    assert gpu.error_flag() == 0  # cleared by check_errors
    with pytest.raises(IndexError):  # host ids are still checked before anything is launched
        gpu.forward(torch.tensor([V, 2]))


def test_reference_layer_attributes(tiny_weights):
    w = tiny_weights
    c = w.cfg
    gpu = DFSSMModel.from_weights(w, device=DEV, batch_size=1)
    for li in (0, c.n_layer - 1):
        L, lw = w.layers[li], gpu.layers[li]
        in_w = unpack_sign_bits(L["in_packed"])     # (IPO, D)
        out_w = unpack_sign_bits(L["out_packed"])   # (D, DI)
        assert lw.in_w_T.dtype == torch.int8 and lw.in_w_T.shape == (c.d_model, c.in_proj_out)
        assert lw.out_w_T.shape == (c.d_inner, c.d_model)
        np.testing.assert_array_equal(lw.in_w_T.cpu().numpy(), in_w.T)
        np.testing.assert_array_equal(lw.out_w_T.cpu().numpy(), out_w.T)

        def deq(a, s):  # the reference's (A.float() * A_s.float().unsqueeze(1)).half()
            return (torch.from_numpy(a).float() * torch.from_numpy(s.astype(np.float32))[:, None]).half()

        for name, a, s in (("in_lora_A", "in_lA", "in_lA_s"), ("in_lora_B", "in_lB", "in_lB_s"),
                           ("out_lora_A", "out_lA", "out_lA_s"), ("out_lora_B", "out_lB", "out_lB_s")):
            got = getattr(lw, name)
            assert got.dtype == torch.float16 and got.device.type == "cuda"
            want = deq(L[a], L[s])
            assert got.shape == want.shape, name
            assert torch.equal(got.cpu().view(torch.int16), want.view(torch.int16)), name
        assert lw.in_w_T is lw.in_w_T  # built once
