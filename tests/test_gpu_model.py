"""End-to-end GPU decode parity against the oracle on seeded random-init models.

Per step: fp16 logits identical to the oracle's on the int8 table (the north star allows 2e-2
absolute), identical greedy tokens; after the run the fp32 SSM state within 1e-3 max relative
error and the conv state close.
"""
import numpy as np
import pytest
import torch

from df_ssm_inference import DFSSMModel
from dfssm.synth import config_1p3b, config_tiny, make_prompts, make_weights
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _np16(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.float16)


def _state_rel(gpu: DFSSMModel, orc: O.OracleModel):
    gh = gpu.h_state.cpu().numpy()
    return np.abs(gh - orc.h).max() / np.abs(orc.h).max()


@pytest.fixture(scope="module")
def tiny_weights():
    return make_weights(config_tiny(n_layer=3), seed=0)


@pytest.mark.parametrize("B", [1, 2, 3, 4, 5, 16, 32, 40, 64])
def test_tiny_forward_stepwise(tiny_weights, B):
    w = tiny_weights
    print(f"tiny forward B={B}", flush=True)
    gpu = DFSSMModel.from_weights(w, device=DEV, batch_size=B)
    orc = O.OracleModel(w, B)
    prompts = make_prompts(B, w.cfg.vocab_size, 6)
    tok = prompts[:, 0]
    worst = 0.0
    for t in range(24):
        logits_g = _np16(gpu.forward(torch.from_numpy(tok).to(DEV))).astype(np.float32)
        logits_o, nxt = orc.step(tok)
        err = np.abs(logits_g - logits_o.astype(np.float32)).max()
        worst = max(worst, err)
        assert err == 0.0, f"step {t}: logits differ by {err}"  # the exact int8 head, every batch
        g_next = logits_g.argmax(axis=1)
        np.testing.assert_array_equal(g_next, nxt)
        tok = prompts[:, t + 1] if t + 1 < prompts.shape[1] else nxt
    rel = _state_rel(gpu, orc)
    print(f"B={B} worst logit err {worst:.3e} state rel {rel:.3e}")
    assert gpu.error_flag() == 0
    assert rel <= 1e-3
    np.testing.assert_allclose(_np16(gpu.conv_state).astype(np.float32), orc.conv.astype(np.float32),
                               atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("B", [1, 4, 32])
def test_tiny_generate_tokens(tiny_weights, B):
    """Graph-replayed generation (8 fused steps per replay) yields the oracle's greedy tokens."""
    w = tiny_weights
    gpu = DFSSMModel.from_weights(w, device=DEV, batch_size=B)
    prompts = make_prompts(B, w.cfg.vocab_size, 8)
    n = 21
    got = gpu.generate(n_tokens=n, prompt=torch.from_numpy(prompts), return_tokens=True, verbose=False)
    ref, _ = O.OracleModel(w, B).generate(prompts, n)
    np.testing.assert_array_equal(got.cpu().numpy(), ref)
    # generating again from a reset state reproduces the same tokens
    again = gpu.generate(n_tokens=n, prompt=torch.from_numpy(prompts), return_tokens=True, verbose=False)
    np.testing.assert_array_equal(again.cpu().numpy(), ref)
    assert gpu.error_flag() == 0


def test_reset_state_and_token_range(tiny_weights):
    gpu = DFSSMModel.from_weights(tiny_weights, device=DEV, batch_size=1)
    gpu.forward(torch.tensor([3]))
    assert float(gpu.h_state.abs().max()) > 0
    gpu.reset_state()
    assert float(gpu.h_state.abs().max()) == 0 and float(gpu.conv_state.abs().max()) == 0
    with pytest.raises(IndexError):
        gpu.forward(torch.tensor([tiny_weights.cfg.vocab_size]))


@pytest.fixture(scope="module")
def w13():
    return make_weights(config_1p3b(), seed=0)


@pytest.mark.parametrize("B,T,n", [(1, 32, 128), (4, 8, 8), (8, 4, 4)])
def test_1p3b_greedy(w13, B, T, n):
    """Config 3 at batch 1 (32-token seeded prompt, 128 generated) and short batch-4 and batch-8
    runs: identical greedy tokens, state within 1e-3 after the run, identical final logits."""
    w = w13
    print(f"1.3B B={B} T={T} n={n}", flush=True)
    prompts = make_prompts(B, w.cfg.vocab_size, T)
    gpu = DFSSMModel.from_weights(w, device=DEV, batch_size=B)
    orc = O.OracleModel(w, B)
    ref, _ = orc.generate(prompts, n)
    got = gpu.generate(n_tokens=n, prompt=torch.from_numpy(prompts), return_tokens=True, verbose=False)
    np.testing.assert_array_equal(got.cpu().numpy(), ref)
    rel = _state_rel(gpu, orc)
    # one more step through forward() on both: logits of the last generated token
    lg = _np16(gpu.forward(torch.from_numpy(ref[:, -1]).to(DEV))).astype(np.float32)
    lo, _ = orc.step(ref[:, -1])
    err = np.abs(lg - lo.astype(np.float32)).max()
    print(f"1.3B B={B}: state rel err {rel:.3e}, final logits max abs err {err:.3e}")
    assert rel <= 1e-3
    assert err == 0.0
    assert gpu.error_flag() == 0


def _require_one_launch(gpu):
    """The one-launch layer must really run for these dims on this device."""
    from dfssm import _C
    props = torch.cuda.get_device_properties(0)
    assert _C.lib().dfssm_one_launch_plan(gpu.dims, props.multi_processor_count, 1) > 0


@pytest.mark.parametrize("B", [1, 2, 3, 4])
def test_one_launch_layer_equals_five_kernels(tiny_weights, B):
    """dfssm_layer_step (one launch at batch <= 4) against dfssm_layer_phase 0..4 (the five-kernel
    form) on the same inputs: x, SSM state and conv state identical bit for bit."""
    from dfssm import _C
    w = tiny_weights
    kernel = 1  # DFSSM_LAYER_FUSED
    print(f"one-launch layer B={B}", flush=True)
    gpu = DFSSMModel.from_weights(w, device=DEV, batch_size=B)
    _require_one_launch(gpu)
    gpu.ingest(torch.from_numpy(make_prompts(B, w.cfg.vocab_size, 5)))  # non-trivial state
    lib = _C.lib()
    x0, h0, c0 = gpu.x.clone(), gpu.h_state.clone(), gpu.conv_state.clone()
    prev = lib.dfssm_set_layer_kernel(kernel)
    try:
        for li in range(w.cfg.n_layer):
            _C.check(lib.dfssm_layer_step(gpu._model, li, gpu.x.data_ptr(), gpu._state, gpu.workspace.data_ptr(),
                                          _C.stream()))
        torch.cuda.synchronize()
    finally:
        lib.dfssm_set_layer_kernel(prev)
    x1, h1, c1 = gpu.x.clone(), gpu.h_state.clone(), gpu.conv_state.clone()
    gpu.x.copy_(x0); gpu.h_state.copy_(h0); gpu.conv_state.copy_(c0)
    for li in range(w.cfg.n_layer):
        for ph in range(5):
            _C.check(lib.dfssm_layer_phase(gpu._model, li, ph, gpu.x.data_ptr(), gpu._state,
                                           gpu.workspace.data_ptr(), _C.stream()))
    torch.cuda.synchronize()
    assert torch.equal(gpu.x.view(torch.int16), x1.view(torch.int16))
    assert torch.equal(gpu.h_state, h1)
    assert torch.equal(gpu.conv_state.view(torch.int16), c1.view(torch.int16))
    assert gpu.error_flag() == 0


def _decode_run(w, B, kernel, steps, prompt_len=5):
    """`steps` greedy decode steps through dfssm_decode_step with layer-kernel setting `kernel`:
    per step the logits and next tokens, then x and both states."""
    from dfssm import _C
    lib = _C.lib()
    gpu = DFSSMModel.from_weights(w, device=DEV, batch_size=B)
    gpu.ingest(torch.from_numpy(make_prompts(B, w.cfg.vocab_size, prompt_len)))
    prev = lib.dfssm_set_layer_kernel(kernel)
    try:
        out = []
        for _ in range(steps):
            lg, nx = gpu.decode_step_eager(None)
            out.append((lg.clone(), nx.clone()))
        torch.cuda.synchronize()
    finally:
        lib.dfssm_set_layer_kernel(prev)
    assert gpu.error_flag() == 0
    return out, gpu.x.clone(), gpu.h_state.clone(), gpu.conv_state.clone()


@pytest.mark.parametrize("B", [1, 2, 3, 4])
def test_one_launch_decode_equals_five_kernels(tiny_weights, B):
    """dfssm_decode_step with the one-launch layer (DFSSM_LAYER_FUSED) against the five-kernel
    form, 6 greedy steps: logits, tokens, x and both states identical bit for bit."""
    print(f"one-launch decode B={B}", flush=True)
    out_x, x_x, h_x, c_x = _decode_run(tiny_weights, B, 1, 6)
    out_5, x_5, h_5, c_5 = _decode_run(tiny_weights, B, 2, 6)
    for (lx, nx), (l5, n5) in zip(out_x, out_5):
        assert torch.equal(lx.view(torch.int16), l5.view(torch.int16))
        assert torch.equal(nx, n5)
    assert torch.equal(x_x.view(torch.int16), x_5.view(torch.int16))
    assert torch.equal(h_x, h_5)
    assert torch.equal(c_x.view(torch.int16), c_5.view(torch.int16))


@pytest.mark.parametrize("B", [5, 16, 17, 33, 64])   # 17, 33: partial row blocks, idle prologue workgroups
def test_batched_ssm_prologue_launch_equals_five_kernels(tiny_weights, B):
    """Batch >= 5: dfssm_decode_step with the default setting (the SSM step and the out_proj
    prologue in one launch, g handed over as tagged words) against DFSSM_LAYER_FIVE (separate SSM
    and prologue kernels), 6 greedy steps: logits, tokens, x and both states identical bit for bit."""
    print(f"ssm+prologue decode B={B}", flush=True)
    out_a, x_a, h_a, c_a = _decode_run(tiny_weights, B, 0, 6)
    out_5, x_5, h_5, c_5 = _decode_run(tiny_weights, B, 2, 6)
    for (la, na), (l5, n5) in zip(out_a, out_5):
        assert torch.equal(la.view(torch.int16), l5.view(torch.int16))
        assert torch.equal(na, n5)
    assert torch.equal(x_a.view(torch.int16), x_5.view(torch.int16))
    assert torch.equal(h_a, h_5)
    assert torch.equal(c_a.view(torch.int16), c_5.view(torch.int16))


@pytest.mark.parametrize("B", [5, 32])
def test_fused_phases_equal_five_phases(tiny_weights, B):
    """dfssm_layer_phase with the fused launches (phases 0 and 1, DFSSM_PHASE_SSM_PROLOGUE = 5,
    DFSSM_PHASE_OUT_PROLOGUE = 6 writing the next layer's prologue, 4 for the last layer) against
    phases 0..4 of every layer on the same inputs: x, SSM state and conv state identical bit for
    bit (each layer's in_proj reads the prologue the fused launch wrote)."""
    from dfssm import _C
    w = tiny_weights
    print(f"fused phases B={B}", flush=True)
    gpu = DFSSMModel.from_weights(w, device=DEV, batch_size=B)
    gpu.ingest(torch.from_numpy(make_prompts(B, w.cfg.vocab_size, 5)))
    lib = _C.lib()
    L = w.cfg.n_layer

    def ph(li, p):
        return lib.dfssm_layer_phase(gpu._model, li, p, gpu.x.data_ptr(), gpu._state, gpu.workspace.data_ptr(),
                                     _C.stream())

    x0, h0, c0 = gpu.x.clone(), gpu.h_state.clone(), gpu.conv_state.clone()
    for li in range(L):
        for p in range(5):
            _C.check(ph(li, p))
    torch.cuda.synchronize()
    x5, h5, c5 = gpu.x.clone(), gpu.h_state.clone(), gpu.conv_state.clone()
    gpu.x.copy_(x0); gpu.h_state.copy_(h0); gpu.conv_state.copy_(c0)
    assert ph(L - 1, _C.PHASE_OUT_PROLOGUE) == _C.DFSSM_E_DIMS  # no next layer
    prepped = False
    for li in range(L):
        if not prepped:
            _C.check(ph(li, 0))
        _C.check(ph(li, 1))
        _C.check(ph(li, _C.PHASE_SSM_PROLOGUE))
        rc = ph(li, _C.PHASE_OUT_PROLOGUE) if li + 1 < L else _C.DFSSM_E_DIMS
        prepped = rc == 0
        if rc == _C.DFSSM_E_DIMS:
            _C.check(ph(li, 4))
        else:
            _C.check(rc)
    torch.cuda.synchronize()
    assert gpu.error_flag() == 0
    assert torch.equal(gpu.x.view(torch.int16), x5.view(torch.int16))
    assert torch.equal(gpu.h_state, h5)
    assert torch.equal(gpu.conv_state.view(torch.int16), c5.view(torch.int16))


def test_fused_phases_wide_model_batch64():
    """d_model 4608 at batch 64: out_proj at 32 output rows per workgroup has one GEMM grid row
    walking two 32-row blocks, followed by the prologue workgroups' rows (the GEMM workgroups must
    take their row ranges from the GEMM rows alone). The decode step against DFSSM_LAYER_FIVE:
    logits, tokens, x and both states identical bit for bit."""
    from dfssm.format import DFSSMConfig
    c = DFSSMConfig(n_layer=2, d_model=4608, d_inner=1024, d_state=128, nheads=16, headdim=64, ngroups=1,
                    vocab_size=4096, kw=4)
    w = make_weights(c, seed=11)
    print("wide model d_model 4608 B=64 decode", flush=True)
    out_a, x_a, h_a, c_a = _decode_run(w, 64, 0, 3)
    out_5, x_5, h_5, c_5 = _decode_run(w, 64, 2, 3)
    for (la, na), (l5, n5) in zip(out_a, out_5):
        assert torch.equal(la.view(torch.int16), l5.view(torch.int16))
        assert torch.equal(na, n5)
    assert torch.equal(x_a.view(torch.int16), x_5.view(torch.int16))
    assert torch.equal(h_a, h_5)
    assert torch.equal(c_a.view(torch.int16), c_5.view(torch.int16))


@pytest.mark.parametrize("B", [1, 4])
def test_one_launch_layer_wide_model(B):
    """d_model 4096 (128 out_proj groups of 32 rows, the widest grid use): the one-launch layer
    against the five-kernel form, bit for bit."""
    from dfssm import _C
    from dfssm.format import DFSSMConfig
    c = DFSSMConfig(n_layer=1, d_model=4096, d_inner=4096, d_state=128, nheads=64, headdim=64, ngroups=1,
                    vocab_size=1000, kw=4)
    w = make_weights(c, seed=5)
    kernel = 1  # DFSSM_LAYER_FUSED
    print(f"wide one-launch layer B={B}", flush=True)
    gpu = DFSSMModel.from_weights(w, device=DEV, batch_size=B)
    _require_one_launch(gpu)
    gpu.ingest(torch.from_numpy(make_prompts(B, c.vocab_size, 3)))
    lib = _C.lib()
    x0, h0, c0 = gpu.x.clone(), gpu.h_state.clone(), gpu.conv_state.clone()
    prev = lib.dfssm_set_layer_kernel(kernel)
    try:
        _C.check(lib.dfssm_layer_step(gpu._model, 0, gpu.x.data_ptr(), gpu._state, gpu.workspace.data_ptr(),
                                      _C.stream()))
        torch.cuda.synchronize()
    finally:
        lib.dfssm_set_layer_kernel(prev)
    x1, h1, c1 = gpu.x.clone(), gpu.h_state.clone(), gpu.conv_state.clone()
    gpu.x.copy_(x0); gpu.h_state.copy_(h0); gpu.conv_state.copy_(c0)
    for ph in range(5):
        _C.check(lib.dfssm_layer_phase(gpu._model, 0, ph, gpu.x.data_ptr(), gpu._state, gpu.workspace.data_ptr(),
                                       _C.stream()))
    torch.cuda.synchronize()
    assert torch.equal(gpu.x.view(torch.int16), x1.view(torch.int16))
    assert torch.equal(gpu.h_state, h1)
    assert torch.equal(gpu.conv_state.view(torch.int16), c1.view(torch.int16))
    assert gpu.error_flag() == 0


@pytest.mark.parametrize("emb_code", [0, 1])
def test_wide_model_head_batch4(emb_code):
    """d_model 4096 at batch 4: the exact head for both table types (the fp16 table's fp64 head
    holds 3 rows in LDS, so it runs the rows in two launches) against the oracle's logits."""
    from dfssm.format import DFSSMConfig
    c = DFSSMConfig(n_layer=1, d_model=4096, d_inner=4096, d_state=128, nheads=64, headdim=64, ngroups=1,
                    vocab_size=1000, kw=4, emb_code=emb_code)
    w = make_weights(c, seed=6)
    B = 4
    print(f"wide head emb_code={emb_code}", flush=True)
    gpu = DFSSMModel.from_weights(w, device=DEV, batch_size=B)
    orc = O.OracleModel(w, B)
    tok = make_prompts(B, c.vocab_size, 1)[:, 0]
    for t in range(3):
        lg = _np16(gpu.forward(torch.from_numpy(tok).to(DEV))).astype(np.float32)
        lo, nxt = orc.step(tok)
        assert np.abs(lg - lo.astype(np.float32)).max() == 0.0, f"step {t}"
        np.testing.assert_array_equal(lg.argmax(axis=1), nxt)
        tok = nxt
    assert gpu.error_flag() == 0


@pytest.mark.parametrize("B", [8, 40, 64])
def test_batched_head_large_final_norm_values(B):
    """The batched exact head splits xf 2^24 into six signed base-256 digits; rows whose xf needs
    only the low four digits (|xf| < 128), five (up to 2^15) or all six (above) must all come out
    exact. Crafted residual rows through dfssm_lmhead_argmax with the final-norm weight of column 0
    set to 2000: ordinary rows put xf in column 0 up to ~1e4 (five digits); a large entry in column
    0 of every fourth row puts it near 3.9e4 (six); the unscaled weight keeps every |xf| below 128
    (four). Logits and tokens identical to the oracle's head (RMSNorm then the exact int8 head)."""
    from dfssm import _C
    w = make_weights(config_tiny(n_layer=1), seed=17)
    D, V = w.cfg.d_model, w.cfg.vocab_size
    lib = _C.lib()
    rng = np.random.default_rng(100 + B)
    for case in ("four", "five", "six"):
        wc = make_weights(config_tiny(n_layer=1), seed=17)
        if case != "four":
            nf = wc.norm_f.astype(np.float64)
            nf[0] = 2000.0
            wc.norm_f = nf.astype(wc.norm_f.dtype)
        x = rng.normal(0.0, 1.0, (B, D)).astype(np.float16)
        if case == "six":
            x[::4, 0] = np.float16(40.0)
        print(f"head digits ({case}), B={B}", flush=True)
        gpu = DFSSMModel.from_weights(wc, device=DEV, batch_size=B)
        xg = torch.from_numpy(x).to(DEV)
        lg = torch.empty((B, V), dtype=torch.float16, device=DEV)
        nx = torch.empty(B, dtype=torch.int64, device=DEV)
        _C.check(lib.dfssm_lmhead_argmax(gpu._model, xg.data_ptr(), gpu.workspace.data_ptr(), lg.data_ptr(),
                                         nx.data_ptr(), None, _C.stream()))
        torch.cuda.synchronize()
        xf = O.rmsnorm(x, wc.norm_f)
        if case == "six":
            assert np.abs(xf[::4, 0].astype(np.float32)).min() >= 32768.0
        lo, no = O.lm_head(wc, xf)
        assert np.isfinite(lo.astype(np.float32)).all()
        got = _np16(lg).astype(np.float32)
        assert np.abs(got - lo.astype(np.float32)).max() == 0.0, case
        np.testing.assert_array_equal(nx.cpu().numpy(), no)
        assert gpu.error_flag() == 0
        del gpu


@pytest.fixture(scope="module")
def tiny_weights_f16():
    # the exporter's fp16 embedding table (format embedding code 0)
    return make_weights(config_tiny(n_layer=3, emb_code=0), seed=4)


@pytest.mark.parametrize("B", [1, 3, 5])
def test_tiny_fp16_embedding(tiny_weights_f16, B):
    """An fp16 tied table: gather and head (fp64-exact at batch <= 4, fp16 matrix cores with fp32
    accumulation above) against the oracle; identical greedy tokens."""
    w = tiny_weights_f16
    assert w.emb.dtype == np.float16 and w.emb_scale is None
    gpu = DFSSMModel.from_weights(w, device=DEV, batch_size=B)
    orc = O.OracleModel(w, B)
    prompts = make_prompts(B, w.cfg.vocab_size, 4)
    tok = prompts[:, 0]
    for t in range(12):
        logits_g = _np16(gpu.forward(torch.from_numpy(tok).to(DEV))).astype(np.float32)
        logits_o, nxt = orc.step(tok)
        err = np.abs(logits_g - logits_o.astype(np.float32)).max()
        if B <= 4:
            assert err == 0.0, f"step {t}: logits differ by {err}"
        assert err <= 2e-2
        np.testing.assert_array_equal(logits_g.argmax(axis=1), nxt)
        tok = prompts[:, t + 1] if t + 1 < prompts.shape[1] else nxt
    got = gpu.generate(n_tokens=9, prompt=torch.from_numpy(prompts), return_tokens=True, verbose=False)
    ref, _ = O.OracleModel(w, B).generate(prompts, 9)
    np.testing.assert_array_equal(got.cpu().numpy(), ref)
    assert gpu.error_flag() == 0


def test_2p7b_layer_shapes_batch64():
    """Config 4's layer shapes (d_model 2560, d_inner 5120, 80 heads, in_proj 10576) at batch 64 on
    the matrix-core path, 4 layers and a 4096-token vocabulary so that the oracle stays fast:
    identical logits and greedy tokens, state within 1e-3 relative."""
    from dfssm.format import DFSSMConfig
    c = DFSSMConfig(n_layer=4, d_model=2560, d_inner=5120, d_state=128, nheads=80, headdim=64, ngroups=1,
                    vocab_size=4096, kw=4)
    w = make_weights(c, seed=5)
    B = 64
    print("2.7B-shape layers, batch 64", flush=True)
    gpu = DFSSMModel.from_weights(w, device=DEV, batch_size=B)
    orc = O.OracleModel(w, B)
    prompts = make_prompts(B, c.vocab_size, 3)
    ref, _ = orc.generate(prompts, 3)
    got = gpu.generate(n_tokens=3, prompt=torch.from_numpy(prompts), return_tokens=True, verbose=False)
    np.testing.assert_array_equal(got.cpu().numpy(), ref)
    assert _state_rel(gpu, orc) <= 1e-3
    lg = _np16(gpu.forward(torch.from_numpy(ref[:, -1]).to(DEV))).astype(np.float32)
    lo, _ = orc.step(ref[:, -1])
    assert np.abs(lg - lo.astype(np.float32)).max() == 0.0
    assert gpu.error_flag() == 0
