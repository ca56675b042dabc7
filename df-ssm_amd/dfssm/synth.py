"""Seeded synthetic DF-SSM models and prompts (random-init weights of the real shapes).

All draws come from numpy's PCG64 through `np.random.default_rng([seed, stream])`, so the
bytes are identical on every machine. Distributions follow the benchmark configurations:
scaffold sign bits uniform, per-row fp16 scales U(0.01, 0.05), rank-16 int8 LoRA
clip(rne(N(0, 20))), int8 embedding clip(rne(N(0, 30))) with a per-row fp16 scale, A_log
U(0, ln 16). Values the configurations leave open are chosen here:
  LoRA B row scale 1/(20*sqrt(K)) * U(0.5, 1.5), LoRA A row scale 1.7e-3 * U(0.5, 1.5)
  (LoRA adds about 10% of the scaffold output); embedding row scale U(0.002, 0.005)
  (tied-head logits have std about 5); conv_w N(0, 0.5^2), conv_b N(0, 0.1^2);
  dt_bias = softplus^-1(exp(U(ln 1e-3, ln 1e-1))) (Mamba-2 init); D, norm weights
  1 + U(-0.1, 0.1) (not exactly 1, so a dropped weight multiply is visible in tests).
"""
from __future__ import annotations

import numpy as np

from .format import (DFSSMConfig, DFSSMWeights, EMB_F16, EMB_I8, LORA_RANK, NORM_F32,
                     layer_tensor_specs)

# Shapes of the benchmark configurations.
def config_1p3b(emb_code: int = EMB_I8) -> DFSSMConfig:
    return DFSSMConfig(n_layer=48, d_model=2048, d_inner=4096, d_state=128, nheads=64, headdim=64,
                       ngroups=1, vocab_size=50288, kw=4, emb_code=emb_code, norm_code=NORM_F32)


def config_2p7b(emb_code: int = EMB_I8) -> DFSSMConfig:
    return DFSSMConfig(n_layer=64, d_model=2560, d_inner=5120, d_state=128, nheads=80, headdim=64,
                       ngroups=1, vocab_size=50288, kw=4, emb_code=emb_code, norm_code=NORM_F32)


def config_tiny(n_layer: int = 2, emb_code: int = EMB_I8) -> DFSSMConfig:
    """Small model for fast parity tests: the kernels' constraints at the smallest sizes."""
    return DFSSMConfig(n_layer=n_layer, d_model=512, d_inner=1024, d_state=128, nheads=16, headdim=64,
                       ngroups=1, vocab_size=1000, kw=4, emb_code=emb_code, norm_code=NORM_F32)


def _i8_normal(rng, sigma, shape):
    return np.clip(np.rint(rng.normal(0.0, sigma, shape)), -127, 127).astype(np.int8)


def make_layer(cfg: DFSSMConfig, seed: int, li: int) -> dict:
    rng = np.random.default_rng([seed, 1, li])
    D, DI, H, R = cfg.d_model, cfg.d_inner, cfg.nheads, LORA_RANK
    IPO, C = cfg.in_proj_out, cfg.d_xbc
    nd = cfg.norm_dtype()
    out = {}
    for pre, n_out, k_in in (("in", IPO, D), ("out", D, DI)):
        out[f"{pre}_packed"] = rng.integers(0, 2 ** 32, size=(n_out, k_in // 32), dtype=np.uint32)
        out[f"{pre}_scale"] = rng.uniform(0.01, 0.05, n_out).astype(np.float16)
        out[f"{pre}_lA"] = _i8_normal(rng, 20.0, (n_out, R))
        out[f"{pre}_lA_s"] = (1.7e-3 * rng.uniform(0.5, 1.5, n_out)).astype(np.float16)
        out[f"{pre}_lB"] = _i8_normal(rng, 20.0, (R, k_in))
        out[f"{pre}_lB_s"] = (rng.uniform(0.5, 1.5, R) / (20.0 * np.sqrt(k_in))).astype(np.float16)
    out["conv_w"] = rng.normal(0.0, 0.5, (C, 4)).astype(np.float16)
    out["conv_b"] = rng.normal(0.0, 0.1, C).astype(np.float16)
    out["A_log"] = rng.uniform(0.0, np.log(16.0), H).astype(np.float32)
    out["D"] = (1.0 + rng.uniform(-0.1, 0.1, H)).astype(np.float32)
    dt = np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), H))
    out["dt_bias"] = (dt + np.log(-np.expm1(-dt))).astype(np.float32)
    out["norm_w"] = (1.0 + rng.uniform(-0.1, 0.1, DI)).astype(nd)
    out["ln_w"] = (1.0 + rng.uniform(-0.1, 0.1, D)).astype(nd)
    for name, shape, dt_ in layer_tensor_specs(cfg):
        assert out[name].shape == shape and out[name].dtype == np.dtype(dt_), name
    return out


def make_weights(cfg: DFSSMConfig, seed: int = 0) -> DFSSMWeights:
    cfg.validate()
    rng = np.random.default_rng([seed, 0])
    V, D = cfg.vocab_size, cfg.d_model
    e8 = _i8_normal(rng, 30.0, (V, D))
    es = rng.uniform(0.002, 0.005, V).astype(np.float16)
    if cfg.emb_code == EMB_I8:
        emb, emb_scale = e8, es
    else:
        emb, emb_scale = (e8.astype(np.float32) * es.astype(np.float32)[:, None]).astype(np.float16), None
    w = DFSSMWeights(cfg, emb, emb_scale)
    w.layers = [make_layer(cfg, seed, li) for li in range(cfg.n_layer)]
    frng = np.random.default_rng([seed, 2])
    w.norm_f = (1.0 + frng.uniform(-0.1, 0.1, D)).astype(cfg.norm_dtype())
    return w


def make_prompts(batch: int, vocab: int, n_tokens: int = 32, base_seed: int = 1000) -> np.ndarray:
    """(batch, n_tokens) int64 prompts; sequence b draws from seed base_seed + b."""
    return np.stack([np.random.default_rng(base_seed + b).integers(0, vocab, n_tokens)
                     for b in range(batch)]).astype(np.int64)
