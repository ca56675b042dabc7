"""Float weights -> `.dfssm`: the reference exporter's conversion (training/export_dfssm.py).

The reference exporter (export_dfssm.py:67-193) loads a distilled student whose scaffold
projections are FrozenDFWWithLoRA modules (training/df_ssm_dfw_lora.py:45-90: a frozen
multi-level weight `frozen_weight` plus trainable `lora_A` (out, r), `lora_B` (r, in) and
`scaling = lora_alpha / r`) and writes, per projection:

  sign bits     bit = 1 where w > 0, else 0 -- (w.sign() + 1) // 2, so an exact zero weight
                (the frozen levels include 0) becomes a 0 bit, i.e. -1    (export_dfssm.py:143-147)
  row scale     fp16(mean_k |w|), the mean taken in fp32                  (:150-151)
  LoRA A, B     quantize_to_int8(lora_A * scaling), quantize_to_int8(lora_B): per row
                s = max(max|row| / 127, 1e-8) in fp32, q = clamp(round(row / s), -128, 127)
                (round half to even), stored s as fp16                    (:45-50,154-162)

and conv weight (C, 1, 4) -> (C, 4) fp16, conv bias fp16, A_log / D / dt_bias / both norms / the
final norm fp32, the embedding fp16 (:125-126,169-193). This module does the same from a state
dict (torch tensors or numpy arrays, the student's parameter names) or from per-layer arrays.
The reductions run in torch on the CPU, as the reference exporter's do (it loads everything with
map_location='cpu'), so means and maxima round identically.

Differences, all optional: the header's headdim field defaults to d_inner / nheads (the reference
writes its constant 32, export_dfssm.py:24,114; pass headdim_field=32 for byte-identical
headers), and emb_code=EMB_I8 stores the tied table as int8 + fp16 row scale (this format's
extension, reserved byte 0) instead of fp16.
"""
from __future__ import annotations

from typing import Dict, Mapping, Optional

import numpy as np

from .format import (D_CONV, EMB_F16, EMB_I8, LORA_RANK, NORM_F32, DFSSMConfig, DFSSMWeights, pack_sign_bits,
                     write_dfssm)


def _t(a):
    import torch
    if isinstance(a, torch.Tensor):
        return a.detach().to("cpu")
    return torch.from_numpy(np.ascontiguousarray(a))


def _np16(t) -> np.ndarray:
    import torch
    return t.to(torch.float16).numpy()


def scaffold_bits_and_scale(w):
    """(out, in) float weight -> ((out, in/32) uint32 sign bits, (out,) fp16 mean |w|)
    (export_dfssm.py:143-151)."""
    import torch
    w = _t(w).to(torch.float32)
    signs = (w > 0).numpy().astype(np.uint8)  # == (sign(w) + 1) // 2 for every non-NaN w
    return pack_sign_bits(signs), _np16(w.abs().mean(dim=1))


def quantize_rows_int8(w):
    """Per-row symmetric int8 (export_dfssm.py:45-50): s = max(max|row| / 127, 1e-8) in fp32,
    q = clamp(round_half_even(row / s), -128, 127); returns (int8 q, fp16 s)."""
    import torch
    w = _t(w).to(torch.float32)
    s = (w.abs().amax(dim=-1) / 127.0).clamp(min=1e-8)
    q = torch.round(w / s.unsqueeze(-1)).clamp(-128, 127).to(torch.int8)
    return q.numpy(), _np16(s)


def lora_factors(lora_A, lora_B, scaling: float):
    """(out, r) A and (r, in) B -> int8 A of A * scaling with its row scales, int8 B with its
    row scales (export_dfssm.py:154-162)."""
    import torch
    A = _t(lora_A).to(torch.float32) * scaling
    qa, sa = quantize_rows_int8(A)
    qb, sb = quantize_rows_int8(lora_B)
    return qa, sa, qb, sb


def export_layer(in_w, in_A, in_B, out_w, out_A, out_B, conv_w, conv_b, A_log, D, dt_bias, norm_w, ln_w,
                 scaling: float) -> Dict[str, np.ndarray]:
    """One layer's float tensors -> the .dfssm layer dict (names of format.layer_tensor_specs)."""
    import torch
    L = {}
    for pre, w, A, B in (("in", in_w, in_A, in_B), ("out", out_w, out_A, out_B)):
        packed, scale = scaffold_bits_and_scale(w)
        qa, sa, qb, sb = lora_factors(A, B, scaling)
        L.update({f"{pre}_packed": packed, f"{pre}_scale": scale, f"{pre}_lA": qa, f"{pre}_lA_s": sa,
                  f"{pre}_lB": qb, f"{pre}_lB_s": sb})
    cw = _t(conv_w)
    if cw.dim() == 3:  # nn.Conv1d weight (C, 1, d_conv)
        cw = cw.squeeze(1)
    L["conv_w"] = _np16(cw)
    L["conv_b"] = _np16(_t(conv_b))
    for name, a in (("A_log", A_log), ("D", D), ("dt_bias", dt_bias), ("norm_w", norm_w), ("ln_w", ln_w)):
        L[name] = _t(a).to(torch.float32).numpy()
    return L


def int8_table(emb16: np.ndarray):
    """fp16 (V, D) table -> int8 table and (V,) fp16 row scale (absmax / 127): the int8 tied-head
    variant of this format (not part of the reference exporter)."""
    e = emb16.astype(np.float32)
    s = np.maximum(np.abs(e).max(axis=1), 1e-8) / 127.0
    q = np.clip(np.rint(e / s[:, None]), -127, 127).astype(np.int8)
    return q, s.astype(np.float16)


def weights_from_state_dict(sd: Mapping[str, object], lora_alpha: float = 1.0, lora_rank: int = LORA_RANK,
                            kw: int = 4, headdim_field: Optional[int] = None,
                            emb_code: int = EMB_F16) -> DFSSMWeights:
    """The student's state dict (after freeze_scaffold_add_lora with lora_layers='all' and
    lora_targets='both', df_ssm_dfw_lora.py:107-150) -> DFSSMWeights, as export_dfssm.py:67-193.

    Keys used: embedding.weight, norm_f.weight, and per layer i under layers.{i}.:
    mixer.{in_proj,out_proj}.{frozen_weight,lora_A,lora_B}, mixer.conv1d.{weight,bias},
    mixer.{A_log,D,dt_bias}, mixer.norm.weight, norm.weight. `scaling` = lora_alpha / lora_rank
    (FrozenDFWWithLoRA.scaling, df_ssm_dfw_lora.py:77; an attribute, not in the state dict)."""
    if lora_rank != LORA_RANK:
        raise ValueError(f"the format stores rank-{LORA_RANK} LoRA factors (got rank {lora_rank})")
    n_layer = 0
    while f"layers.{n_layer}.mixer.in_proj.frozen_weight" in sd:
        n_layer += 1
    if n_layer == 0:
        raise KeyError("no layers.{i}.mixer.in_proj.frozen_weight in the state dict")
    emb = _t(sd["embedding.weight"])
    V, Dm = emb.shape
    p0 = "layers.0.mixer."
    DI = int(_t(sd[p0 + "norm.weight"]).shape[0])
    H = int(_t(sd[p0 + "A_log"]).shape[0])
    IPO = int(_t(sd[p0 + "in_proj.frozen_weight"]).shape[0])
    N = (IPO - 2 * DI - H) // 2  # ngroups = 1 (export_dfssm.py:22)
    cfg = DFSSMConfig(n_layer=n_layer, d_model=int(Dm), d_inner=DI, d_state=N, nheads=H,
                      headdim=headdim_field if headdim_field is not None else DI // H, ngroups=1,
                      vocab_size=int(V), kw=kw, emb_code=emb_code, norm_code=NORM_F32)
    cfg.validate()
    scaling = lora_alpha / lora_rank
    layers = []
    for i in range(n_layer):
        p = f"layers.{i}.mixer."
        layers.append(export_layer(
            sd[p + "in_proj.frozen_weight"], sd[p + "in_proj.lora_A"], sd[p + "in_proj.lora_B"],
            sd[p + "out_proj.frozen_weight"], sd[p + "out_proj.lora_A"], sd[p + "out_proj.lora_B"],
            sd[p + "conv1d.weight"], sd[p + "conv1d.bias"], sd[p + "A_log"], sd[p + "D"], sd[p + "dt_bias"],
            sd[p + "norm.weight"], sd[f"layers.{i}.norm.weight"], scaling))
    e16 = _np16(emb)
    if emb_code == EMB_I8:
        table, scale = int8_table(e16)
    else:
        table, scale = e16, None
    import torch
    norm_f = _t(sd["norm_f.weight"]).to(torch.float32).numpy()
    return DFSSMWeights(cfg, table, scale, layers, norm_f)


def export_dfssm(sd: Mapping[str, object], path: str, **kw) -> int:
    """weights_from_state_dict(sd, **kw) written to `path`; returns the byte count."""
    return write_dfssm(path, weights_from_state_dict(sd, **kw))


__all__ = ["scaffold_bits_and_scale", "quantize_rows_int8", "lora_factors", "export_layer", "int8_table",
           "weights_from_state_dict", "export_dfssm", "D_CONV", "EMB_I8", "EMB_F16"]
