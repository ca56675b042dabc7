"""
Drop-in for the reference's pybind module `df_ssm_kernels` (inference/gpu/df_ssm_kernels.cu:153-157).

    conv_step(conv_state, xBC, conv_weight, conv_bias, d_xBC)        df_ssm_kernels.cu:109-125
    ssm_step(h_state, xBC, dt, dt_bias, A_log, D_param, y_out)      df_ssm_kernels.cu:127-151

Same argument order and meaning, launched asynchronously on the current stream like the
reference. Differences, all deliberate:
  - h_state is fp32 (batch, nheads, headdim, d_state); the reference's state is fp16.
  - the head dimension is read from h_state.shape (the reference hard-codes 32) and the
    dimensions come from the tensors, not compile-time constants;
  - arguments are validated (dtype, device, shape, contiguity) and errors raise; the reference
    does no checking and reports no errors;
  - y_out is fully written, so the caller need not zero it first (df_ssm_inference.py:188).
"""
from __future__ import annotations

import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from dfssm import ops as _ops  # noqa: E402


def conv_step(conv_state, xBC, conv_weight, conv_bias, d_xBC):
    if xBC.dim() != 2 or xBC.shape[1] != d_xBC:
        raise ValueError(f"xBC must be (batch, {d_xBC}), got {tuple(xBC.shape)}")
    _ops.conv_step(conv_state, xBC, conv_weight, conv_bias)


def ssm_step(h_state, xBC, dt, dt_bias, A_log, D_param, y_out):
    B, H, P, N = h_state.shape
    if xBC.shape[0] != B or xBC.shape[1] < H * P + 2 * N:
        raise ValueError("xBC must hold x | B | C for every sequence")
    if dt.shape != (B, H) or y_out.shape[0] != B or y_out.shape[1] < H * P:
        raise ValueError("dt must be (batch, nheads) and y_out (batch, >= nheads*headdim)")
    _ops.ssm_step(h_state, xBC, dt, dt_bias, A_log, D_param, y_out)
