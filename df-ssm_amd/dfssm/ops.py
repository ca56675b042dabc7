"""Single-operator wrappers over the C ABI, taking torch tensors on the GPU.

These are the operator-level entry points (scaffold GEMM, RMSNorm+quantize, conv step, SSM step,
bit/embedding tiling). Every call launches on torch's current stream and raises on any error;
there is no CPU fallback.
"""
from __future__ import annotations

import torch

from . import _C


def _need(t: torch.Tensor, dtype, name: str):
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise TypeError(f"{name} must be a CUDA (HIP) tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")


def tile_bits(packed: torch.Tensor, rows: int, k: int) -> torch.Tensor:
    """(rows, k/32) int32 sign-bit words -> tiled copy for the scaffold kernels."""
    _need(packed, torch.int32, "packed")
    if not packed.is_contiguous() or packed.numel() != rows * (k // 32):
        raise ValueError("packed must be a contiguous (rows, k/32) int32 tensor")
    out = torch.empty(_C.lib().dfssm_tiled_bits_bytes(rows, k) // 4, dtype=torch.int32, device=packed.device)
    _C.check(_C.lib().dfssm_tile_bits(packed.data_ptr(), out.data_ptr(), rows, k, _C.stream()), "tile_bits")
    return out


def scaffold_gemm(tiled_bits: torch.Tensor, q: torch.Tensor, N: int, xscale=None, wscale=None, want_y=False):
    """int32 acc (M, N) = q (M, K) int8 x sign-bit matrix^T; optionally y fp16 (M, N)."""
    _need(q, torch.int8, "q")
    M, K = q.shape
    acc = torch.empty(M, N, dtype=torch.int32, device=q.device)
    y = torch.empty(M, N, dtype=torch.float16, device=q.device) if want_y else None
    _C.check(_C.lib().dfssm_scaffold_gemm(
        tiled_bits.data_ptr(), q.contiguous().data_ptr(), _C.ptr(xscale), _C.ptr(wscale), M, N, K,
        acc.data_ptr(), _C.ptr(y), _C.stream()), "scaffold_gemm")
    return (acc, y) if want_y else acc


SCAFFOLD_WORKSPACE_BYTES = 64 << 10   # DFSSM_SCAFFOLD_WORKSPACE_BYTES
SCAFFOLD_ERROR_OFFSET = 1024          # DFSSM_SCAFFOLD_ERROR_OFFSET
_scaffold_ws = {}


def scaffold_workspace(device) -> torch.Tensor:
    """The exchange workspace of dfssm_scaffold_lora_gemm for `device` (zeroed at allocation, one
    per device; calls on one device are ordered by torch's current stream)."""
    dev = torch.device(device)
    key = (dev.type, dev.index if dev.index is not None else torch.cuda.current_device())
    if key not in _scaffold_ws:
        _scaffold_ws[key] = torch.zeros(SCAFFOLD_WORKSPACE_BYTES // 4, dtype=torch.int32, device=dev)
    return _scaffold_ws[key]


def scaffold_error(workspace: torch.Tensor) -> int:
    """The workspace's error word (synchronizes): non-zero after a call whose wait timed out."""
    return int(workspace[SCAFFOLD_ERROR_OFFSET // 4].item())


def scaffold_lora_gemm(tiled_bits: torch.Tensor, wscale: torch.Tensor, q: torch.Tensor, xscale: torch.Tensor,
                       xn: torch.Tensor, lA: torch.Tensor, lA_s: torch.Tensor, lBq: torch.Tensor, N: int,
                       workspace="auto"):
    """One projection with its LoRA (dfssm_scaffold_lora_gemm): returns (acc int32 (M, N),
    y fp16 (M, N), lora_h fp16 (M, 16)). q (M, K) int8 with fp16 scales xscale (M,), xn (M, K) fp16,
    lA (N, 16) int8, lA_s (N,) fp16, lBq (16, K) fp16, wscale (N,) fp16. workspace: "auto" (the
    device's exchange workspace: one launch at M <= 4), None (no workspace) or an int32 tensor of
    SCAFFOLD_WORKSPACE_BYTES, zeroed before its first use."""
    _need(q, torch.int8, "q")
    _need(xn, torch.float16, "xn")
    _need(lBq, torch.float16, "lBq")
    _need(lA, torch.int8, "lA")
    M, K = q.shape
    if xn.shape != (M, K) or lBq.shape != (16, K) or lA.shape != (N, 16):
        raise ValueError("shape mismatch: q/xn (M, K), lBq (16, K), lA (N, 16)")
    acc = torch.empty(M, N, dtype=torch.int32, device=q.device)
    y = torch.empty(M, N, dtype=torch.float16, device=q.device)
    h = torch.empty(M, 16, dtype=torch.float16, device=q.device)
    if isinstance(workspace, str):
        if workspace != "auto":
            raise ValueError('workspace must be "auto", None or a tensor')
        workspace = scaffold_workspace(q.device)
    elif workspace is not None:
        _need(workspace, torch.int32, "workspace")
        if workspace.numel() * 4 < SCAFFOLD_WORKSPACE_BYTES:
            raise ValueError(f"workspace must hold {SCAFFOLD_WORKSPACE_BYTES} bytes")
    _C.check(_C.lib().dfssm_scaffold_lora_gemm(
        tiled_bits.data_ptr(), wscale.contiguous().data_ptr(), q.contiguous().data_ptr(),
        xscale.contiguous().data_ptr(), xn.contiguous().data_ptr(), lA.contiguous().data_ptr(),
        lA_s.contiguous().data_ptr(), lBq.contiguous().data_ptr(), M, N, K, h.data_ptr(), acc.data_ptr(),
        y.data_ptr(), _C.ptr(workspace), _C.stream()), "scaffold_lora_gemm")
    return acc, y, h


def rmsnorm_quantize(x: torch.Tensor, w: torch.Tensor):
    """x (M, K) fp16, w (K) fp32 -> (xn fp16 (M, K), q int8 (M, K), scale fp16 (M,))."""
    _need(x, torch.float16, "x")
    _need(w, torch.float32, "w")
    M, K = x.shape
    xn = torch.empty_like(x)
    q = torch.empty(M, K, dtype=torch.int8, device=x.device)
    s = torch.empty(M, dtype=torch.float16, device=x.device)
    _C.check(_C.lib().dfssm_rmsnorm_quantize(x.contiguous().data_ptr(), w.contiguous().data_ptr(), M, K,
                                             xn.data_ptr(), q.data_ptr(), s.data_ptr(), _C.stream()),
             "rmsnorm_quantize")
    return xn, q, s


def conv_step(conv_state: torch.Tensor, xbc: torch.Tensor, conv_w: torch.Tensor, conv_b: torch.Tensor) -> None:
    """In place: conv_state (B, C, 3) fp16 and xbc (B, C) fp16 (row stride honoured)."""
    for t, n in ((conv_state, "conv_state"), (xbc, "xBC"), (conv_w, "conv_weight"), (conv_b, "conv_bias")):
        _need(t, torch.float16, n)
    B, C = xbc.shape
    if conv_state.shape != (B, C, 3) or not conv_state.is_contiguous():
        raise ValueError(f"conv_state must be contiguous ({B}, {C}, 3)")
    if xbc.stride(1) != 1:
        raise ValueError("xBC rows must be contiguous")
    _C.check(_C.lib().dfssm_conv_step(conv_state.data_ptr(), xbc.data_ptr(), xbc.stride(0),
                                      conv_w.contiguous().data_ptr(), conv_b.contiguous().data_ptr(), B, C,
                                      _C.stream()), "conv_step")


def ssm_step(h: torch.Tensor, xbc: torch.Tensor, dt: torch.Tensor, dt_bias, A_log, D, y_out: torch.Tensor) -> None:
    """h (B, H, P, N) fp32 in place; xbc rows x|B|C fp16; dt (B, H) fp16; y_out (B, H*P) fp16."""
    _need(h, torch.float32, "h_state")
    _need(xbc, torch.float16, "xBC")
    _need(dt, torch.float16, "dt")
    _need(y_out, torch.float16, "y_out")
    for t, n in ((dt_bias, "dt_bias"), (A_log, "A_log"), (D, "D")):
        _need(t, torch.float32, n)
    B, H, P, N = h.shape
    if not h.is_contiguous() or xbc.stride(1) != 1 or dt.stride(1) != 1 or y_out.stride(1) != 1:
        raise ValueError("h_state must be contiguous and xBC / dt / y_out rows contiguous")
    _C.check(_C.lib().dfssm_ssm_step(h.data_ptr(), xbc.data_ptr(), xbc.stride(0), dt.data_ptr(), dt.stride(0),
                                     dt_bias.contiguous().data_ptr(), A_log.contiguous().data_ptr(),
                                     D.contiguous().data_ptr(), y_out.data_ptr(), y_out.stride(0),
                                     B, H, P, N, _C.stream()), "ssm_step")
