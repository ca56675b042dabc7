"""ctypes binding of libdfssm_hip.so (declarations: include/dfssm.h).

Only plain pointers, sizes and the stream cross the boundary; torch tensors are unpacked here
with data_ptr() and torch.cuda.current_stream().cuda_stream, so every launch lands on the
caller's current stream and can be captured into a HIP graph. There is no fallback: if the
library is missing or a call fails, an exception is raised.
"""
from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libdfssm_hip.so")

c_int, c_void_p, c_size_t = ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t
P = ctypes.c_void_p


class DFSSMError(RuntimeError):
    pass


class Dims(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("n_layer", "d_model", "d_inner", "d_state", "nheads", "headdim", "ngroups",
                 "vocab_size", "batch", "emb_code")]


LAYER_FIELDS = ("in_bits", "in_scale", "in_lA", "in_lA_s", "in_lB", "in_lB_s",
                "out_bits", "out_scale", "out_lA", "out_lA_s", "out_lB", "out_lB_s",
                "conv_w", "conv_b", "A_log", "D", "dt_bias", "norm_w", "ln_w", "in_lBq", "out_lBq")


class Layer(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in LAYER_FIELDS]


class Model(ctypes.Structure):
    _fields_ = [("dims", Dims), ("layers", ctypes.POINTER(Layer)), ("emb", c_void_p),
                ("emb_scale", c_void_p), ("norm_f", c_void_p)]


class State(ctypes.Structure):
    _fields_ = [("h", c_void_p), ("conv", c_void_p)]


class SampleParams(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_p", ctypes.c_float), ("penalty", ctypes.c_float),
                ("mode", ctypes.c_int32), ("seed", ctypes.c_uint64)]


_SIGS = {
    "dfssm_version": (c_int, []),
    "dfssm_error_string": (ctypes.c_char_p, [c_int]),
    "dfssm_check_dims": (c_int, [ctypes.POINTER(Dims)]),
    "dfssm_one_launch_plan": (c_int, [ctypes.POINTER(Dims), c_int, c_int]),
    "dfssm_set_layer_kernel": (c_int, [c_int]),
    "dfssm_tiled_bits_bytes": (c_size_t, [c_int, c_int]),
    "dfssm_tiled_emb_bytes": (c_size_t, [c_int, c_int]),
    "dfssm_tile_bits": (c_int, [P, P, c_int, c_int, P]),
    "dfssm_tile_embedding": (c_int, [P, P, c_int, c_int, P]),
    "dfssm_dequant_lora_b": (c_int, [P, P, c_int, P, P]),
    "dfssm_scaffold_gemm": (c_int, [P, P, P, P, c_int, c_int, c_int, P, P, P]),
    "dfssm_scaffold_lora_gemm": (c_int, [P, P, P, P, P, P, P, P, c_int, c_int, c_int, P, P, P, P, P]),
    "dfssm_rmsnorm_quantize": (c_int, [P, P, c_int, c_int, P, P, P, P]),
    "dfssm_conv_step": (c_int, [P, P, c_int, P, P, c_int, c_int, P]),
    "dfssm_ssm_step": (c_int, [P, P, c_int, P, c_int, P, P, P, P, c_int, c_int, c_int, c_int, c_int, P]),
    "dfssm_workspace_bytes": (c_size_t, [ctypes.POINTER(Dims)]),
    "dfssm_workspace_init": (c_int, [ctypes.POINTER(Dims), P, P]),
    "dfssm_workspace_error_flag": (P, [ctypes.POINTER(Dims), P]),
    "dfssm_embed": (c_int, [ctypes.POINTER(Model), P, P, P, P]),
    "dfssm_layer_step": (c_int, [ctypes.POINTER(Model), c_int, P, ctypes.POINTER(State), P, P]),
    "dfssm_layer_phase": (c_int, [ctypes.POINTER(Model), c_int, c_int, P, ctypes.POINTER(State), P, P]),
    "dfssm_lmhead_argmax": (c_int, [ctypes.POINTER(Model), P, P, P, P, P, P]),
    "dfssm_decode_step": (c_int, [ctypes.POINTER(Model), P, P, ctypes.POINTER(State), P, P, P, c_int, P]),
    "dfssm_decode_step_static": (c_int, [ctypes.POINTER(Model), P, P, ctypes.POINTER(State), P, P, c_int, P, P]),
    "dfssm_state_density_field": (c_int, [P, P, ctypes.c_int64, c_int, P, c_int, c_int, P]),
    "dfssm_sample": (c_int, [ctypes.POINTER(Model), P, P, P, ctypes.POINTER(SampleParams), P, P, P, P]),
    "dfssm_prefill_workspace_bytes": (c_size_t, [ctypes.POINTER(Dims), c_int]),
    "dfssm_prefill": (c_int, [ctypes.POINTER(Model), P, c_int, P, ctypes.POINTER(State), P, P, c_int, P, P,
                              c_int, P]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Load the HIP library (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise DFSSMError(f"{LIB_PATH} not found: build it with `python -m dfssm.build` "
                             "or __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    return list(_SIGS)


# return codes and layer phases of include/dfssm.h used from Python
DFSSM_E_DIMS = -2
PHASE_SSM_PROLOGUE = 5   # DFSSM_PHASE_SSM_PROLOGUE
PHASE_OUT_PROLOGUE = 6   # DFSSM_PHASE_OUT_PROLOGUE


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = lib().dfssm_error_string(rc).decode()
        raise DFSSMError(f"{what}: {msg} (code {rc})")


def ptr(t) -> int:
    """Device pointer of a torch tensor (or 0 for None)."""
    return 0 if t is None else t.data_ptr()


def stream() -> int:
    import torch
    return torch.cuda.current_stream().cuda_stream
