"""CPU oracle for the DF-SSM decode step -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module; the
product path (df-ssm_amd/) never does. It wraps oracle/liboracle.so (dfssm_oracle.c, the plain-C
restatement) and chains its steps into a whole decode step with the dataflow of the reference:

  GPU-reference numerics (OracleModel):   df_ssm_inference.py:160-224, 234-236
  CPU-reference numerics (OracleCPUModel): cpu_inference.c:303-376 + cpu_inference_driver.py:159-204

Which check pins which function (each test named in tests/):
  unpack bits              known answers from export_dfssm.py:34-42 + pack/unpack round trip
                           (test_oracle_pins.py::test_bit_order_*)
  scaffold accumulators    brute-force numpy int64 dot on random and extreme inputs, and the
                           compiled reference scaffold_matvec_avx512 driven with integer inputs
                           (test_oracle_pins.py::test_scaffold_*)
  fp16 conversion          exhaustive against numpy float16 (test_oracle_pins.py::test_f2h_*)
  quantizer, rmsnorm,      torch CPU evaluating the reference's own tensor expressions in fp16
  gate, LoRA, dequant      (test_oracle_pins.py::test_*_vs_torch)
  conv, SSM, rms_norm,     compiled reference static functions (oracle/_ref, HEADDIM=64) and
  gate_norm, lora, layer   layer_forward (test_oracle_vs_reference.py); closed forms for the SSM
                           (B=0 decay, x=0 readout, D skip)
  LM head + argmax         float64 matmul + numpy argmax first-index rule (test_oracle_pins.py)
  sampling (or_sample)     top_p = 0 equals the argmax of the penalized logits; the kept set
                           against a float64 NumPy evaluation of the reference's sort/cumsum
                           drop rule (gen_test.py:76-80) on logits with separated masses; the
                           penalty modes against their closed forms; the draw frequencies
                           against softmax over the kept set (chi-square); the inverse-CDF
                           draw against a NumPy restatement (test_sampling.py)
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import List, Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

LORA_R = 16


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run `make -C oracle` (or __graft_entry__.build())")
        _LIB = ctypes.CDLL(path)
    return _LIB


def _p(a: Optional[np.ndarray]):
    if a is None:
        return ctypes.c_void_p(0)
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("oracle arguments must be C-contiguous")
    # data_as keeps a reference to the array, so temporaries live until the call returns
    return a.ctypes.data_as(ctypes.c_void_p)


def _pv(a: np.ndarray, byte_offset: int = 0):
    """Pointer into a (possibly row-strided) view; keeps the view alive for the call."""
    if byte_offset == 0:
        return a.ctypes.data_as(ctypes.c_void_p)
    return ctypes.c_void_p(a.ctypes.data + byte_offset)


def _h(a: np.ndarray) -> np.ndarray:
    """fp16 array -> its uint16 view (contiguous)."""
    a = np.ascontiguousarray(a)
    assert a.dtype == np.float16, a.dtype
    return a.view(np.uint16)


# ---------------------------------------------------------------- step wrappers ----------------

def f2h(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f2h_array(_p(x), _p(out), ctypes.c_long(x.size))
    return out.view(np.float16)


def unpack_bits(packed: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint32)
    rows, kw = packed.shape
    out = np.empty((rows, kw * 32), np.int8)
    lib().or_unpack_bits(_p(packed), rows, kw, _p(out))
    return out


def scaffold_acc(bits: np.ndarray, q: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint32)
    q = np.ascontiguousarray(q, dtype=np.int8)
    M, K = q.shape
    N = bits.shape[0]
    assert bits.shape[1] * 32 == K
    acc = np.empty((M, N), np.int32)
    lib().or_scaffold_acc(_p(bits), _p(q), M, N, K, _p(acc))
    return acc


def rmsnorm(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    xh = _h(x)
    M, K = xh.shape
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty((M, K), np.uint16)
    lib().or_rmsnorm(_p(xh), _p(w), M, K, _p(out))
    return out.view(np.float16)


def quantize(xn: np.ndarray):
    xh = _h(xn)
    M, K = xh.shape
    q = np.empty((M, K), np.int8)
    s = np.empty(M, np.uint16)
    lib().or_quantize(_p(xh), M, K, _p(q), _p(s))
    return q, s.view(np.float16)


def lora_h(xn: np.ndarray, lB: np.ndarray, lBs: np.ndarray) -> np.ndarray:
    xh = _h(xn)
    M, K = xh.shape
    h = np.empty((M, LORA_R), np.uint16)
    lib().or_lora_h(_p(xh), _p(np.ascontiguousarray(lB)), _p(_h(lBs)), M, K, _p(h))
    return h.view(np.float16)


def dequant_lora(acc, xs, ws, h16, lA, lAs) -> np.ndarray:
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    M, N = acc.shape
    out = np.empty((M, N), np.uint16)
    lib().or_dequant_lora(_p(acc), _p(_h(xs)), _p(_h(ws)), _p(_h(h16)), _p(np.ascontiguousarray(lA)),
                          _p(_h(lAs)), M, N, _p(out))
    return out.view(np.float16)


def projection(xn: np.ndarray, bits, ws, lA, lAs, lB, lBs, return_acc: bool = False):
    """Quantize -> scaffold -> dequant -> LoRA: in_proj / out_proj (df_ssm_inference.py:168-173)."""
    q, xs = quantize(xn)
    acc = scaffold_acc(bits, q)
    h16 = lora_h(xn, lB, lBs)
    out = dequant_lora(acc, xs, ws, h16, lA, lAs)
    if return_acc:
        return out, dict(q=q, xs=xs, acc=acc, h16=h16)
    return out


def conv_step(state: np.ndarray, xbc: np.ndarray, w: np.ndarray, b: np.ndarray) -> None:
    """In place on `state` (M, C, 3) fp16 and `xbc` (M, C) fp16 (may be a row-strided view)."""
    assert state.dtype == np.float16 and state.flags["C_CONTIGUOUS"]
    M, C = xbc.shape
    assert xbc.dtype == np.float16 and xbc.strides[1] == 2
    ld = xbc.strides[0] // 2
    lib().or_conv_step(_p(state), _pv(xbc), ld, _p(_h(w)), _p(_h(b)), M, C)


def ssm_step(h: np.ndarray, xbc: np.ndarray, dt_raw: np.ndarray, dt_bias, A_log, Dp) -> np.ndarray:
    """h (M, H, P, N) fp32 updated in place; returns y (M, H*P) fp16."""
    assert h.dtype == np.float32 and h.flags["C_CONTIGUOUS"]
    M, H, P, N = h.shape
    assert xbc.strides[1] == 2 and dt_raw.strides[1] == 2
    y = np.empty((M, H * P), np.uint16)
    lib().or_ssm_step(_p(h), _pv(xbc), xbc.strides[0] // 2,
                      _pv(dt_raw), dt_raw.strides[0] // 2,
                      _p(np.ascontiguousarray(dt_bias, np.float32)), _p(np.ascontiguousarray(A_log, np.float32)),
                      _p(np.ascontiguousarray(Dp, np.float32)), M, H, P, N, _p(y))
    return y.view(np.float16)


def gate(y: np.ndarray, z: np.ndarray) -> np.ndarray:
    yh = _h(y)
    M, DI = yh.shape
    assert z.strides[1] == 2
    g = np.empty((M, DI), np.uint16)
    lib().or_gate(_p(yh), _pv(z), z.strides[0] // 2, M, DI, _p(g))
    return g.view(np.float16)


def residual(x: np.ndarray, o: np.ndarray) -> None:
    assert x.flags["C_CONTIGUOUS"] and x.dtype == np.float16
    M, D = x.shape
    lib().or_residual(_p(x), _p(_h(o)), M, D)


def embed(w, tokens: np.ndarray) -> np.ndarray:
    tok = np.ascontiguousarray(tokens, dtype=np.int64)
    M, D = tok.shape[0], w.cfg.d_model
    x = np.empty((M, D), np.uint16)
    if w.cfg.emb_code:
        lib().or_embed(_p(w.emb), _p(_h(w.emb_scale)), None, 1, _p(tok), M, D, _p(x))
    else:
        lib().or_embed(None, None, _p(_h(w.emb)), 0, _p(tok), M, D, _p(x))
    return x.view(np.float16)


def lm_head(w, xf: np.ndarray):
    """Returns (logits fp16 (M, V), next int64 (M,))."""
    xh = _h(xf)
    M, D = xh.shape
    V = w.cfg.vocab_size
    logits = np.empty((M, V), np.uint16)
    nxt = np.empty(M, np.int64)
    if w.cfg.emb_code:
        lib().or_lm_head(_p(xh), _p(w.emb), _p(_h(w.emb_scale)), None, 1, M, V, D, _p(logits), _p(nxt))
    else:
        lib().or_lm_head(_p(xh), None, None, _p(_h(w.emb)), 0, M, V, D, _p(logits), _p(nxt))
    return logits.view(np.float16), nxt


def sample(logits16: np.ndarray, counts: np.ndarray, step: np.ndarray, temperature: float, top_p: float,
           penalty: float, mode: int, seed: int, want_kept: bool = False):
    """The sampling head's definition (or_sample). counts (M, V) int32 and step (M) uint32 are
    updated in place as the kernel does. Returns next (M,) int64 [, kept (M, V) bool]."""
    lg = _h(logits16)
    M, V = lg.shape
    assert counts.dtype == np.int32 and counts.flags["C_CONTIGUOUS"] and counts.shape == (M, V)
    assert step.dtype == np.uint32 and step.flags["C_CONTIGUOUS"] and step.shape == (M,)
    nxt = np.empty(M, np.int64)
    kept = np.empty((M, V), np.uint8) if want_kept else None
    f = lib().or_sample
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                  ctypes.c_float, ctypes.c_float, ctypes.c_int, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p]
    f(_p(lg), _p(counts), _p(step), M, V, temperature, top_p, penalty, mode, seed, _p(nxt), _p(kept))
    return (nxt, kept.astype(bool)) if want_kept else nxt


# ---------------------------------------------------------------- whole model -------------------

def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class OracleModel:
    """Decode step with the GPU-reference numerics; batch rows are independent sequences.

    State: h (L, B, H, P, N) fp32 and conv (L, B, C, 3) fp16, zero after reset_state()
    (df_ssm_inference.py:112-139, fp32 SSM state per the benchmark configuration).
    """

    def __init__(self, weights, batch: int):
        self.w = weights
        self.cfg = c = weights.cfg
        if c.ngroups != 1:
            raise NotImplementedError("oracle supports ngroups=1")
        self.B = batch
        self.h = np.zeros((c.n_layer, batch, c.nheads, c.p, c.d_state), np.float32)
        self.conv = np.zeros((c.n_layer, batch, c.d_xbc, 3), np.float16)
        self.x = None

    def reset_state(self):
        self.h[...] = 0
        self.conv[...] = 0

    def layer(self, li: int, x: np.ndarray, trace: Optional[dict] = None) -> None:
        """One layer of _run_layers (df_ssm_inference.py:161-207); x (B, D) fp16 updated in place."""
        c, L = self.cfg, self.w.layers[li]
        DI, C, H = c.d_inner, c.d_xbc, c.nheads
        xn = rmsnorm(x, _f32(L["ln_w"]))
        proj, aux = projection(xn, L["in_packed"], L["in_scale"], L["in_lA"], L["in_lA_s"],
                               L["in_lB"], L["in_lB_s"], return_acc=True)
        z = proj[:, :DI]
        xbc = proj[:, DI:DI + C]
        dt_raw = proj[:, DI + C:DI + C + H]
        conv_state = np.ascontiguousarray(self.conv[li])
        conv_step(conv_state, xbc, L["conv_w"], L["conv_b"])
        self.conv[li] = conv_state
        h = np.ascontiguousarray(self.h[li])
        y = ssm_step(h, xbc, dt_raw, L["dt_bias"], L["A_log"], L["D"])
        self.h[li] = h
        g = gate(y, z)
        yn = rmsnorm(g, _f32(L["norm_w"]))
        out, aux2 = projection(yn, L["out_packed"], L["out_scale"], L["out_lA"], L["out_lA_s"],
                               L["out_lB"], L["out_lB_s"], return_acc=True)
        residual(x, out)
        if trace is not None:
            trace.update(xn=xn, q_in=aux["q"], xs_in=aux["xs"], acc_in=aux["acc"], proj=proj, y=y, g=g,
                         yn=yn, q_out=aux2["q"], xs_out=aux2["xs"], acc_out=aux2["acc"], out=out,
                         x=x.copy())

    def step(self, tokens: np.ndarray, traces: Optional[List[dict]] = None):
        """forward(token_ids) (df_ssm_inference.py:219-224) + greedy argmax (:236)."""
        x = np.ascontiguousarray(embed(self.w, tokens))
        for li in range(self.cfg.n_layer):
            t = {} if traces is not None else None
            self.layer(li, x, t)
            if traces is not None:
                traces.append(t)
        xf = rmsnorm(x, _f32(self.w.norm_f))
        logits, nxt = lm_head(self.w, xf)
        self.x = x
        return logits, nxt

    def generate(self, prompts: np.ndarray, n_new: int, keep_logits: bool = False):
        """Consume `prompts` (B, T) step by step, then decode greedily: T + n_new - 1 steps.

        Returns (generated (B, n_new) int64, list of per-step logits if keep_logits). generated[:, 0]
        is the argmax after the last prompt token; generated[:, i] is fed to step T + i.
        """
        B, T = prompts.shape
        assert B == self.B
        self.reset_state()
        all_logits = []
        nxt = None
        for t in range(T):
            logits, nxt = self.step(prompts[:, t])
            if keep_logits:
                all_logits.append(logits)
        out = np.empty((B, n_new), np.int64)
        for i in range(n_new):
            out[:, i] = nxt
            if i + 1 < n_new:            # the last greedy token is recorded, not consumed
                logits, nxt = self.step(out[:, i])
                if keep_logits:
                    all_logits.append(logits)
        return out, all_logits


# ---------------------------------------------------------------- CPU-reference numerics --------

def c_scaffold(bits, x, scale):
    x = _f32(np.atleast_2d(x))
    M, K = x.shape
    N = bits.shape[0]
    out = np.empty((M, N), np.float32)
    lib().or_c_scaffold(_p(np.ascontiguousarray(bits, np.uint32)), _p(x), _p(_f32(scale)), M, N, K, _p(out))
    return out


def c_lora(A, As, B, Bs, x, out):
    x = _f32(np.atleast_2d(x))
    M, K = x.shape
    N = A.shape[0]
    assert out.flags["C_CONTIGUOUS"] and out.dtype == np.float32 and out.shape == (M, N)
    lib().or_c_lora(_p(np.ascontiguousarray(A)), _p(_f32(As)), _p(np.ascontiguousarray(B)), _p(_f32(Bs)),
                    _p(x), _p(out), M, N, K)


class OracleCPUModel:
    """Single-sequence decode with the CPU-reference numerics (cpu_inference.c + driver).

    Mirrors CPUModel (cpu_inference_driver.py:77-204): fp32 activations and state, the embedding
    as an fp32 table (for the int8 variant: fp32(E_i8 * s_E), i.e. the fp16 table the GPU path
    gathers, widened), layer_forward per layer, final_rms_norm, fp32 head, argmax.
    """

    def __init__(self, weights):
        self.w = weights
        c = self.cfg = weights.cfg
        self.h = np.zeros((c.n_layer, c.nheads, c.p, c.d_state), np.float32)
        self.conv = np.zeros((c.n_layer, c.d_xbc, 3), np.float32)
        self.emb32 = weights.emb_f16().astype(np.float32)

    def reset_state(self):
        self.h[...] = 0
        self.conv[...] = 0

    def layer(self, li: int, x: np.ndarray) -> None:
        c, L = self.cfg, self.w.layers[li]
        D, DI, C, H, P, N = c.d_model, c.d_inner, c.d_xbc, c.nheads, c.p, c.d_state
        lb = lib()
        xn = np.empty((1, D), np.float32)
        lb.or_c_rms_norm(_p(x), _p(_f32(L["ln_w"])), _p(xn), 1, D)
        proj = c_scaffold(L["in_packed"], xn, L["in_scale"])
        c_lora(L["in_lA"], L["in_lA_s"], L["in_lB"], L["in_lB_s"], xn, proj)
        conv = np.ascontiguousarray(self.conv[li])
        lb.or_c_conv(_p(conv), _pv(proj, 4 * DI), proj.shape[1],
                     _p(_f32(L["conv_w"])), _p(_f32(L["conv_b"])), 1, C)
        self.conv[li] = conv
        h = np.ascontiguousarray(self.h[li])
        y = np.empty((1, DI), np.float32)
        lb.or_c_ssm(_p(h), _pv(proj, 4 * DI), proj.shape[1],
                    _pv(proj, 4 * (DI + C)), proj.shape[1],
                    _p(_f32(L["dt_bias"])), _p(_f32(L["A_log"])), _p(_f32(L["D"])), 1, H, P, N, _p(y))
        self.h[li] = h
        g = np.empty((1, DI), np.float32)
        lb.or_c_gate_norm(_p(y), _p(proj), proj.shape[1], _p(_f32(L["norm_w"])), _p(g), 1, DI)
        out = c_scaffold(L["out_packed"], g, L["out_scale"])
        c_lora(L["out_lA"], L["out_lA_s"], L["out_lB"], L["out_lB_s"], g, out)
        x += out[0]

    def step(self, token: int):
        c = self.cfg
        x = self.emb32[token].copy()
        for li in range(c.n_layer):
            self.layer(li, x)
        xf = np.empty(c.d_model, np.float32)
        lib().or_c_rms_norm(_p(x), _p(_f32(self.w.norm_f)), _p(xf), 1, c.d_model)
        logits = xf @ self.emb32.T
        return logits, int(np.argmax(logits))


def state_density_field(h: np.ndarray, thresholds: np.ndarray, sd_error: Optional[np.ndarray] = None,
                        sd_bits: int = 8):
    """or_state_df on a copy: (rows, 128) fp32 state (and sigma-delta error) after the chunk-
    boundary quantization of df_ssd_scan (training/df_ssm_mamba2_distill_dfw.py:139-165) with the
    bank's sorted thresholds. Returns (h, sd_error or None)."""
    h = np.ascontiguousarray(h, np.float32).reshape(-1, 128).copy()
    e = None if sd_error is None else np.ascontiguousarray(sd_error, np.float32).reshape(-1, 128).copy()
    R = np.ascontiguousarray(thresholds, np.float32).reshape(-1)
    f = lib().or_state_df
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_long, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    f.restype = None
    f(h.ctypes.data, None if e is None else e.ctypes.data, h.shape[0], R.ctypes.data, R.size, sd_bits)
    return h, e
