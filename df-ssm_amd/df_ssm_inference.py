"""
DF-SSM decode on MI355X: the drop-in for the reference's inference/gpu/df_ssm_inference.py.

Same surface as the reference (df_ssm_inference.py:47-252):
    DFSSMModel(path, device="cuda", batch_size=1)
    .reset_state()
    .forward(token_ids) -> fp16 logits (batch, vocab)     (advances the state by one token)
    .generate(n_tokens=128)                              (prints timing like the reference)
    python df_ssm_inference.py model.dfssm --batch_size B --n_tokens N

What runs underneath is different: the scaffold stays 1 bit per weight in HBM (re-tiled, not
unpacked to int8), every layer is one hand-written gfx950 kernel launch at batch <= 4 (five at larger
batches) behind the C ABI of
libdfssm_hip.so (include/dfssm.h), the SSM state is fp32, the tied head is the int8 table with
a fused greedy argmax, and a whole decode step (embedding, all layers, head) is one HIP graph.
Compatible extensions: generate(n_tokens, prompt=None, return_tokens=False, verbose=True) ingests
a (batch, T) prompt step by step and does not leave warm-up state behind (the reference's warm-up
forward advances the state, df_ssm_inference.py:230; the CPU driver resets after it,
cpu_inference_driver.py:191-192).
"""
from __future__ import annotations

import ctypes
import os
import sys
import time
from typing import List, Optional

import numpy as np
import torch

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from dfssm import _C  # noqa: E402
from dfssm.format import DFSSMWeights, EMB_I8, LORA_RANK, read_dfssm  # noqa: E402


def _untile_signs(tiled: torch.Tensor, rows: int, k: int) -> torch.Tensor:
    """(rows, k) int8 +-1 matrix from the tiled sign bits of dfssm_tile_bits
    ([rows_pad/64][k/128][64 rows][4 words], word h of chunk c = columns 128c + 32h .. + 31, bit b =
    column + b, 1 = +1) -- the matrix the reference unpacks at load (df_ssm_inference.py:23-29)."""
    rp = (rows + 63) // 64 * 64
    words = tiled.view(rp // 64, k // 128, 64, 4).permute(0, 2, 1, 3).reshape(rp, k // 32)[:rows]
    words = words.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(32, device=tiled.device, dtype=torch.int64)
    bits = (words[:, :, None] >> shifts) & 1                     # (rows, k/32, 32): column 32j + b
    return (2 * bits - 1).to(torch.int8).reshape(rows, k)


class LayerWeights:
    """Device tensors of one layer, with the reference's LayerWeights attributes
    (df_ssm_inference.py:32-44, built at :70-98): in_scale / out_scale, conv_weight, conv_bias,
    A_log, D, dt_bias, norm_weight, layer_norm_weight as stored; in_w_T / out_w_T ((K, N) int8 +-1,
    pre-transposed) and the fp16-dequantized in_lora_A (N, 16), in_lora_B (16, K), out_lora_A,
    out_lora_B are read-only views built on first access (the kernels never read them).
    What the kernels read: the scaffold as tiled sign bits (in_bits / out_bits, 1 bit per weight),
    the LoRA factors as stored in the file (int8 in_lA / in_lB with fp16 row scales in_lA_s /
    in_lB_s, likewise out_*), and the load-time fp16 LoRA-B tables in_lora_Bq / out_lora_Bq."""
    __slots__ = (
        "in_bits", "in_scale", "out_bits", "out_scale",
        "in_lA", "in_lA_s", "in_lB", "in_lB_s",
        "out_lA", "out_lA_s", "out_lB", "out_lB_s",
        "conv_weight", "conv_bias", "A_log", "D", "dt_bias",
        "norm_weight", "layer_norm_weight", "in_lora_Bq", "out_lora_Bq",
        "dims", "_compat",
    )

    def _view(self, name, build):
        if self._compat is None:
            self._compat = {}
        if name not in self._compat:
            self._compat[name] = build()
        return self._compat[name]

    @property
    def in_w_T(self) -> torch.Tensor:
        """(d_model, in_proj_out) int8 +-1: the reference's in_w_T (df_ssm_inference.py:72-74)."""
        D, IPO = self.dims[0], self.dims[2]
        return self._view("in_w_T", lambda: _untile_signs(self.in_bits, IPO, D).t().contiguous())

    @property
    def out_w_T(self) -> torch.Tensor:
        """(d_inner, d_model) int8 +-1: the reference's out_w_T (df_ssm_inference.py:87-89)."""
        D, DI = self.dims[0], self.dims[1]
        return self._view("out_w_T", lambda: _untile_signs(self.out_bits, D, DI).t().contiguous())

    @staticmethod
    def _deq(a: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
        return (a.float() * s.float().unsqueeze(1)).half()

    @property
    def in_lora_A(self) -> torch.Tensor:
        """(in_proj_out, 16) fp16 = (lA * lA_s).half(), df_ssm_inference.py:82."""
        return self._view("in_lora_A", lambda: self._deq(self.in_lA, self.in_lA_s))

    @property
    def in_lora_B(self) -> torch.Tensor:
        """(16, d_model) fp16 = (lB * lB_s).half(), df_ssm_inference.py:83 (the table the kernels
        read, in_lora_Bq)."""
        return self.in_lora_Bq

    @property
    def out_lora_A(self) -> torch.Tensor:
        """(d_model, 16) fp16, df_ssm_inference.py:96."""
        return self._view("out_lora_A", lambda: self._deq(self.out_lA, self.out_lA_s))

    @property
    def out_lora_B(self) -> torch.Tensor:
        """(16, d_inner) fp16, df_ssm_inference.py:97 (= out_lora_Bq)."""
        return self.out_lora_Bq


def _require_gpu(device) -> torch.device:
    dev = torch.device(device)
    if dev.type != "cuda" or not torch.cuda.is_available():
        raise RuntimeError("DFSSMModel runs only on an MI355X GPU (torch.cuda / HIP device); "
                           f"got device={device!r}, cuda available={torch.cuda.is_available()}")
    _C.lib()  # fail loudly if the HIP library is missing
    return dev


def _dev(a: np.ndarray, dev) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    elif a.dtype == np.float16:
        return torch.from_numpy(a.view(np.int16)).to(dev).view(torch.float16)
    return torch.from_numpy(a).to(dev)


# Bits of the workspace error flag (include/dfssm.h DFSSM_ERR_*; set by the kernels, read and
# cleared by DFSSMModel). Each bounded wait between workgroups has its own bit, named for the
# launch whose wait gave up.
ERR_TOKEN_RANGE = 1          # a token id outside [0, vocab) reached the embedding gather (row 0 was used)
ERR_WAIT_LAYER = 4           # the one-launch layer (batch <= 4)
ERR_WAIT_SSM_PROLOGUE = 8    # the SSM + out_proj-prologue launch (batch >= 5)
ERR_WAIT_OUT_PROLOGUE = 16   # the out_proj + next-layer-prologue launch (batch >= 5)

_WAIT_CAUSE = ("(its workgroups were not all running at once, e.g. because another process or stream "
               "shared the GPU, or a workgroup it waited for failed)")


def describe_error_flag(flag: int) -> str:
    """Human-readable causes of a nonzero workspace error flag."""
    causes = []
    if flag & ERR_TOKEN_RANGE:
        causes.append("token id out of range [0, vocab) in a device token tensor (embedding row 0 was used)")
    if flag & ERR_WAIT_LAYER:
        causes.append("a wait between workgroups of the one-launch layer (batch <= 4) timed out " + _WAIT_CAUSE)
    if flag & ERR_WAIT_SSM_PROLOGUE:
        causes.append("a wait of the SSM + gated-norm prologue launch (batch >= 5) timed out " + _WAIT_CAUSE)
    if flag & ERR_WAIT_OUT_PROLOGUE:
        causes.append("a wait of the out_proj + next-layer prologue launch (batch >= 5) timed out " + _WAIT_CAUSE)
    rest = flag & ~(ERR_TOKEN_RANGE | ERR_WAIT_LAYER | ERR_WAIT_SSM_PROLOGUE | ERR_WAIT_OUT_PROLOGUE)
    if rest:
        causes.append(f"unknown error bits {rest:#x}")
    return "; ".join(causes)


def _check_token_range(t: torch.Tensor, vocab: int) -> None:
    """Raise IndexError unless every id of t is in [0, vocab); on a device tensor this syncs."""
    if t.numel() == 0:
        return
    lo, hi = int(t.min()), int(t.max())
    if lo < 0 or hi >= vocab:
        raise IndexError(f"token id out of range [0, {vocab}): min {lo}, max {hi}")


class StateDensityField:
    """Density-field state at inference (df_ssd_scan, training/df_ssm_mamba2_distill_dfw.py:114-173):
    thresholds (num_banks, K*K) per-bank sorted thresholds (SprayBank.thresholds, :79-91; rows are
    sorted here), block_len the chunk length, sigma_delta and sd_bits as DensityFieldConfig
    (:96-103)."""

    def __init__(self, thresholds, block_len: int = 64, sigma_delta: bool = True, sd_bits: int = 8):
        t = np.sort(np.asarray(thresholds, np.float32), axis=-1)
        if t.ndim != 2 or not 1 <= t.shape[1] <= 1024:
            raise ValueError("thresholds must be (num_banks, K*K) with K*K <= 1024")
        if block_len < 1 or sd_bits < 1:
            raise ValueError("block_len and sd_bits must be >= 1")
        self.thresholds = np.ascontiguousarray(t)
        self.block_len, self.sigma_delta, self.sd_bits = int(block_len), bool(sigma_delta), int(sd_bits)
        self._dev = {}

    @classmethod
    def random(cls, K: int = 8, num_banks: int = 256, seed: int = 0, **kw):
        """Bank of uniform sorted thresholds, as SprayBank.__init__ draws them (torch.rand)."""
        g = torch.Generator().manual_seed(seed)
        return cls(torch.rand(num_banks, K * K, generator=g).numpy(), **kw)

    def device_thresholds(self, device) -> torch.Tensor:
        key = str(device)
        if key not in self._dev:
            self._dev[key] = torch.from_numpy(self.thresholds).to(device)
        return self._dev[key]


class DFSSMModel:
    def __init__(self, path, device="cuda", batch_size=1, weights: Optional[DFSSMWeights] = None):
        self.device = _require_gpu(device)
        self.batch_size = int(batch_size)
        self.layers: List[LayerWeights] = []
        w = weights if weights is not None else read_dfssm(path)
        self.cfg = w.cfg
        self._load(w)
        self._alloc_state()
        self._graph = None       # forward(): one decode step reading self._tok
        self._gen_graphs = {}    # generation: S fused steps per replay
        self._pos = 0

    @classmethod
    def from_weights(cls, weights: DFSSMWeights, device="cuda", batch_size=1):
        return cls(None, device=device, batch_size=batch_size, weights=weights)

    # ------------------------------------------------------------------ load
    def _tile_bits(self, packed: np.ndarray, rows: int, k: int, dst: torch.Tensor) -> None:
        src = _dev(packed, self.device)
        assert dst.numel() * 4 == _C.lib().dfssm_tiled_bits_bytes(rows, k)
        _C.check(_C.lib().dfssm_tile_bits(src.data_ptr(), dst.data_ptr(), rows, k, _C.stream()), "tile_bits")

    def _dequant_lora_b(self, B: torch.Tensor, Bs: torch.Tensor, k: int, out: torch.Tensor) -> None:
        _C.check(_C.lib().dfssm_dequant_lora_b(B.data_ptr(), Bs.data_ptr(), k, out.data_ptr(), _C.stream()),
                 "dequant_lora_b")

    def _load(self, w: DFSSMWeights):
        c = self.cfg
        dims = _C.Dims(c.n_layer, c.d_model, c.d_inner, c.d_state, c.nheads, c.p, c.ngroups,
                       c.vocab_size, self.batch_size, c.emb_code)
        rc = _C.lib().dfssm_check_dims(dims)
        if rc != 0:
            raise _C.DFSSMError(f"model {c} / batch {self.batch_size} not supported: "
                                f"{_C.lib().dfssm_error_string(rc).decode()}")
        self.dims = dims
        dev = self.device
        D, DI, IPO = c.d_model, c.d_inner, c.in_proj_out
        descs = (_C.Layer * c.n_layer)()
        # One allocation per field for all layers (layer l at a fixed stride), so that the decode
        # step can run every layer in one launch (dfssm_decode_step checks the strides).
        nL = c.n_layer

        def stacked(key, cast=None):
            return _dev(np.stack([cast(L[key]) if cast else L[key] for L in w.layers]), dev)

        in_bits = torch.empty(nL, _C.lib().dfssm_tiled_bits_bytes(IPO, D) // 4, dtype=torch.int32, device=dev)
        out_bits = torch.empty(nL, _C.lib().dfssm_tiled_bits_bytes(D, DI) // 4, dtype=torch.int32, device=dev)
        for li, L in enumerate(w.layers):
            self._tile_bits(L["in_packed"], IPO, D, in_bits[li])
            self._tile_bits(L["out_packed"], D, DI, out_bits[li])
        f32 = lambda a: a.astype(np.float32)
        fields = {
            "in_scale": stacked("in_scale"), "in_lA": stacked("in_lA"), "in_lA_s": stacked("in_lA_s"),
            "in_lB": stacked("in_lB"), "in_lB_s": stacked("in_lB_s"),
            "out_scale": stacked("out_scale"), "out_lA": stacked("out_lA"), "out_lA_s": stacked("out_lA_s"),
            "out_lB": stacked("out_lB"), "out_lB_s": stacked("out_lB_s"),
            "conv_w": stacked("conv_w"), "conv_b": stacked("conv_b"),
            "A_log": stacked("A_log"), "D": stacked("D"), "dt_bias": stacked("dt_bias"),
            "norm_w": stacked("norm_w", f32), "ln_w": stacked("ln_w", f32),
        }
        in_lBq = torch.empty(nL, LORA_RANK, D, dtype=torch.float16, device=dev)
        out_lBq = torch.empty(nL, LORA_RANK, DI, dtype=torch.float16, device=dev)
        for li in range(nL):
            self._dequant_lora_b(fields["in_lB"][li], fields["in_lB_s"][li], D, in_lBq[li])
            self._dequant_lora_b(fields["out_lB"][li], fields["out_lB_s"][li], DI, out_lBq[li])
        fields.update(in_bits=in_bits, out_bits=out_bits, in_lBq=in_lBq, out_lBq=out_lBq)
        self._stacked = fields
        for li in range(nL):
            F = {k: v[li] for k, v in fields.items()}
            lw = LayerWeights()
            lw.in_bits, lw.in_scale = F["in_bits"], F["in_scale"]
            lw.in_lA, lw.in_lA_s = F["in_lA"], F["in_lA_s"]
            lw.in_lB, lw.in_lB_s = F["in_lB"], F["in_lB_s"]
            lw.out_bits, lw.out_scale = F["out_bits"], F["out_scale"]
            lw.out_lA, lw.out_lA_s = F["out_lA"], F["out_lA_s"]
            lw.out_lB, lw.out_lB_s = F["out_lB"], F["out_lB_s"]
            lw.dims, lw._compat = (D, DI, IPO), None
            lw.conv_weight, lw.conv_bias = F["conv_w"], F["conv_b"]
            lw.A_log, lw.D, lw.dt_bias = F["A_log"], F["D"], F["dt_bias"]
            lw.norm_weight, lw.layer_norm_weight = F["norm_w"], F["ln_w"]
            lw.in_lora_Bq, lw.out_lora_Bq = F["in_lBq"], F["out_lBq"]
            self.layers.append(lw)
            d = descs[li]
            for field, t in F.items():
                setattr(d, field, t.data_ptr())
        # the table (int8 + row scale, or fp16 as the exporter writes it) re-tiled for the head
        row_bytes = D if c.emb_code == EMB_I8 else 2 * D
        emb_src = _dev(w.emb, dev)
        self.embedding_tiled = torch.empty(_C.lib().dfssm_tiled_emb_bytes(c.vocab_size, row_bytes),
                                           dtype=torch.int8, device=dev)
        _C.check(_C.lib().dfssm_tile_embedding(emb_src.data_ptr(), self.embedding_tiled.data_ptr(), c.vocab_size,
                                               row_bytes, _C.stream()), "tile_embedding")
        self._emb_view = None
        del emb_src
        self.embedding_scale = _dev(w.emb_scale, dev) if c.emb_code == EMB_I8 else None
        self.norm_f_weight = _dev(w.norm_f.astype(np.float32), dev)
        self._descs = descs
        self._model = _C.Model(dims, descs, self.embedding_tiled.data_ptr(),
                               self.embedding_scale.data_ptr() if self.embedding_scale is not None else None,
                               self.norm_f_weight.data_ptr())
        torch.cuda.synchronize(dev)

    @property
    def embedding(self) -> torch.Tensor:
        """The (vocab, d_model) fp16 table, as the reference's attribute (df_ssm_inference.py:65,
        used as norm_out @ embedding.T at :224). The kernels read a re-tiled copy
        (embedding_tiled, [V/64][row bytes/16][64 rows][16 B]); this row-major view is built from
        it on first access (a further vocab x d_model x 2 bytes of HBM). For an int8 table
        (format extension) it is fp16(E_i8 * row scale); the head itself computes
        fp16(fp32(sum_k xf_k E_i8[v, k]) * scale[v]), which may differ from xf @ embedding.T by
        the fp16 rounding of the table."""
        if self._emb_view is None:
            c = self.cfg
            rb = c.d_model if c.emb_code == EMB_I8 else 2 * c.d_model
            vp = (c.vocab_size + 63) // 64 * 64
            t = self.embedding_tiled.view(torch.uint8).view(vp // 64, rb // 16, 64, 16)
            rows = t.permute(0, 2, 1, 3).reshape(vp, rb)[:c.vocab_size].contiguous()
            if c.emb_code == EMB_I8:
                e = rows.view(torch.int8).float() * self.embedding_scale.float()[:, None]
                self._emb_view = e.half()
            else:
                self._emb_view = rows.view(torch.float16)
        return self._emb_view

    # ------------------------------------------------------------------ state
    def _alloc_state(self):
        c, B, d = self.cfg, self.batch_size, self.device
        self.h_state = torch.zeros(c.n_layer, B, c.nheads, c.p, c.d_state, dtype=torch.float32, device=d)
        self.conv_state = torch.zeros(c.n_layer, B, c.d_xbc, 3, dtype=torch.float16, device=d)
        self.h_states = [self.h_state[l] for l in range(c.n_layer)]        # reference attribute names
        self.conv_states = [self.conv_state[l] for l in range(c.n_layer)]
        self._state = _C.State(self.h_state.data_ptr(), self.conv_state.data_ptr())
        self.x = torch.zeros(B, c.d_model, dtype=torch.float16, device=d)
        self.logits = torch.empty(B, c.vocab_size, dtype=torch.float16, device=d)
        self._tok = torch.zeros(B, dtype=torch.int64, device=d)
        self._next = torch.zeros(B, dtype=torch.int64, device=d)
        nbytes = _C.lib().dfssm_workspace_bytes(self.dims)
        self.workspace = torch.empty(nbytes, dtype=torch.uint8, device=d)
        _C.check(_C.lib().dfssm_workspace_init(self.dims, self.workspace.data_ptr(), _C.stream()), "workspace_init")
        self._err = _C.lib().dfssm_workspace_error_flag(self.dims, self.workspace.data_ptr())
        # one eager head launch outside any capture (sets the kernel's LDS attribute)
        _C.check(_C.lib().dfssm_lmhead_argmax(self._model, self.x.data_ptr(), self.workspace.data_ptr(),
                                              self.logits.data_ptr(), self._next.data_ptr(), None,
                                              _C.stream()), "lmhead")
        torch.cuda.synchronize(d)

    def reset_state(self):
        self.h_state.zero_()
        self.conv_state.zero_()
        if getattr(self, "_df_err", None) is not None:
            self._df_err.zero_()

    # ------------------------------------------------------------------ density-field state
    def apply_state_density_field(self, df: "StateDensityField", chunk: int) -> None:
        """Quantize every layer's SSM state as df_ssd_scan does at the end of chunk `chunk`
        (training/df_ssm_mamba2_distill_dfw.py:139-165), with bank chunk % num_banks and, if
        df.sigma_delta, the sigma-delta error carried between chunks (zeroed by reset_state)."""
        R = df.device_thresholds(self.device)
        err = None
        if df.sigma_delta:
            if getattr(self, "_df_err", None) is None:
                self._df_err = torch.zeros_like(self.h_state)
            err = self._df_err
        bank = R[chunk % R.shape[0]]
        _C.check(_C.lib().dfssm_state_density_field(
            self.h_state.data_ptr(), None if err is None else err.data_ptr(), self.h_state.numel() // 128,
            self.cfg.d_state, bank.data_ptr(), R.shape[1], df.sd_bits, _C.stream()), "state_density_field")

    def _generate_state_df(self, n_tokens: int, prompt: torch.Tensor, df: "StateDensityField"):
        """Greedy decode with the density-field state: the prompt is prefilled in segments that
        end at chunk boundaries and the steps run in graphs that do not cross one; after the
        token at position t (from 0, prompt included) with (t + 1) % block_len == 0 the state
        is quantized with chunk index (t + 1) / block_len - 1."""
        L = df.block_len
        pos = 0

        def boundary():
            if pos % L == 0:
                self.apply_state_density_field(df, pos // L - 1)

        if self._graph is None:
            self._capture_graph()
        body = prompt[:, :-1]
        while pos < body.shape[1]:
            n = min(L - pos % L, body.shape[1] - pos)
            self.prefill(body[:, pos:pos + n])
            pos += n
            boundary()
        torch.cuda.synchronize(self.device)
        start = time.perf_counter()
        self._tok.copy_(prompt[:, -1])
        self._graph.replay()
        out = [self._next.clone()[:, None]]
        pos += 1
        boundary()
        done = 1
        while done < n_tokens:
            s = min(8, n_tokens - done, L - pos % L)
            g, hist = self._gen_graph(s)
            g.replay()
            out.append(hist.t().clone())
            done += s
            pos += s
            boundary()
        torch.cuda.synchronize(self.device)
        return torch.cat(out, dim=1)[:, :n_tokens], time.perf_counter() - start

    # ------------------------------------------------------------------ steps
    def _decode(self, tokens: Optional[torch.Tensor], logits: Optional[torch.Tensor], nxt: torch.Tensor, fuse: bool):
        _C.check(_C.lib().dfssm_decode_step(
            self._model, None if tokens is None else tokens.data_ptr(), self.x.data_ptr(), self._state,
            self.workspace.data_ptr(), None if logits is None else logits.data_ptr(), nxt.data_ptr(),
            1 if fuse else 0, _C.stream()), "decode_step")

    def decode_step_eager(self, token_ids: Optional[torch.Tensor] = None, want_logits: bool = True):
        """One decode step without graphs (tests, debugging). Returns (logits or None, next)."""
        if token_ids is not None:
            self._tok.copy_(token_ids.view(-1).to(self.device, torch.int64))
        self._decode(self._tok if token_ids is not None else None,
                     self.logits if want_logits else None, self._next, fuse=True)
        return (self.logits if want_logits else None), self._next

    def _capture(self, fn):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        return g

    def _capture_graph(self):
        self._graph = self._capture(lambda: self._decode(self._tok, self.logits, self._next, fuse=True))

    def forward(self, token_ids):
        """token_ids (batch,) int64 -> fp16 logits (batch, vocab); advances the state by one token.

        Like the reference's forward (df_ssm_inference.py:219-224) this only enqueues work: for
        token ids already on the device it never waits for the GPU, so the reference's loop
        `logits = forward(t); t = logits.argmax(-1)` (:234-236) stays asynchronous. Host token ids
        (lists, CPU tensors) are range-checked here (IndexError, nothing launched); device ids
        out of range set ERR_TOKEN_RANGE in the error flag (row 0 is used), which check_errors(),
        generate(), decode(), prefill() and ingest() report."""
        tok = torch.as_tensor(token_ids).view(-1)
        if tok.numel() != self.batch_size:
            raise ValueError(f"expected {self.batch_size} token ids, got {tok.numel()}")
        if tok.device.type != "cuda":
            _check_token_range(tok, self.cfg.vocab_size)
        self._tok.copy_(tok.to(self.device, torch.int64))
        if self._graph is None:
            self._capture_graph()
        self._graph.replay()
        return self.logits.clone()

    def _gen_graph(self, S: int):
        if S not in self._gen_graphs:
            hist = torch.zeros(S, self.batch_size, dtype=torch.int64, device=self.device)

            def body():
                for i in range(S):
                    self._decode(None, None, hist[i], fuse=True)
            self._gen_graphs[S] = (self._capture(body), hist)
        return self._gen_graphs[S]

    PREFILL_MAX_ROWS = 16384  # batch x tokens per prefill chunk (workspace ~ rows x 38 KB at 1.3B)

    def prefill(self, prompt: torch.Tensor, want_logits: bool = False) -> torch.Tensor:
        """Consume a (batch, T) prompt in one layer-major pass (dfssm_prefill): bit-for-bit the
        result of T decode steps. Afterwards self._next holds the greedy token after the prompt
        and self.x its embedding; returns the last token's logits if want_logits, else None."""
        prompt = torch.as_tensor(prompt)
        if prompt.dim() == 1:
            prompt = prompt.view(-1, 1)
        if prompt.shape[0] != self.batch_size or prompt.shape[1] < 1:
            raise ValueError(f"prompt must be (batch={self.batch_size}, T >= 1), got {tuple(prompt.shape)}")
        _check_token_range(prompt, self.cfg.vocab_size)
        prompt = prompt.to(self.device, torch.int64).contiguous()
        rows = min(self.PREFILL_MAX_ROWS, self.batch_size * prompt.shape[1])
        rows = max(rows, self.batch_size)
        if getattr(self, "_pf_rows", 0) < rows:
            nbytes = _C.lib().dfssm_prefill_workspace_bytes(self.dims, rows)
            if nbytes == 0:
                raise _C.DFSSMError(f"prefill of {rows} rows not supported")
            self._pf_ws = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
            self._pf_rows = rows
        _C.check(_C.lib().dfssm_prefill(
            self._model, prompt.data_ptr(), prompt.shape[1], self.x.data_ptr(), self._state,
            self.workspace.data_ptr(), self._pf_ws.data_ptr(), self._pf_rows,
            self.logits.data_ptr() if want_logits else None, self._next.data_ptr(), 1, _C.stream()), "prefill")
        self._tok.copy_(prompt[:, -1])
        out = self.logits.clone() if want_logits else None
        self.check_errors()
        return out

    def ingest(self, prompt: torch.Tensor, step_by_step: bool = False) -> None:
        """Consume a (batch, T) prompt; afterwards self._next holds the greedy token after the
        prompt and self.x its embedding. By default one layer-major prefill pass; with
        step_by_step, T decode steps (graph replays), which give the same bits."""
        prompt = torch.as_tensor(prompt)
        _check_token_range(prompt, self.cfg.vocab_size)
        prompt = prompt.to(self.device, torch.int64)
        if prompt.dim() == 1:
            prompt = prompt.view(-1, 1)
        if not step_by_step:
            self.prefill(prompt)
            return
        if self._graph is None:
            self._capture_graph()
        for t in range(prompt.shape[1]):
            self._tok.copy_(prompt[:, t])
            self._graph.replay()
        self.check_errors()

    def decode(self, n_steps: int, steps_per_graph: int = 8) -> torch.Tensor:
        """n_steps greedy steps continuing from the current state (x holds the embedding of
        self._next). Returns the (batch, n_steps) tokens produced, the first being the token after
        the one already in x."""
        S = max(1, min(steps_per_graph, n_steps))
        out = []
        done = 0
        while done < n_steps:
            s = S if n_steps - done >= S else 1
            g, hist = self._gen_graph(s)
            g.replay()
            out.append(hist.t().clone())
            done += s
        toks = torch.cat(out, dim=1)[:, :n_steps]
        self.check_errors()
        return toks

    # ------------------------------------------------------------------ sampling
    def _sampler(self, temperature, top_p, penalty, mode, seed):
        if getattr(self, "_counts", None) is None:
            V = self.cfg.vocab_size
            self._counts = torch.zeros(self.batch_size, V, dtype=torch.int32, device=self.device)
            self._sstep = torch.zeros(self.batch_size, dtype=torch.int32, device=self.device)
            self._gnext = torch.zeros(self.batch_size, dtype=torch.int64, device=self.device)
        return _C.SampleParams(float(temperature), float(top_p), float(penalty), int(mode), int(seed) & (2**64 - 1))

    def _sample_step(self, params, tokens: Optional[torch.Tensor], out: torch.Tensor) -> None:
        """One decode step whose next token is drawn by dfssm_sample instead of the argmax;
        x receives the drawn token's embedding."""
        self._decode(tokens, self.logits, self._gnext, fuse=False)
        _C.check(_C.lib().dfssm_sample(self._model, self.logits.data_ptr(), self._counts.data_ptr(),
                                       self._sstep.data_ptr(), ctypes.byref(params), out.data_ptr(),
                                       self.x.data_ptr(), self.workspace.data_ptr(), _C.stream()), "sample")

    def _sample_graph(self, S: int, params):
        key = (S, params.temperature, params.top_p, params.penalty, params.mode, params.seed)
        graphs = self.__dict__.setdefault("_sample_graphs", {})
        if key not in graphs:
            hist = torch.zeros(S, self.batch_size, dtype=torch.int64, device=self.device)

            def body():
                for i in range(S):
                    self._sample_step(params, None, hist[i])
            graphs[key] = (self._capture(body), hist)
        return graphs[key]

    def _generate_sampled(self, n_tokens, prompt, temperature, top_p, penalty, mode, seed):
        """Sampled decode (eval/gen_test.py:54-95 semantics, see dfssm_sample): the prompt is
        counted as seen, ingested, then n_tokens draws; returns (tokens (B, n), seconds)."""
        params = self._sampler(temperature, top_p, penalty, mode, seed)
        self._counts.zero_()
        self._sstep.zero_()
        self._counts.scatter_add_(1, prompt, torch.ones_like(prompt, dtype=torch.int32))
        S = 8 if n_tokens > 8 else 1
        g, hist = self._sample_graph(S, params)
        g1, hist1 = self._sample_graph(1, params)
        if prompt.shape[1] > 1:
            self.ingest(prompt[:, :-1])
        first = torch.empty(self.batch_size, dtype=torch.int64, device=self.device)
        torch.cuda.synchronize(self.device)
        start = time.perf_counter()
        self._sample_step(params, prompt[:, -1].contiguous(), first)
        out = [first[:, None].clone()]
        done = 1
        while done < n_tokens:
            if n_tokens - done >= S:
                g.replay()
                out.append(hist.t().clone())
                done += S
            else:
                g1.replay()
                out.append(hist1.t().clone())
                done += 1
        torch.cuda.synchronize(self.device)
        self._next.copy_(out[-1][:, -1])
        return torch.cat(out, dim=1)[:, :n_tokens], time.perf_counter() - start

    def generate(self, n_tokens=128, prompt=None, return_tokens=False, verbose=True, temperature=None,
                 top_p=1.0, repetition_penalty=1.0, penalty_mode=0, seed=0, state_df=None):
        """Greedy decode timed like the reference's generate (df_ssm_inference.py:226-243).

        The timed region holds n_tokens decode steps: the first consumes the last prompt token
        (token 0 without a prompt, as in the reference), each later one the previous greedy
        token. With return_tokens, returns the (batch, n_tokens) greedy tokens those steps
        produced; earlier prompt tokens are ingested before the timer starts.

        With a temperature, the tokens are drawn instead (dfssm_sample: temperature, top_p,
        repetition_penalty over the prompt and the tokens drawn so far; penalty_mode 0 is
        eval/gen_test.py:54-95, 1 the training script's :1066-1078), from a generator seeded by
        `seed`.

        With state_df (a StateDensityField; greedy only), the SSM state is quantized at every
        block_len-token chunk boundary as in training (apply_state_density_field).
        """
        B = self.batch_size
        if prompt is None:
            prompt = torch.zeros(B, 1, dtype=torch.int64)
        prompt = torch.as_tensor(prompt)
        if prompt.dim() == 1:
            prompt = prompt.view(-1, 1)
        if prompt.dim() != 2 or prompt.shape[0] != B or prompt.shape[1] < 1:
            raise ValueError(f"prompt must be (batch={B}, T >= 1), got {tuple(prompt.shape)}")
        _check_token_range(prompt, self.cfg.vocab_size)  # before any kernel reads the ids
        self.reset_state()
        prompt = prompt.to(self.device, torch.int64)
        if state_df is not None:
            if temperature is not None:
                raise ValueError("state_df is supported with greedy decoding only")
            toks, elapsed = self._generate_state_df(n_tokens, prompt, state_df)
            self.check_errors()
            self.last_elapsed = elapsed
            if verbose:
                print(f"batch={B}  {n_tokens} steps (density-field state)  {n_tokens * B} total tokens")
                print(f"  {elapsed*1000:.1f} ms  ({n_tokens * B / elapsed:.0f} tok/s total)")
            return toks if return_tokens else None
        if temperature is not None:
            toks, elapsed = self._generate_sampled(n_tokens, prompt, temperature, top_p, repetition_penalty,
                                                   penalty_mode, seed)
            self.check_errors()
            self.last_elapsed = elapsed
            if verbose:
                print(f"batch={B}  {n_tokens} sampled steps  {n_tokens * B} total tokens")
                print(f"  {elapsed*1000:.1f} ms  ({n_tokens * B / elapsed:.0f} tok/s total)")
            return toks if return_tokens else None
        # graphs are captured before the timer starts; capture executes nothing
        if self._graph is None:
            self._capture_graph()
        S = 8 if n_tokens > 8 else 1
        self._gen_graph(S)
        self._gen_graph(1)
        if prompt.shape[1] > 1:
            self.ingest(prompt[:, :-1])
        torch.cuda.synchronize(self.device)
        start = time.perf_counter()
        self._tok.copy_(prompt[:, -1])
        self._graph.replay()
        first = self._next.clone()
        rest = self.decode(n_tokens - 1, S) if n_tokens > 1 else None
        torch.cuda.synchronize(self.device)
        elapsed = time.perf_counter() - start
        self.check_errors()
        total = n_tokens * B
        if verbose:
            print(f"batch={B}  {n_tokens} steps  {total} total tokens")
            print(f"  {elapsed*1000:.1f} ms  ({total/elapsed:.0f} tok/s total, "
                  f"{elapsed/n_tokens*1e6:.0f} μs/step, {total/elapsed/B:.0f} tok/s/seq)")
        self.last_elapsed = elapsed
        if return_tokens:
            return first[:, None] if rest is None else torch.cat([first[:, None], rest], dim=1)
        return None

    def error_flag(self) -> int:
        """The workspace error flag (synchronizes): 0, or an OR of ERR_TOKEN_RANGE (1: a token id
        outside [0, vocab) reached the embedding gather, which then read row 0) and the wait
        bits ERR_WAIT_LAYER (4), ERR_WAIT_SSM_PROLOGUE (8), ERR_WAIT_OUT_PROLOGUE (16): a bounded
        wait between workgroups of that launch timed out, so its output is wrong. The flag stays
        set until clear_error_flag()."""
        off = self._err - self.workspace.data_ptr()
        return int(self.workspace[off:off + 4].view(torch.int32).item())

    def clear_error_flag(self) -> None:
        off = self._err - self.workspace.data_ptr()
        self.workspace[off:off + 4].zero_()

    def check_errors(self) -> None:
        """Read the workspace error flag (synchronizes); if it is set, clear it and raise
        DFSSMError naming the cause. generate(), decode(), prefill() and ingest() call it after
        their work; forward() does not (it only enqueues, as the reference's forward does)."""
        flag = self.error_flag()
        if flag:
            self.clear_error_flag()
            raise _C.DFSSMError(f"decode kernels reported error flag {flag:#x}: {describe_error_flag(flag)}")


if __name__ == "__main__":
    import argparse
    p = argparse.ArgumentParser()
    p.add_argument("model"); p.add_argument("--batch_size", type=int, default=1)
    p.add_argument("--n_tokens", type=int, default=128)
    a = p.parse_args()
    DFSSMModel(a.model, batch_size=a.batch_size).generate(n_tokens=a.n_tokens)
