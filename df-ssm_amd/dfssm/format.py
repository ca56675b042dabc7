"""`.dfssm` model format: 64-byte header, embedding, per-layer tensor stream, final norm.

Byte layout follows the reference writer, training/export_dfssm.py:104-193:

  header  struct '8s9I20s' (export_dfssm.py:106-121): magic "DFSSM001", u32 n_layer,
          d_model, d_inner, d_state, nheads, headdim, ngroups, vocab_size, Kw, 20 reserved bytes
  embedding (V, D) fp16                                   (export_dfssm.py:125-126)
  per layer, in this order                                (export_dfssm.py:135-185)
      in_packed  (IPO, D/32) int32 sign bits, LSB first   (export_dfssm.py:34-42,143-147)
      in_scale   (IPO) fp16                               (:150-151)
      in_lA (IPO, R) int8, in_lA_s (IPO) fp16             (:154-157)
      in_lB (R, D) int8,   in_lB_s (R) fp16               (:160-162)
      out_packed (D, DI/32) int32, out_scale (D) fp16, out_lA (D, R) int8, out_lA_s (D) fp16,
      out_lB (R, DI) int8, out_lB_s (R) fp16
      conv_w (C, 4) fp16, conv_b (C) fp16                 (:170-174)
      A_log, D, dt_bias (H) fp32                          (:177-179)
      norm_w (DI) fp32 (mixer norm), ln_w (D) fp32 (pre-layer norm)   (:182,185)
  norm_f (D) fp32                                         (:193)

with IPO = 2*DI + 2*ngroups*N + H, C = DI + 2*ngroups*N, R = 16 (LoRA rank) and d_conv = 4, both
implied constants of the reference (export_dfssm.py:26-29).

Two extensions live in the reserved bytes, so files the reference exporter writes (all zero there)
keep their meaning:
  reserved[0]  embedding code: 0 = fp16 (V, D) as the exporter writes it;
               1 = int8 (V, D) followed by a (V) fp16 per-row scale (the tied int8 head).
  reserved[1]  norm dtype code: 0 = fp32 (the writer, export_dfssm.py:182,185,193);
               1 = fp16 (what the reference GPU loader assumes, df_ssm_inference.py:105-106,110).
Every other reserved byte must be zero.

The reader derives the SSM head dimension as d_inner / nheads (Mamba-2 semantics, training
df_ssm_mamba2_distill_dfw.py:309-316) and reports the header's headdim field separately, because
the reference exporter writes 32 there for a 64-wide head (export_dfssm.py:24,114).
The reader computes the exact file size from the header and rejects any mismatch before parsing.
"""
from __future__ import annotations

import struct
import warnings
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import numpy as np

MAGIC = b"DFSSM001"
HEADER_SIZE = 64
HEADER_FMT = "<8s9I20s"
LORA_RANK = 16
D_CONV = 4

EMB_F16 = 0
EMB_I8 = 1
NORM_F32 = 0
NORM_F16 = 1


class DFSSMFormatError(ValueError):
    """Raised for a malformed, truncated or inconsistent .dfssm file."""


@dataclass(frozen=True)
class DFSSMConfig:
    n_layer: int
    d_model: int
    d_inner: int
    d_state: int
    nheads: int
    headdim: int          # header field as written; the SSM uses `p` below
    ngroups: int
    vocab_size: int
    kw: int = 4           # density-field training parameter carried through the header
    emb_code: int = EMB_I8
    norm_code: int = NORM_F32

    @property
    def d_xbc(self) -> int:
        return self.d_inner + 2 * self.ngroups * self.d_state

    @property
    def in_proj_out(self) -> int:
        return 2 * self.d_inner + 2 * self.ngroups * self.d_state + self.nheads

    @property
    def p(self) -> int:
        """SSM head dimension derived from the dims (d_inner / nheads)."""
        return self.d_inner // self.nheads

    def validate(self) -> None:
        for name in ("n_layer", "d_model", "d_inner", "d_state", "nheads", "ngroups", "vocab_size"):
            if getattr(self, name) <= 0:
                raise DFSSMFormatError(f"header field {name} must be positive, got {getattr(self, name)}")
        if self.d_model % 32 or self.d_inner % 32:
            raise DFSSMFormatError("d_model and d_inner must be multiples of 32 (bit packing)")
        if self.d_inner % self.nheads:
            raise DFSSMFormatError(f"d_inner={self.d_inner} is not a multiple of nheads={self.nheads}")
        if self.nheads % self.ngroups:
            raise DFSSMFormatError("nheads must be a multiple of ngroups")
        if self.emb_code not in (EMB_F16, EMB_I8):
            raise DFSSMFormatError(f"unknown embedding code {self.emb_code}")
        if self.norm_code not in (NORM_F32, NORM_F16):
            raise DFSSMFormatError(f"unknown norm dtype code {self.norm_code}")

    def header_bytes(self) -> bytes:
        reserved = bytes([self.emb_code, self.norm_code]) + b"\x00" * 18
        return struct.pack(HEADER_FMT, MAGIC, self.n_layer, self.d_model, self.d_inner, self.d_state,
                           self.nheads, self.headdim, self.ngroups, self.vocab_size, self.kw, reserved)

    def norm_dtype(self):
        return np.float32 if self.norm_code == NORM_F32 else np.float16


def layer_tensor_specs(cfg: DFSSMConfig) -> List[Tuple[str, Tuple[int, ...], type]]:
    """(name, shape, dtype) of each per-layer tensor in file order (export_dfssm.py:135-185)."""
    D, DI, H, R = cfg.d_model, cfg.d_inner, cfg.nheads, LORA_RANK
    IPO, C = cfg.in_proj_out, cfg.d_xbc
    nd = cfg.norm_dtype()
    return [
        ("in_packed", (IPO, D // 32), np.uint32),
        ("in_scale", (IPO,), np.float16),
        ("in_lA", (IPO, R), np.int8),
        ("in_lA_s", (IPO,), np.float16),
        ("in_lB", (R, D), np.int8),
        ("in_lB_s", (R,), np.float16),
        ("out_packed", (D, DI // 32), np.uint32),
        ("out_scale", (D,), np.float16),
        ("out_lA", (D, R), np.int8),
        ("out_lA_s", (D,), np.float16),
        ("out_lB", (R, DI), np.int8),
        ("out_lB_s", (R,), np.float16),
        ("conv_w", (C, D_CONV), np.float16),
        ("conv_b", (C,), np.float16),
        ("A_log", (H,), np.float32),
        ("D", (H,), np.float32),
        ("dt_bias", (H,), np.float32),
        ("norm_w", (DI,), nd),
        ("ln_w", (D,), nd),
    ]


def _nbytes(shape, dtype) -> int:
    n = 1
    for s in shape:
        n *= s
    return n * np.dtype(dtype).itemsize


def layer_bytes(cfg: DFSSMConfig) -> int:
    return sum(_nbytes(s, d) for _, s, d in layer_tensor_specs(cfg))


def embedding_bytes(cfg: DFSSMConfig) -> int:
    V, D = cfg.vocab_size, cfg.d_model
    if cfg.emb_code == EMB_F16:
        return V * D * 2
    return V * D + V * 2


def expected_size(cfg: DFSSMConfig) -> int:
    nd = np.dtype(cfg.norm_dtype()).itemsize
    return HEADER_SIZE + embedding_bytes(cfg) + cfg.n_layer * layer_bytes(cfg) + cfg.d_model * nd


def parse_header(hdr: bytes) -> DFSSMConfig:
    if len(hdr) < HEADER_SIZE:
        raise DFSSMFormatError(f"file shorter than the {HEADER_SIZE}-byte header")
    magic, L, D, DI, N, H, hd, ng, V, kw, reserved = struct.unpack(HEADER_FMT, hdr[:HEADER_SIZE])
    if magic != MAGIC:
        raise DFSSMFormatError(f"bad magic {magic!r}, expected {MAGIC!r}")
    if any(reserved[2:]):
        raise DFSSMFormatError("reserved header bytes 2..19 must be zero")
    cfg = DFSSMConfig(L, D, DI, N, H, hd, ng, V, kw, reserved[0], reserved[1])
    cfg.validate()
    return cfg


@dataclass
class DFSSMWeights:
    """Host (numpy) copy of a .dfssm model. Layer dicts use the names of layer_tensor_specs."""
    cfg: DFSSMConfig
    emb: np.ndarray                    # (V, D) int8 or fp16
    emb_scale: Optional[np.ndarray]    # (V,) fp16 for EMB_I8, else None
    layers: List[Dict[str, np.ndarray]] = field(default_factory=list)
    norm_f: Optional[np.ndarray] = None

    def emb_f16(self) -> np.ndarray:
        """The fp16 table the embedding gather and tied head see: fp16(E_i8 * s_E) for int8."""
        if self.cfg.emb_code == EMB_F16:
            return self.emb
        return (self.emb.astype(np.float32) * self.emb_scale.astype(np.float32)[:, None]).astype(np.float16)


def read_dfssm(path: str) -> DFSSMWeights:
    """Parse a .dfssm file after checking its size against the header."""
    with open(path, "rb") as f:
        hdr = f.read(HEADER_SIZE)
        cfg = parse_header(hdr)
        f.seek(0, 2)
        size = f.tell()
    want = expected_size(cfg)
    if size != want:
        raise DFSSMFormatError(
            f"{path}: size {size} B does not match the {want} B implied by the header "
            f"(L={cfg.n_layer} D={cfg.d_model} DI={cfg.d_inner} H={cfg.nheads} V={cfg.vocab_size} "
            f"emb_code={cfg.emb_code} norm_code={cfg.norm_code})")
    if cfg.headdim != cfg.p:
        warnings.warn(f"header headdim={cfg.headdim} differs from d_inner/nheads={cfg.p}; "
                      f"the SSM uses {cfg.p}")
    raw = np.fromfile(path, dtype=np.uint8)
    off = HEADER_SIZE

    def take(shape, dtype):
        nonlocal off
        nb = _nbytes(shape, dtype)
        arr = raw[off:off + nb].view(dtype).reshape(shape).copy()
        off += nb
        return arr

    V, D = cfg.vocab_size, cfg.d_model
    if cfg.emb_code == EMB_F16:
        emb, emb_scale = take((V, D), np.float16), None
    else:
        emb, emb_scale = take((V, D), np.int8), take((V,), np.float16)
    w = DFSSMWeights(cfg, emb, emb_scale)
    specs = layer_tensor_specs(cfg)
    for _ in range(cfg.n_layer):
        w.layers.append({name: take(shape, dt) for name, shape, dt in specs})
    w.norm_f = take((D,), cfg.norm_dtype())
    assert off == size
    return w


def write_dfssm(path: str, w: DFSSMWeights) -> int:
    """Write `w` in .dfssm layout; returns the byte count (checked against expected_size)."""
    cfg = w.cfg
    cfg.validate()
    specs = layer_tensor_specs(cfg)
    total = 0
    with open(path, "wb") as f:
        hdr = cfg.header_bytes()
        assert len(hdr) == HEADER_SIZE
        f.write(hdr)
        total += len(hdr)

        def put(arr, shape, dtype, name):
            nonlocal total
            a = np.asarray(arr)
            if a.shape != tuple(shape) or a.dtype != np.dtype(dtype):
                raise DFSSMFormatError(f"{name}: got {a.shape} {a.dtype}, expected {shape} {np.dtype(dtype)}")
            b = np.ascontiguousarray(a).tobytes()
            f.write(b)
            total += len(b)

        V, D = cfg.vocab_size, cfg.d_model
        if cfg.emb_code == EMB_F16:
            put(w.emb, (V, D), np.float16, "embedding")
        else:
            put(w.emb, (V, D), np.int8, "embedding")
            put(w.emb_scale, (V,), np.float16, "embedding scale")
        if len(w.layers) != cfg.n_layer:
            raise DFSSMFormatError(f"{len(w.layers)} layers given, header says {cfg.n_layer}")
        for li, layer in enumerate(w.layers):
            for name, shape, dt in specs:
                put(layer[name], shape, dt, f"layer {li} {name}")
        put(w.norm_f, (D,), cfg.norm_dtype(), "norm_f")
    if total != expected_size(cfg):
        raise DFSSMFormatError(f"wrote {total} B, expected {expected_size(cfg)}")
    return total


# --- bit packing (export_dfssm.py:34-42) ------------------------------------------------------

def pack_sign_bits(signs01: np.ndarray) -> np.ndarray:
    """Pack a (rows, cols) array of 0/1 into (rows, cols/32) uint32: word j bit b <- column 32j+b.

    Restates pack_bits_to_int32 (export_dfssm.py:34-42): `packed |= bits[:, b::32] << b`.
    """
    rows, cols = signs01.shape
    if cols % 32:
        raise ValueError(f"cols={cols} must be a multiple of 32")
    b = signs01.astype(np.uint32).reshape(rows, cols // 32, 32)
    shifts = np.arange(32, dtype=np.uint32)
    return np.bitwise_or.reduce(b << shifts, axis=2).astype(np.uint32)


def unpack_sign_bits(packed: np.ndarray) -> np.ndarray:
    """(rows, K/32) uint32 -> (rows, K) int8 of +1 (bit set) / -1 (bit clear).

    Restates _unpack_to_int8 (df_ssm_inference.py:23-29): w[:, b::32] = 2*((packed >> b) & 1) - 1.
    """
    p = np.ascontiguousarray(packed, dtype=np.uint32)
    rows, words = p.shape
    bits = np.unpackbits(p.view(np.uint8).reshape(rows, words * 4), axis=1, bitorder="little")
    return (bits.astype(np.int8) * 2 - 1).reshape(rows, words * 32)
