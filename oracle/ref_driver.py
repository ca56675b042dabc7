"""ctypes driver for the reference CPU decode kernels (oracle/_ref/libcpu_inference_h64.so).

TEST / BASELINE INFRASTRUCTURE ONLY (used by tests/ and bench.py's cpu_baseline leg).

Reproduces the behaviour of the reference driver inference/cpu/cpu_inference_driver.py:77-204 in
this build's own code: weights widened to fp32 at load (:96,105,111-131), row sums precomputed
with the reference's precompute_row_sums (:106-108,117-119), per token embedding_lookup,
layer_forward for every layer, final_rms_norm, an fp32 NumPy LM head and argmax (:159-184,197).
The library is the reference's cpu_inference.c compiled with HEADDIM = 64 (oracle/build_ref.sh);
its dimensions are compile-time constants, so only the 1.3B shape can be driven.
"""
from __future__ import annotations

import ctypes
import os
import time

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_ref", "libcpu_inference_h64.so")
F_P = ctypes.POINTER(ctypes.c_float)


def host_supports_reference() -> bool:
    """The reference kernels need AVX-512 F/BW and VNNI."""
    try:
        flags = open("/proc/cpuinfo").read()
    except OSError:
        return False
    return all(f in flags for f in ("avx512f", "avx512bw", "avx512_vnni"))


def available() -> bool:
    return os.path.exists(LIB_PATH) and host_supports_reference()


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


class RefCPUModel:
    def __init__(self, weights):
        c = weights.cfg
        if (c.d_model, c.d_inner, c.nheads, c.p, c.d_state, c.in_proj_out) != (2048, 4096, 64, 64, 128, 8512):
            raise ValueError("the reference CPU kernels are compiled for the 1.3B shape only")
        self.lib = ctypes.CDLL(LIB_PATH)
        self.lib.layer_forward.restype = None
        self.lib.precompute_row_sums.restype = None
        self.cfg = c
        f32 = lambda a: np.ascontiguousarray(a, dtype=np.float32)  # noqa: E731
        self.layers = []
        for L in weights.layers:
            lw = {}
            for pre, N, K in (("in", c.in_proj_out, c.d_model), ("out", c.d_model, c.d_inner)):
                lw[pre + "_packed"] = np.ascontiguousarray(L[pre + "_packed"], dtype=np.uint32)
                lw[pre + "_scale"] = f32(L[pre + "_scale"])
                rs = np.empty(N, np.int32)
                self.lib.precompute_row_sums(_p(lw[pre + "_packed"]), _p(rs), N, K // 32)
                lw[pre + "_rs"] = rs
                lw[pre + "_lA"] = np.ascontiguousarray(L[pre + "_lA"])
                lw[pre + "_lAs"] = f32(L[pre + "_lA_s"])
                lw[pre + "_lB"] = np.ascontiguousarray(L[pre + "_lB"])
                lw[pre + "_lBs"] = f32(L[pre + "_lB_s"])
            for k in ("conv_w", "conv_b", "A_log", "D", "dt_bias", "norm_w", "ln_w"):
                lw[k] = f32(L[k])
            self.layers.append(lw)
        self.embedding = weights.emb_f16().astype(np.float32)
        self.norm_f = f32(weights.norm_f)
        self.h = np.zeros((c.n_layer, c.nheads, c.p, c.d_state), np.float32)
        self.conv = np.zeros((c.n_layer, c.d_xbc, 3), np.float32)
        self.x = np.empty(c.d_model, np.float32)
        self.scratch = [np.empty(n, np.float32) for n in (c.d_model, c.in_proj_out, c.d_inner, c.d_model)]
        self.norm_out = np.empty(c.d_model, np.float32)

    def reset(self):
        self.h[...] = 0
        self.conv[...] = 0

    def forward(self, token: int) -> np.ndarray:
        c = self.cfg
        self.x[:] = self.embedding[token]
        for li, w in enumerate(self.layers):
            self.lib.layer_forward(
                _p(self.x), _p(w["in_packed"]), _p(w["in_scale"]), _p(w["in_rs"]),
                _p(w["out_packed"]), _p(w["out_scale"]), _p(w["out_rs"]),
                _p(w["in_lA"]), _p(w["in_lAs"]), _p(w["in_lB"]), _p(w["in_lBs"]),
                _p(w["out_lA"]), _p(w["out_lAs"]), _p(w["out_lB"]), _p(w["out_lBs"]),
                _p(w["conv_w"]), _p(w["conv_b"]), _p(w["A_log"]), _p(w["D"]), _p(w["dt_bias"]),
                _p(w["norm_w"]), _p(w["ln_w"]), _p(self.h[li]), _p(self.conv[li]),
                *[_p(s) for s in self.scratch])
        self.lib.final_rms_norm(_p(self.x), _p(self.norm_f), _p(self.norm_out), c.d_model)
        return self.norm_out @ self.embedding.T

    def generate(self, prompt, n_tokens: int):
        """cpu_inference_driver.py:186-204 with a prompt: warm-up forward, reset, the prompt
        step by step (untimed), then n_tokens timed greedy steps. Returns (tokens, seconds)."""
        self.forward(int(prompt[0]))
        self.reset()
        logits = None
        for t in prompt:
            logits = self.forward(int(t))
        tok = int(np.argmax(logits))
        out = [tok]
        t0 = time.perf_counter()
        for _ in range(n_tokens):
            tok = int(np.argmax(self.forward(tok)))
            out.append(tok)
        return out, time.perf_counter() - t0


def cpu_description() -> dict:
    """CPU model, sockets and physical cores per socket from /proc/cpuinfo; CPUs this process may
    run on from its affinity mask."""
    model, phys, cores = "unknown", set(), {}
    cur = {}
    try:
        text = open("/proc/cpuinfo").read()
    except OSError:
        text = ""
    for block in text.split("\n\n"):
        cur = {}
        for ln in block.splitlines():
            if ":" in ln:
                k, v = ln.split(":", 1)
                cur[k.strip()] = v.strip()
        if "model name" in cur:
            model = cur["model name"]
        if "physical id" in cur:
            phys.add(cur["physical id"])
            if "cpu cores" in cur:
                cores[cur["physical id"]] = int(cur["cpu cores"])
    try:
        allowed_set = sorted(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed_set = list(range(os.cpu_count() or 1))
    per_socket = max(cores.values()) if cores else (os.cpu_count() or 1)
    phys_allowed = _physical_cores(allowed_set)
    quota = _cgroup_cpu_quota()
    usable = phys_allowed if quota is None else max(1, min(phys_allowed, int(quota)))
    return {"model": model, "sockets": max(1, len(phys)), "cores_per_socket": per_socket,
            "logical_cpus": os.cpu_count(), "allowed_cpus": len(allowed_set),
            "allowed_physical_cores": phys_allowed, "cgroup_cpu_quota": quota, "usable_cores": usable}


def _physical_cores(cpus) -> int:
    """Number of distinct physical cores among `cpus` (SMT siblings counted once), from
    /sys/devices/system/cpu/cpuN/topology/thread_siblings_list; len(cpus) if that is unreadable."""
    groups = set()
    for c in cpus:
        try:
            groups.add(open(f"/sys/devices/system/cpu/cpu{c}/topology/thread_siblings_list").read().strip())
        except OSError:
            return len(cpus)
    return max(1, len(groups))


def _cgroup_cpu_quota():
    """CPUs this process's cgroup may use (quota / period), or None when unlimited or unknown:
    cgroup v2 cpu.max ("max 100000" or "<quota> <period>"), else v1 cpu.cfs_quota_us / cfs_period_us."""
    try:
        q, p = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        return None if q == "max" else float(q) / float(p)
    except (OSError, ValueError):
        pass
    try:
        q = float(open("/sys/fs/cgroup/cpu/cpu.cfs_quota_us").read())
        p = float(open("/sys/fs/cgroup/cpu/cpu.cfs_period_us").read())
        return None if q <= 0 else q / p
    except (OSError, ValueError):
        return None


def main(argv=None) -> int:
    """Time the reference CPU decode on a .dfssm file: the protocol of generate() above, printed as
    one JSON line. OpenMP threads come from the environment (OMP_NUM_THREADS, OMP_PROC_BIND,
    OMP_PLACES), read when the library loads."""
    import argparse
    import json
    import sys
    ap = argparse.ArgumentParser()
    ap.add_argument("--model", required=True)
    ap.add_argument("--prompt", required=True, help="comma-separated token ids")
    ap.add_argument("--tokens", type=int, default=128)
    a = ap.parse_args(argv)
    repo = os.path.dirname(_HERE)
    sys.path.insert(0, os.path.join(repo, "df-ssm_amd"))
    from dfssm.format import read_dfssm
    if not available():
        print(json.dumps({"error": "reference CPU kernels unavailable (not built or no AVX-512 VNNI)"}))
        return 1
    w = read_dfssm(a.model)
    prompt = [int(t) for t in a.prompt.split(",")]
    m = RefCPUModel(w)
    toks, secs = m.generate(prompt, a.tokens)
    print(json.dumps({"tokens": a.tokens, "seconds": secs, "tok_s": a.tokens / secs,
                      "threads": int(os.environ.get("OMP_NUM_THREADS", "0") or 0),
                      "first_tokens": toks[:8]}))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
