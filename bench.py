#!/usr/bin/env python3
"""DF-SSM decode throughput on one MI355X.

Workload: the 1.3B-shaped DF-SSM (d_model 2048, 48 layers, d_inner 4096,
64 heads x 64, d_state 128, vocab 50288, rank-16 int8 LoRA, int8 tied embedding) with seeded
random-init weights, written to and loaded from a .dfssm file; a seeded 32-token prompt per
sequence is ingested (dfssm_prefill, bit-identical to step-by-step ingestion; its time is reported
under "prefill"), then greedy decode steps are timed. One step = one token for
every sequence of the batch: embedding, 48 layers, final norm, tied head, argmax, with the
greedy token fed back on the device (HIP graph of 8 steps per replay). value = batch * steps /
seconds over the timed steps, inputs resident in HBM.

Also reported: per-kernel timing of the five layer kernels and the head (HIP events around graphs
of 48 back-to-back launches of one kernel, divided by the launch count), the roofline of the
dominant kernel, the whole-step HBM roofline fraction, and the reference CPU decode (the
reference's cpu_inference.c, HEADDIM 64, compiled in oracle/_ref) on a bounded sample.

    python bench.py [--gpus 1] [--steps 128] [--warmup 16] [--batch 1] [--no-cpu]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "df-ssm_amd"))
sys.path.insert(0, REPO)

PEAK_GBS = 8000.0     # MI355X HBM3E, GB/s
STEPS_PER_GRAPH = 8
SCAFFOLD_WS_BYTES = 64 << 10   # DFSSM_SCAFFOLD_WORKSPACE_BYTES
SCAFFOLD_ERR_OFFSET = 1024     # DFSSM_SCAFFOLD_ERROR_OFFSET


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algorithmic_bytes(cfg, B):
    """Bytes a decode step must move: every weight once + SSM/conv state read and written."""
    from dfssm.format import layer_bytes
    D, DI, H, P, N, C, V, L = (cfg.d_model, cfg.d_inner, cfg.nheads, cfg.p, cfg.d_state, cfg.d_xbc,
                               cfg.vocab_size, cfg.n_layer)
    IPO = cfg.in_proj_out
    weights = L * layer_bytes(cfg) + V * D + 2 * V + 4 * D
    state = B * L * 2 * (H * P * N * 4 + C * 3 * 2)
    ns = H * (P // 16)  # SSM blocks per sequence (partials of sum(g^2))
    per_phase = {
        # prep_in: x, ln_w, LoRA B + scales in; q bytes, bit planes, scalars, h out
        0: B * D * 2 + 4 * D + 16 * D + 32 + B * (2 * D + 8 + 64),
        # gemv_in: bits, scales, LoRA A + scales, planes + prep scalars, conv w/b + state r+w, proj out
        1: IPO * D // 8 + 2 * IPO + 16 * IPO + 2 * IPO + B * (D + 8 + 64) + 8 * C + 2 * C
           + B * C * 6 * 2 + B * IPO * 2,
        # SSM: state r+w, x/B/C/dt/z in, params, g out, block partials
        1.5: B * H * P * N * 4 * 2 + B * (DI + 2 * N + H + DI) * 2 + 12 * H + B * DI * 2 + B * ns * 8,
        # prep_out: g, partials, norm_w, LoRA B + scales in; q, planes, scalars, h out
        2: B * DI * 2 + B * ns * 8 + 4 * DI + 16 * DI + 32 + B * (2 * DI + 8 + 64),
        # gemv_out: bits, scales, LoRA A + scales, planes + scalars, x r+w
        2.5: D * DI // 8 + 2 * D + 16 * D + 2 * D + B * (DI + 8 + 64) + B * D * 4,
        # head: int8 table + row scales + norm_f + x
        3: V * D + 2 * V + 4 * D + B * D * 2,
        # one-launch layer (batch <= 4): the layer's weights, its SSM/conv state read and written,
        # x read and written
        4: layer_bytes(cfg) + B * (H * P * N * 4 + C * 3 * 2) * 2 + B * D * 4,
        # SSM + out_proj prologue in one launch (batch >= 5): the SSM's bytes without g out and the
        # partials, the prologue's without g in (g passes between the launch's workgroups): norm_w,
        # LoRA B + scales in; q, scale, h out
        5: B * H * P * N * 4 * 2 + B * (DI + 2 * N + H + DI) * 2 + 12 * H + 4 * DI + 16 * DI + 32 + B * (DI + 68),
        # out_proj + the next layer's in_proj prologue (batch >= 5): gemv_out's bytes, the next ln_w,
        # LoRA B + scales in; q, scale, h out (x passes between the launch's workgroups)
        6: D * DI // 8 + 2 * D + 16 * D + 2 * D + B * (DI + 8 + 64) + B * D * 4 + 4 * D + 16 * D + 32 + B * (D + 68),
    }
    return weights, state, per_phase


LAYER_KERNELS = {"auto": 0, "fused": 1, "five": 2}  # dfssm_set_layer_kernel codes
LAYER_KERNEL = "auto"


def build_model(B, path, shape="1p3b"):
    import torch
    from df_ssm_inference import DFSSMModel
    from dfssm.format import expected_size, write_dfssm
    from dfssm.synth import config_1p3b, config_2p7b, make_weights
    cfg = config_1p3b() if shape == "1p3b" else config_2p7b()
    w = None
    if not (os.path.exists(path) and os.path.getsize(path) == expected_size(cfg)):
        t = time.time()
        w = make_weights(cfg, seed=0)
        write_dfssm(path + ".tmp", w)
        os.replace(path + ".tmp", path)
        log(f"wrote synthetic {shape} model to {path} ({time.time() - t:.1f}s)")
    t = time.time()
    m = DFSSMModel(path, device="cuda:0", batch_size=B)
    torch.cuda.synchronize()
    log(f"loaded {path} for batch {B} ({time.time() - t:.1f}s)")
    if LAYER_KERNEL != "auto":
        from dfssm import _C
        _C.lib().dfssm_set_layer_kernel(LAYER_KERNELS[LAYER_KERNEL])
        log(f"layer kernel: {LAYER_KERNEL}")
    return m, w


def time_prefill(m, prompts):
    """Prompt ingestion by dfssm_prefill (layer-major, bit-identical to step-by-step decode): one
    untimed call (workspace allocation), then one timed with HIP events from a reset state.
    Leaves the state after the prompt."""
    import torch
    p = torch.from_numpy(prompts).to("cuda:0")
    m.reset_state()
    m.prefill(p)
    m.reset_state()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    m.prefill(p)
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1)


def time_state_df(m, reps=20):
    """One density-field quantization of the whole state (dfssm_state_density_field with
    sigma-delta, K = 8 bank), averaged over `reps` calls timed with HIP events on the library's
    stream. Returns (us per call, bytes per call): the state and the error are read and written."""
    import torch
    from df_ssm_inference import StateDensityField
    df = StateDensityField.random(K=8, num_banks=64)
    m.apply_state_density_field(df, 0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for c in range(reps):
        m.apply_state_density_field(df, c)
    e1.record()
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    m.reset_state()
    return us, 4 * m.h_state.numel() * 4


def replay_steps(graph_of, n):
    """Replay decode graphs covering exactly n steps: graphs of STEPS_PER_GRAPH steps, then one
    graph of the remainder. graph_of(S) returns (graph, history) for S fused steps."""
    full, rest = divmod(n, STEPS_PER_GRAPH)
    if full:
        g, _ = graph_of(STEPS_PER_GRAPH)
        for _ in range(full):
            g.replay()
    if rest:
        graph_of(rest)[0].replay()


def time_decode(m, prompts, steps, warmup):
    """Exactly `warmup` untimed then `steps` timed greedy steps (HIP events on the launch stream);
    returns (ms, steps)."""
    import torch
    m.reset_state()
    m.ingest(torch.from_numpy(prompts))
    for S in {STEPS_PER_GRAPH, steps % STEPS_PER_GRAPH, warmup % STEPS_PER_GRAPH} - {0}:
        m._gen_graph(S)  # capture before timing
    replay_steps(m._gen_graph, warmup)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    replay_steps(m._gen_graph, steps)
    e1.record()
    e1.synchronize()
    ms = e0.elapsed_time(e1)
    return ms, steps


def time_sampled(m, prompts, steps, warmup, T=0.7, top_p=0.9, penalty=1.2):
    """Decode with the sampling head (gen_test.py's settings: temperature 0.7, top-p 0.9,
    repetition penalty 1.2) instead of the argmax: graphs of 8 steps, HIP events. Returns ms
    per step and the sampler's own time per call, all its kernels (graph of 48 calls on fixed logits)."""
    import torch
    from dfssm import _C
    m.reset_state()
    params = m._sampler(T, top_p, penalty, 0, 1234)
    m._counts.zero_()
    m._sstep.zero_()
    m.ingest(torch.from_numpy(prompts))
    graph_of = lambda S: m._sample_graph(S, params)  # noqa: E731
    for S in {STEPS_PER_GRAPH, steps % STEPS_PER_GRAPH, warmup % STEPS_PER_GRAPH} - {0}:
        graph_of(S)
    replay_steps(graph_of, warmup)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    replay_steps(graph_of, steps)
    e1.record()
    e1.synchronize()
    ms = e0.elapsed_time(e1) / steps
    lib = _C.lib()
    out = torch.zeros(m.batch_size, dtype=torch.int64, device="cuda:0")
    ks = torch.cuda.CUDAGraph()
    with torch.cuda.graph(ks):
        for _ in range(48):
            _C.check(lib.dfssm_sample(m._model, m.logits.data_ptr(), m._counts.data_ptr(), m._sstep.data_ptr(),
                                      ctypes.byref(params), out.data_ptr(), None, m.workspace.data_ptr(),
                                      _C.stream()))
    ks.replay()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(5):
        ks.replay()
    e1.record()
    e1.synchronize()
    return ms, e0.elapsed_time(e1) * 1e3 / (5 * 48)


def time_kernels(m, reps=10):
    """Per-launch time of each layer kernel and of the head: HIP events on the launch stream around
    `reps` replays of a graph of 48 back-to-back launches of that kernel alone, divided by the
    launch count. This is the kernel's duration plus the gap between dependent launches, i.e. what
    one launch costs inside the decode step; the same arrangement with an empty kernel gives the
    gap alone. Returns {name: (us_per_launch, launches_per_step)}; "empty" holds the gap."""
    import torch
    from dfssm import _C
    L = m.cfg.n_layer
    lib = _C.lib()

    def graph_time(body, n):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            body()
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (reps * n)

    one = torch.zeros(1, device="cuda:0")
    empty = graph_time(lambda: [one.mul_(1.0) for _ in range(L)], L)
    out = {"empty": (empty, 0)}
    def phase(p, li):
        return lib.dfssm_layer_phase(m._model, li, p, m.x.data_ptr(), m._state, m.workspace.data_ptr(),
                                     _C.stream())

    if m.batch_size <= 4:
        # the decode path runs each layer as one launch at this batch
        def layer():
            for li in range(L):
                _C.check(lib.dfssm_layer_step(m._model, li, m.x.data_ptr(), m._state,
                                              m.workspace.data_ptr(), _C.stream()))
        out["layer (one launch)"] = (graph_time(layer, L), L)
        # the stand-alone scaffold GEMV kernel, timed as a microbenchmark
        plan = [("in_proj+conv", 1, L, 0)]
    else:
        # the launches of the decode step at this batch (dfssm_decode_step): in_proj, the SSM with
        # out_proj's prologue and out_proj with the next layer's prologue where the shape takes
        # them (probed once, eagerly), the prologue of layer 0 and out_proj of the last layer
        ssm_fused = phase(_C.PHASE_SSM_PROLOGUE, 0) == 0
        out_fused = L > 1 and phase(_C.PHASE_OUT_PROLOGUE, 0) == 0
        torch.cuda.synchronize()
        plan = [("prep_in", 0, L, 1 if out_fused else L), ("in_proj+conv", 1, L, L)]
        plan += [("ssm+prologue", _C.PHASE_SSM_PROLOGUE, L, L)] if ssm_fused else \
            [("ssm+gate", 2, L, L), ("prep_out", 3, L, L)]
        plan += [("out_proj+prologue", _C.PHASE_OUT_PROLOGUE, L - 1, L - 1), ("out_proj+residual", 4, L, 1)] \
            if out_fused else [("out_proj+residual", 4, L, L)]
    for name, p, nl, per_step in plan:
        def body(p=p, nl=nl):
            for li in range(nl):
                _C.check(phase(p, li))
        out[name] = (graph_time(body, nl), per_step)

    def head():
        for _ in range(L):
            _C.check(lib.dfssm_lmhead_argmax(m._model, m.x.data_ptr(), m.workspace.data_ptr(), None,
                                             m._next.data_ptr(), None, _C.stream()))
    out["head+argmax"] = (graph_time(head, L), 1)
    return out


def cpu_baseline(model_path, prompt, n_tokens):
    """The reference's cpu_inference.c (oracle/_ref, HEADDIM 64) on the same .dfssm file and prompt,
    timed on this host: warm-up step, reset, the prompt untimed, n_tokens timed greedy steps
    (cpu_inference_driver.py:186-204). Run in child processes, so that OpenMP reads its settings at
    load: 4 threads (the reference's published setting, README.md:67), every physical core this
    process may use -- SMT siblings counted once, capped by the cgroup's CPU quota and by one
    socket's cores and the 16 CPUs a one-GPU box shares -- and half of those, all with
    OMP_PROC_BIND=close OMP_PLACES=cores and the NumPy BLAS threads set to match. value = the
    fastest; when more threads run slower, the record says so (OpenMP threads that fill the
    cgroup's quota are throttled whenever any other thread of the container runs, and each of the
    decode's per-layer parallel regions then waits for the throttled thread)."""
    import subprocess
    from oracle import ref_driver
    if not ref_driver.available():
        log("reference CPU kernels unavailable (not built or no AVX-512 VNNI on this host)")
        return None
    info = ref_driver.cpu_description()
    socket_threads = max(1, min(info["cores_per_socket"], info["usable_cores"], 16))
    log(f"host CPUs: {info}")
    runs = []
    for threads in sorted({4, max(1, socket_threads // 2), socket_threads}):
        env = dict(os.environ)
        env.update(OMP_NUM_THREADS=str(threads), OMP_PROC_BIND="close", OMP_PLACES="cores",
                   OPENBLAS_NUM_THREADS=str(threads), MKL_NUM_THREADS=str(threads))
        cmd = [sys.executable, "-u", "-m", "oracle.ref_driver", "--model", model_path,
               "--prompt", ",".join(str(int(t)) for t in prompt), "--tokens", str(n_tokens)]
        log(f"reference CPU decode, {threads} threads, {n_tokens} steps")
        r = subprocess.run(cmd, cwd=REPO, env=env, capture_output=True, text=True, timeout=600)
        if r.returncode != 0:
            log(f"reference CPU run failed: {r.stderr[-400:]}")
            continue
        d = json.loads(r.stdout.strip().splitlines()[-1])
        runs.append({"threads": threads, "tok_s": round(d["tok_s"], 3), "seconds": round(d["seconds"], 2),
                     "us_per_token": round(1e6 * d["seconds"] / n_tokens, 1)})
        log(f"  {d['tok_s']:.2f} tok/s")
    if not runs:
        return None
    best = max(runs, key=lambda r: r["tok_s"])
    most = max(runs, key=lambda r: r["threads"])
    note = None
    if most is not best:
        note = (f"{most['threads']} threads ran slower than {best['threads']} ({most['tok_s']} against "
                f"{best['tok_s']} tok/s) on {info['usable_cores']} usable cores (cgroup CPU quota "
                f"{info['cgroup_cpu_quota']}): threads that fill the quota are throttled whenever another "
                "thread of the container runs, and each per-layer parallel region waits for the slowest")
        log(note)
    return {"value": best["tok_s"], "unit": "tok/s", "cores": best["threads"], "kind": "reference",
            "sample": f"batch 1, 1.3B shape (the bench's .dfssm file): warm-up step, reset, {len(prompt)}-token "
                      f"prompt untimed, {n_tokens} timed greedy steps of the reference cpu_inference.c "
                      "(HEADDIM 64, AVX-512 VNNI, OpenMP, OMP_PROC_BIND=close OMP_PLACES=cores) + NumPy fp32 "
                      "head; value = the faster of the runs below",
            "runs": runs, "cpu": info, "note": note}


def scaffold_op_bytes(M, N, K):
    """Algorithmic bytes of one dfssm_scaffold_lora_gemm call (acc not written): sign bits, row
    scales, LoRA A + scales, the fp16 LoRA-B table, q + scales, xn, the intermediates h, y."""
    return N * K // 8 + 2 * N + 16 * N + 2 * N + 32 * K + M * K + 2 * M + 2 * M * K + 2 * 16 * M + 2 * M * N


def scaffold_microbench(Ms=(1, 4, 16, 32), min_bytes=1 << 30, reps=3):
    """BASELINE config 1 in isolation: in_proj (K 2048 -> N 8512) and out_proj (K 4096 -> N 2048),
    each call = dfssm_scaffold_lora_gemm (LoRA intermediates + scaffold GEMV/GEMM + LoRA epilogue).
    The calls rotate over distinct weight copies (bits, scales, LoRA A, LoRA-B table) totalling more
    than `min_bytes`, so the weights stream from HBM, not from the 256 MB last-level cache; one graph
    holds one call per copy, timed with HIP events. Returns {proj: {M: result}}."""
    import numpy as np
    import torch
    from dfssm import _C
    lib = _C.lib()
    dev = "cuda:0"
    out = {}
    for name, N, K in (("in_proj", 8512, 2048), ("out_proj", 2048, 4096)):
        tiled = lib.dfssm_tiled_bits_bytes(N, K)
        per_copy = tiled + 2 * N + 16 * N + 2 * N + 32 * K
        n = -(-min_bytes // per_copy)
        g = torch.Generator(device=dev).manual_seed(1)
        bits = torch.randint(-2**31, 2**31 - 1, (n, tiled // 4), dtype=torch.int32, device=dev, generator=g)
        ws = (torch.rand(n, N, device=dev, generator=g) * 0.04 + 0.01).half()
        lA = torch.randint(-127, 128, (n, N, 16), dtype=torch.int8, device=dev, generator=g)
        lAs = (torch.rand(n, N, device=dev, generator=g) * 1.7e-3 + 0.85e-3).half()
        lBq = (torch.randn(n, 16, K, device=dev, generator=g) / (np.sqrt(K))).half()
        res = {}
        for M in Ms:
            xn = torch.randn(M, K, device=dev, generator=g).half()
            q = torch.clamp(torch.round(torch.randn(M, K, device=dev, generator=g) * 40), -127, 127).to(torch.int8)
            xs = (torch.rand(M, device=dev, generator=g) * 0.04 + 0.01).half()
            h = torch.empty(M, 16, dtype=torch.float16, device=dev)
            y = torch.empty(M, N, dtype=torch.float16, device=dev)
            xw = torch.zeros(SCAFFOLD_WS_BYTES // 4, dtype=torch.int32, device=dev)  # exchange workspace

            def call(i):
                _C.check(lib.dfssm_scaffold_lora_gemm(
                    bits[i].data_ptr(), ws[i].data_ptr(), q.data_ptr(), xs.data_ptr(), xn.data_ptr(),
                    lA[i].data_ptr(), lAs[i].data_ptr(), lBq[i].data_ptr(), M, N, K, h.data_ptr(), None,
                    y.data_ptr(), xw.data_ptr(), _C.stream()), "scaffold_lora_gemm")
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                for i in range(n):
                    call(i)
            gr.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                gr.replay()
            e1.record()
            e1.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (reps * n)
            if int(xw[SCAFFOLD_ERR_OFFSET // 4].item()):
                raise RuntimeError("scaffold op: a wait for the LoRA intermediates timed out")
            b = scaffold_op_bytes(M, N, K)
            gbs = b / (us * 1e-6) / 1e9
            res[M] = {"us_per_call": round(us, 3), "bytes_per_call": b, "gbs": round(gbs, 1),
                      "frac": round(gbs / PEAK_GBS, 4), "ops_per_call": 2 * M * N * K,
                      "tops": round(2 * M * N * K / (us * 1e-6) / 1e12, 3), "weight_copies": n,
                      "rotated_bytes": n * per_copy}
            log(f"scaffold {name} M={M}: {us:.2f} us/call, {gbs:.0f} GB/s ({100 * gbs / PEAK_GBS:.1f}% of HBM), "
                f"{n} copies x {per_copy / 1e6:.2f} MB")
        out[name] = res
        del bits, ws, lA, lAs, lBq
        torch.cuda.empty_cache()
    return out


def phase_sweep(B, path, layers=12):
    """Counter-run driver (for rocprofv3 --pmc): the 1.3B model at batch B, 4 prompt tokens
    ingested, then each of the five layer kernels (dfssm_layer_phase) on `layers` layers and the
    head once; no timing, prints a line per stage."""
    import torch
    from dfssm import _C
    from dfssm.synth import make_prompts
    m, _ = build_model(B, path)
    m.ingest(torch.from_numpy(make_prompts(B, m.cfg.vocab_size, 4)), step_by_step=True)
    lib = _C.lib()
    for li in range(layers):
        for ph in range(5):
            _C.check(lib.dfssm_layer_phase(m._model, li, ph, m.x.data_ptr(), m._state, m.workspace.data_ptr(),
                                           _C.stream()))
    _C.check(lib.dfssm_lmhead_argmax(m._model, m.x.data_ptr(), m.workspace.data_ptr(), None, m._next.data_ptr(),
                                     None, _C.stream()))
    torch.cuda.synchronize()
    log(f"phase sweep batch {B}: {layers} layers x 5 kernels + head done")


TIMELINE_STAMPS = {0: "start", 16: "A: x arrived (wave 0)", 18: "A: sum of squares barrier",
                   14: "A: x normalized", 20: "A: amax barrier", 1: "A: prologue done (GEMV workgroups)",
                   2: "A: GEMV done", 3: "A: LoRA h in",
                   4: "A: epilogue / LoRA rank stored", 5: "B: poll start", 6: "B: item inputs in",
                   7: "B: SSM done", 8: "C: prologue start", 17: "C: g arrived (wave 0)", 19: "C: sum of squares barrier",
                   15: "C: g normalized", 21: "C: amax barrier",
                   9: "C: prologue done", 10: "C: GEMV done",
                   11: "C: LoRA h in", 12: "C: epilogue / LoRA rank stored", 13: "end"}


def timeline(B, path, graphs=4):
    """Per-phase wall-clock timeline of the one-launch layer (batch <= 4) from the profiling build
    libdfssm_hip_timeline.so (s_memrealtime stamps per workgroup, 10 ns resolution), measured on the
    last 64 layer launches of `graphs` replays of 8-step decode graphs (warm, as in the timed
    decode). Per stamp: the earliest, median and latest workgroup, in us after the launch's first
    workgroup started, as the median over launches; and the gap from one launch's last workgroup
    to the next launch's first."""
    import numpy as np
    import torch
    from dfssm import _C
    from dfssm import build as dfb
    from dfssm.synth import make_prompts
    if not os.path.exists(dfb.LIB_TIMELINE):
        raise SystemExit(f"{dfb.LIB_TIMELINE} not built (python -m dfssm.build)")
    _C.LIB_PATH = dfb.LIB_TIMELINE
    lib = _C.lib()
    lib.dfssm_timeline_read.restype = ctypes.c_int
    lib.dfssm_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    m, _ = build_model(B, path)
    m.ingest(torch.from_numpy(make_prompts(B, m.cfg.vocab_size, 8)))
    g, _ = m._gen_graph(STEPS_PER_GRAPH)
    for _ in range(graphs):
        g.replay()
    torch.cuda.synchronize()
    buf = np.zeros((64, 256, 24), np.uint64)
    _C.check(lib.dfssm_timeline_read(buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes), "timeline_read")
    names, kernel = TIMELINE_STAMPS, "layer_fused_kernel"
    t = buf.astype(np.int64)
    starts = np.where(t[:, :, 0] > 0, t[:, :, 0], np.iinfo(np.int64).max).min(axis=1)
    ends = t[:, :, 13].max(axis=1)
    order = np.argsort(starts)
    rows = {k: [] for k in names}
    gaps, lengths = [], []
    for i, sl in enumerate(order):
        if starts[sl] == np.iinfo(np.int64).max:
            continue
        lengths.append((ends[sl] - starts[sl]) * 0.01)
        if i > 0:
            gaps.append((starts[sl] - ends[order[i - 1]]) * 0.01)
        for k in names:
            v = t[sl, :, k]
            v = (v[v > 0] - starts[sl]) * 0.01
            if v.size:
                rows[k].append((v.min(), np.median(v), v.max(), v.size))
    out = {"kernel": kernel, "batch": B, "launches": len(lengths), "layer_us_median": round(float(np.median(lengths)), 2),
           "gap_us_median": round(float(np.median(gaps)), 2) if gaps else None, "stamps": {}}
    log(f"timeline {kernel} batch {B}: {len(lengths)} launches, layer {out['layer_us_median']} us (first start to last end), "
        f"gap to the next launch {out['gap_us_median']} us (median; the head runs in one gap per step)")
    meds = {k: np.median(np.array(rows[k]), axis=0) for k in names if rows[k]}
    for k in sorted(meds, key=lambda k: (k == 13, meds[k][1])):  # in time order, the end last
        med, name = meds[k], names[k]
        out["stamps"][name] = {"min": round(float(med[0]), 2), "median": round(float(med[1]), 2),
                               "max": round(float(med[2]), 2), "workgroups": int(med[3])}
        log(f"  {name:46s} min {med[0]:6.2f}  med {med[1]:6.2f}  max {med[2]:6.2f} us  ({int(med[3])} WGs)")
    return out


def decode_only(B, path, shape, graphs):
    """Only the decode step: a seeded 8-token prompt ingested, then `graphs` replays of the 8-step
    decode graph (HIP events around them), nothing else -- the run to trace with rocprofv3 for the
    kernels' durations inside the decode step (the per-kernel timing graphs of time_kernels run one
    kernel back to back, which can rank variants differently)."""
    import torch
    from dfssm.synth import make_prompts
    m, _ = build_model(B, path, shape=shape)
    m.ingest(torch.from_numpy(make_prompts(B, m.cfg.vocab_size, 8)))
    g, _ = m._gen_graph(STEPS_PER_GRAPH)
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(graphs):
        g.replay()
    e1.record()
    e1.synchronize()
    if m.error_flag():
        raise RuntimeError(f"decode reported error flag {m.error_flag():#x}")
    us = e0.elapsed_time(e1) * 1e3 / (graphs * STEPS_PER_GRAPH)
    log(f"decode only, {shape} batch {B}: {us:.1f} us/step, {B * 1e6 / us:.0f} tok/s ({graphs} graphs of "
        f"{STEPS_PER_GRAPH} steps)")
    return {"shape": shape, "batch": B, "us_per_step": round(us, 1), "tok_s": round(B * 1e6 / us, 1)}


def measure(B, path, steps, warmup, shape="1p3b", prompt_len=32):
    """Decode throughput and per-kernel timing at batch B (one model instance)."""
    import torch
    from dfssm.synth import make_prompts
    m, w = build_model(B, path, shape)
    cfg = m.cfg
    prompts = make_prompts(B, cfg.vocab_size, prompt_len)
    pf_ms = time_prefill(m, prompts)
    L, R = cfg.n_layer, B * prompt_len
    pf_ops = 2 * R * L * (cfg.in_proj_out * cfg.d_model + cfg.d_model * cfg.d_inner)
    prefill = {"batch": B, "prompt_tokens": prompt_len, "ms": round(pf_ms, 3),
               "tok_s": round(R / (pf_ms * 1e-3), 1),
               "gemm_ops": pf_ops, "gemm_tops_whole_prefill": round(pf_ops / (pf_ms * 1e-3) / 1e12, 2)}
    log(f"prefill batch {B} x {prompt_len} tokens: {pf_ms:.1f} ms, {prefill['tok_s']:.0f} tok/s")
    ms, nsteps = time_decode(m, prompts, steps, warmup)
    ms_per_step = ms / nsteps
    tok_s = B * nsteps / (ms / 1e3)
    weights, state, per_phase = algorithmic_bytes(cfg, B)
    step_bytes = weights + state
    step_gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"decode batch {B}: {ms_per_step * 1e3:.1f} us/step, {tok_s:.0f} tok/s, "
        f"{step_gbs:.0f} GB/s algorithmic ({100 * step_gbs / PEAK_GBS:.1f}% of HBM peak)")
    if m.error_flag():
        raise RuntimeError(f"decode reported error flag {m.error_flag():#x}")
    samp_ms, samp_us = time_sampled(m, prompts, steps, warmup)
    sampled = {"settings": "temperature 0.7, top-p 0.9, repetition penalty 1.2 (gen_test.py)",
               "ms_per_step": round(samp_ms, 4), "tok_s": round(B / (samp_ms * 1e-3), 1),
               "sample_kernel_us_per_launch": round(samp_us, 2)}
    log(f"sampled decode batch {B}: {samp_ms * 1e3:.1f} us/step, {sampled['tok_s']:.0f} tok/s "
        f"(sampler {samp_us:.1f} us/launch)")
    df_us, df_bytes = time_state_df(m)
    state_df = {"us_per_call": round(df_us, 2), "bytes_per_call": df_bytes,
                "gbs": round(df_bytes / (df_us * 1e-6) / 1e9, 1),
                "note": "quantization of every layer's state at a chunk boundary (once per block_len tokens)"}
    log(f"density-field state batch {B}: {df_us:.1f} us per boundary, {state_df['gbs']:.0f} GB/s")
    kt = time_kernels(m)
    phase_of = {"prep_in": 0, "in_proj+conv": 1, "ssm+gate": 1.5, "prep_out": 2, "out_proj+residual": 2.5,
                "head+argmax": 3, "layer (one launch)": 4, "ssm+prologue": 5, "out_proj+prologue": 6}
    kernels = {}
    for name, (us, n) in kt.items():
        if name == "empty":
            continue
        b = per_phase[phase_of[name]]
        kernels[name] = {"us_per_launch": round(us, 2), "launches_per_step": n,
                         "us_per_step": round(us * n, 1), "bytes_per_launch": b,
                         "gbs": round(b / (us * 1e-6) / 1e9, 1)}
        log(f"  {name:18s} {us:7.2f} us/launch x{n:2d}  {b / 1e6:8.3f} MB  {b / (us * 1e-6) / 1e9:7.1f} GB/s")
    log(f"  empty kernel in the same arrangement: {kt['empty'][0]:.2f} us/launch")
    res = {"batch": B, "tok_s": round(tok_s, 1), "ms_per_step": round(ms_per_step, 4), "steps": nsteps,
           "step_roofline": {"bytes_per_step": step_bytes, "weights": weights, "state": state,
                             "achieved_gbs": round(step_gbs, 1), "frac": round(step_gbs / PEAK_GBS, 4),
                             "roofline_tok_s": round(B / (step_bytes / (PEAK_GBS * 1e9)), 1)},
           "kernels": kernels, "dispatch_us_per_launch": round(kt["empty"][0], 2), "prefill": prefill,
           "sampled": sampled, "state_df": state_df}
    del m
    torch.cuda.empty_cache()
    return res, w, prompts


def copy_calibration(mib):
    """10 copies of `mib` MiB between two device buffers: a kernel whose HBM traffic is known
    (mib MiB read + mib MiB written per launch), to scale the profiler's FETCH_SIZE/WRITE_SIZE."""
    import torch
    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copied {mib} MiB x10")


TRAFFIC_FILE = os.path.join(REPO, "profiles", "hbm_traffic_decode_1p3b.md")


def measured_traffic(batch, phase):
    """HBM bytes per launch of `phase` at `batch` from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, each scaled by a plain copy's reading); None if not profiled."""
    try:
        lines = open(TRAFFIC_FILE).read().splitlines()
    except OSError:
        return None
    for ln in lines:
        cells = [c.strip() for c in ln.strip().strip("|").split("|")]
        if len(cells) == 9 and cells[0] == str(batch) and cells[2] == phase:
            try:
                return int(cells[6])
            except ValueError:
                return None
    return None


PEAK_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA, TOP/s


def mfma_use(res, cfg):
    """int8 matrix-core rate of the batched scaffold GEMMs (2 B N K ops per launch, the
    algorithmic count: padding rows and the +-1 expansion are not counted) against the dense
    int8 peak; batch > 4 only (the one-launch layer at batch <= 4 uses no matrix cores)."""
    B = res["batch"]
    if B <= 4:
        return None
    dims = {"in_proj+conv": (cfg.in_proj_out, cfg.d_model), "out_proj+residual": (cfg.d_model, cfg.d_inner)}
    out = {}
    for name, (N, K) in dims.items():
        us = res["kernels"][name]["us_per_launch"]
        ops = 2 * B * N * K
        tops = ops / (us * 1e-6) / 1e12
        out[name] = {"ops_per_launch": ops, "achieved": round(tops, 2), "peak": PEAK_INT8_TOPS,
                     "unit": "TOP/s", "frac": round(tops / PEAK_INT8_TOPS, 5)}
    return out


def roofline_of(res, name=None):
    ks = res["kernels"]
    dom = name or max(ks, key=lambda k: ks[k]["us_per_step"])
    d = ks[dom]
    return {"bound": "hbm", "kernel": dom, "batch": res["batch"], "achieved": d["gbs"], "peak": PEAK_GBS,
            "unit": "GB/s", "frac": round(d["gbs"] / PEAK_GBS, 4),
            "traffic": measured_traffic(res["batch"], dom),
            "bytes_per_launch": d["bytes_per_launch"], "us_per_launch": d["us_per_launch"]}


def scaffold_roofline(sc):
    """The metric's "scaffold matmul % HBM roofline": the rotated microbench's in_proj call at M = 1."""
    r = sc["in_proj"][1]
    return {"bound": "hbm", "kernel": "dfssm_scaffold_lora_gemm in_proj (K 2048 -> N 8512), M = 1, "
                                      f"{r['weight_copies']} rotated weight copies",
            "achieved": r["gbs"], "peak": PEAK_GBS, "unit": "GB/s", "frac": r["frac"],
            "bytes_per_launch": r["bytes_per_call"], "us_per_launch": r["us_per_call"],
            "traffic": measured_traffic(1, "scaffold in_proj M=1")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--batch", type=int, default=1, help="batch of the headline value")
    ap.add_argument("--batch2", type=int, default=32, help="second batch reported beside it (0: skip)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-steps", type=int, default=128)
    ap.add_argument("--model-path", default=os.path.join(os.environ.get("TMPDIR", "/tmp"), "dfssm_1p3b_seed0.dfssm"))
    ap.add_argument("--config4", type=int, default=1,
                    help="also measure config 4: 2.7B shape, batch 64, 512-token prompt, 256 timed steps (0: skip)")
    ap.add_argument("--model-path-2p7b", default=os.path.join(os.environ.get("TMPDIR", "/tmp"), "dfssm_2p7b_seed0.dfssm"))
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="only run 10 device-to-device copies of this many MiB (counter calibration) and exit")
    ap.add_argument("--phase-sweep", type=int, default=0,
                    help="only run the five layer kernels on 12 layers and the head at this batch (counter runs)")
    ap.add_argument("--scaffold", type=int, default=1, help="run the rotated scaffold microbench (0: skip)")
    ap.add_argument("--scaffold-only", type=int, default=0,
                    help="run only the rotated scaffold microbench at this M (a short program for counter runs)")
    ap.add_argument("--timeline", type=int, default=0,
                    help="only print the per-phase timeline of the one-launch layer at this batch (1..4), "
                         "from the profiling build libdfssm_hip_timeline.so")
    ap.add_argument("--layer-kernel", choices=sorted(LAYER_KERNELS), default="auto",
                    help="layer kernel at batch <= 4 (dfssm_set_layer_kernel; auto: the library's default)")
    ap.add_argument("--decode-only", type=int, default=0,
                    help="only replay the decode graph this many times at --batch (and --shape), for kernel traces")
    ap.add_argument("--shape", choices=("1p3b", "2p7b"), default="1p3b", help="model shape of --decode-only")
    a = ap.parse_args()
    global LAYER_KERNEL
    LAYER_KERNEL = a.layer_kernel
    if a.copy_mib:
        copy_calibration(a.copy_mib)
        return
    if a.phase_sweep:
        phase_sweep(a.phase_sweep, a.model_path)
        return
    if a.timeline:
        print(json.dumps(timeline(a.timeline, a.model_path)), flush=True)
        return
    if a.scaffold_only:
        print(json.dumps(scaffold_microbench(Ms=(a.scaffold_only,))), flush=True)
        return
    if a.decode_only:
        path = a.model_path if a.shape == "1p3b" else a.model_path_2p7b
        print(json.dumps(decode_only(a.batch, path, a.shape, a.decode_only)), flush=True)
        return
    if a.gpus != 1:
        print("bench.py: this build runs on one GPU; multi-GPU decode (data-parallel batch sharding) "
              "(every GPU decoding its own shard of the sequences, no collective in the step) is not measured here",
              file=sys.stderr)
        sys.exit(2)

    main_res, w, prompts = measure(a.batch, a.model_path, a.steps, a.warmup)
    scaffold = scaffold_microbench() if a.scaffold else None
    second = None
    if a.batch2 and a.batch2 != a.batch:
        second, _, _ = measure(a.batch2, a.model_path, a.steps, a.warmup)

    c4 = None
    if a.config4:
        c4, _, _ = measure(64, a.model_path_2p7b, 256, 16, shape="2p7b", prompt_len=512)

    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline(a.model_path, prompts[0], a.cpu_steps)
        if cpu:
            log(f"reference CPU: {cpu['value']} tok/s on {cpu['cores']} threads")

    from dfssm.synth import config_1p3b, config_2p7b
    cfg = config_1p3b()
    B = a.batch
    out = {
        "metric": "decode tok/s, 1.3B-shape b=1 & b=32; scaffold matmul % HBM roofline",
        "value": main_res["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": main_res["steps"], "warmup": a.warmup,
        "ms_per_step": main_res["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded random-init weights of the 1.3B shape, .dfssm file; seeded prompts)",
        "config": {"workload": f"config3: 1.3B-shape DF-SSM greedy decode, batch {B}, 32-token prompt "
                               f"ingested, {main_res['steps']} timed steps", "batch": B, "d_model": cfg.d_model,
                   "n_layer": cfg.n_layer, "d_inner": cfg.d_inner, "nheads": cfg.nheads, "headdim": cfg.p,
                   "d_state": cfg.d_state, "vocab": cfg.vocab_size, "embedding": "int8+row scale",
                   "arith": "1-bit x int8 scaffold (int32 acc), fp16 activations, fp32 SSM state"},
        "roofline": roofline_of(main_res),
        "scaffold_roofline": scaffold_roofline(scaffold) if scaffold else roofline_of(main_res, "in_proj+conv"),
        "scaffold_microbench": scaffold,
        "step_roofline": main_res["step_roofline"],
        "kernels": main_res["kernels"],
        "cpu_baseline": cpu,
        "prefill": main_res["prefill"],
        "sampled": main_res["sampled"],
        "state_df": main_res["state_df"],
    }
    if second:
        out["batch2"] = {"batch": second["batch"], "tok_s": second["tok_s"], "ms_per_step": second["ms_per_step"],
                         "step_roofline": second["step_roofline"], "roofline": roofline_of(second),
                         "scaffold_roofline": roofline_of(second, "in_proj+conv"), "mfma": mfma_use(second, cfg),
                         "kernels": second["kernels"], "prefill": second["prefill"], "sampled": second["sampled"]}
    if c4:
        out["config4"] = {"workload": "config4: 2.7B-shape DF-SSM greedy decode, batch 64, 512-token prompt "
                                      "ingested, 256 timed steps", "batch": 64, "tok_s": c4["tok_s"],
                          "ms_per_step": c4["ms_per_step"], "step_roofline": c4["step_roofline"],
                          "roofline": roofline_of(c4), "mfma": mfma_use(c4, config_2p7b()), "kernels": c4["kernels"],
                          "prefill": c4["prefill"]}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
