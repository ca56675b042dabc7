"""Write tests/golden/ref_cpu_1p3b_2layer.npz: outputs of the reference's own compiled CPU decode
kernels (inference/cpu/cpu_inference.c, built into oracle/_ref by oracle/build_ref.sh with
HEADDIM 64) on seeded inputs, so that the oracle's CPU-numerics restatement stays pinned on hosts
where the reference cannot be built or run.

Contents (all inputs are regenerated from the seeds by dfssm.synth):
  logits      (8, 4096) fp32  RefCPUModel.forward for the 8 prompt tokens, in order; model =
                              make_weights(1.3B layer dims, n_layer 2, vocab 4096, seed 11),
                              prompt = make_prompts(1, 4096, 8)[0]
  h_sum, h_sq (2, 64)   fp64  per layer and head: sum and sum of squares of the SSM state after
                              the 8 tokens
  conv_sum, conv_sq (2,) fp64  per layer: sum and sum of squares of the conv state
  acc_in      (8512,) int32   scaffold_matvec_avx512 on the integer input of
                              test_int32_accumulators_bit_exact_through_reference (seed [7, 0])
    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "df-ssm_amd"))
sys.path.insert(0, REPO)

from dfssm.format import DFSSMConfig, EMB_I8  # noqa: E402
from dfssm.synth import make_prompts, make_weights  # noqa: E402

OUT = os.path.join(HERE, "ref_cpu_1p3b_2layer.npz")


def golden_config():
    return DFSSMConfig(n_layer=2, d_model=2048, d_inner=4096, d_state=128, nheads=64, headdim=64,
                       ngroups=1, vocab_size=4096, kw=4, emb_code=EMB_I8)


def scaffold_case():
    """bits (8512, 64) and x (2048,) fp32 integer-valued plus one 127.5, the exact int input."""
    rng = np.random.default_rng([7, 0])
    bits = rng.integers(0, 2 ** 32, (8512, 64), dtype=np.uint32)
    xi = rng.integers(-127, 128, 2048).astype(np.float32)
    x = xi.copy()
    x[5] = 127.5
    xi[5] = 127
    return bits, x, xi.astype(np.int8)


def main():
    import ctypes
    from oracle import ref_driver
    if not ref_driver.available():
        sys.exit("reference CPU kernels not built (oracle/build_ref.sh) or no AVX-512 VNNI on this host")
    w = make_weights(golden_config(), seed=11)
    m = ref_driver.RefCPUModel(w)
    prompt = make_prompts(1, w.cfg.vocab_size, 8)[0]
    logits = np.stack([m.forward(int(t)) for t in prompt]).astype(np.float32)
    h = m.h.astype(np.float64)
    bits, x, _ = scaffold_case()
    lib = ctypes.CDLL(ref_driver.LIB_PATH)
    rs = np.empty(8512, np.int32)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    lib.precompute_row_sums(p(bits), p(rs), 8512, 64)
    out = np.empty(8512, np.float32)
    lib.ref_scaffold_matvec(p(bits), p(x), p(np.ones(8512, np.float32)), p(rs), p(out), 8512, 64)
    np.savez_compressed(OUT, logits=logits, h_sum=h.sum(axis=(2, 3)), h_sq=(h * h).sum(axis=(2, 3)),
                        conv_sum=m.conv.astype(np.float64).sum(axis=(1, 2)),
                        conv_sq=(m.conv.astype(np.float64) ** 2).sum(axis=(1, 2)), acc_in=out.astype(np.int32),
                        prompt=prompt)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} B)")


if __name__ == "__main__":
    main()
