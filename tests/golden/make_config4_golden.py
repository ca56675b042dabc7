"""Write tests/golden/oracle_2p7b_64layer_b4.npz: the oracle's (oracle/oracle.py OracleModel) greedy
decode of the full config-4 model -- the 2.7B shape with all 64 layers and the 50288-token
vocabulary, weights make_weights(config_2p7b(), seed 0), the model bench.py measures -- at batch 4,
so that the GPU path at full depth (64 layers of launch tags, the prefill's wide GEMMs over
>= 256-row chunks at d_model 2560) is checked against it without running the oracle on the GPU box
(one run takes ~90 s on this container's CPU).

Protocol: prompt = make_prompts(4, 50288, 129); the oracle consumes it step by step and then decodes
greedily, generate(prompt, 4) (129 + 3 steps); then one more step on the last generated token, whose
logits and resulting state are hashed.

Contents:
  prompt       (4, 129) int64
  tokens       (4, 4) int64   the 4 greedy tokens
  next_token   (4,) int64     the greedy token after the extra step
  logits_sha256  ()  str      SHA-256 of the extra step's (4, 50288) fp16 logits, C order
  state_sha256   ()  str      SHA-256 of the fp32 SSM state after it, (64, 4, 80, 64, 128) C order
  conv_sha256    ()  str      SHA-256 of the fp16 conv state after it, (64, 4, 5376, 3) C order
  logits_head  (4, 8) fp16    logits[:, :8] (a readable excerpt)

    python tests/golden/make_config4_golden.py
"""
import hashlib
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "df-ssm_amd"))
sys.path.insert(0, REPO)

from dfssm.synth import config_2p7b, make_prompts, make_weights  # noqa: E402
from oracle import oracle as O  # noqa: E402

OUT = os.path.join(HERE, "oracle_2p7b_64layer_b4.npz")
B, T, N_NEW = 4, 129, 4


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main():
    t0 = time.time()
    w = make_weights(config_2p7b(), seed=0)
    prompt = make_prompts(B, w.cfg.vocab_size, T)
    orc = O.OracleModel(w, B)
    tokens, _ = orc.generate(prompt, N_NEW)
    logits, nxt = orc.step(tokens[:, -1])
    np.savez(OUT, prompt=prompt, tokens=tokens, next_token=np.asarray(nxt, np.int64),
             logits_sha256=np.array(sha(np.asarray(logits, np.float16))),
             state_sha256=np.array(sha(np.asarray(orc.h, np.float32))),
             conv_sha256=np.array(sha(np.asarray(orc.conv, np.float16))),
             logits_head=np.asarray(logits, np.float16)[:, :8])
    print(f"wrote {OUT} ({time.time() - t0:.0f} s): tokens {tokens.tolist()}")


if __name__ == "__main__":
    main()
