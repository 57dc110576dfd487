"""Write tests/golden/retrieval_small.npz from the CPU oracle.

Inputs are seeded; outputs are the oracle's (oracle/aq_oracle.c) for the
explicit-order contracts.  The reference tree holds no test vectors, so these
fixtures pin this build against its own oracle across changes (regression),
on the CPU and on the GPU.

    python tests/golden/make_golden.py
"""
from pathlib import Path
import sys

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import orc  # noqa: E402

OUT = Path(__file__).with_name("retrieval_small.npz")


def make():
    g = torch.Generator().manual_seed(2024)
    # retrieval: the fast scorer's geometry (G=4, M=32, K=256) with a short
    # head dim so the fixture stays small; codebook values are bf16-exact and
    # stored as their 16-bit patterns
    Hq, Hkv, T, D, M, K = 8, 2, 512, 16, 32, 256
    q = torch.randn(Hq, D, generator=g).bfloat16()
    cb = (torch.randn(M, K, D, generator=g) * 0.2).bfloat16()
    codes = torch.randint(0, 256, (Hkv, T, M), generator=g, dtype=torch.uint8).numpy()
    lut = orc.lut_build(q.float().numpy(), cb.float().numpy())
    scores = orc.score_grouped(lut, codes, 4)
    cs, ce = orc.candidate_window(T, T, 4, 64)
    k = orc.budget_k(ce - cs)
    idx_head = orc.topk(scores, k, 1, cs, ce)
    idx_group = orc.topk(scores, 64, 4, cs, ce, key_bf16=True)
    # encode: small codebooks, head dim 64
    ecb = torch.randn(4, 64, 64, generator=g) * 0.3
    x = (torch.randn(16, 64, generator=g) * (torch.rand(64, generator=g) * 3.5 + 0.5)).numpy()
    enc_codes, enc_rnorm = orc.encode(x, ecb.numpy())
    np.savez_compressed(
        OUT, q_bf16=q.view(torch.int16).numpy(), cb_bf16=cb.view(torch.int16).numpy(),
        codes=codes, lut=lut, scores=scores, cand=np.array([cs, ce, k]), idx_head=idx_head,
        idx_group=idx_group, enc_cb=ecb.numpy(), x=x, enc_codes=enc_codes,
        enc_rnorm=enc_rnorm)
    return OUT


if __name__ == "__main__":
    print(make())
