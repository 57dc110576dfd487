"""Seeded synthetic inputs shared by the GPU parity tests.

* ``gaussian_codebooks``: the configs' codebooks, fp32 N(0, 0.02) [32, 256, D].
* ``residual_codebooks``: codebooks with the magnitudes of trained,
  residual-ordered ones.  The reference's shipped Llama-3.1 codebooks
  (loaded by laprune/llm/aq_kv.py:277-342) have stage norms that fall from
  about 11.5 (m = 0) to about 2.2 (m = 31) and an absolute maximum near 9.
  Here stage m's entries are unit-variance Laplace draws times a
  per-channel scale (U(0.5, 2), normalised to unit mean square), scaled so
  the mean entry norm of stage m is 11.5 * (2.2 / 11.5) ** (m / 31).  The
  Laplace tails and heavy channels put the largest entries near 9-10.  No
  reference file is read.
* ``c3_keys``: BASELINE config C3's post-RoPE keys (pre-RoPE bf16 N(0, 1) x
  per-channel U(0.5, 4), rotate-half RoPE with theta 500000).
"""
from __future__ import annotations

import torch

STAGE_NORM_FIRST, STAGE_NORM_LAST = 11.5, 2.2


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def gaussian_codebooks(seed: int, D: int = 128, M: int = 32, K: int = 256,
                       std: float = 0.02) -> torch.Tensor:
    return torch.randn(M, K, D, generator=gen(seed)) * std


def stage_norms(M: int = 32) -> torch.Tensor:
    m = torch.arange(M, dtype=torch.float64)
    return STAGE_NORM_FIRST * (STAGE_NORM_LAST / STAGE_NORM_FIRST) ** (m / max(M - 1, 1))


def residual_codebooks(seed: int, D: int = 128, M: int = 32, K: int = 256) -> torch.Tensor:
    g = gen(seed)
    ch = torch.rand(D, generator=g, dtype=torch.float64) * 1.5 + 0.5
    ch = ch / ch.pow(2).mean().sqrt()
    u = torch.rand(M, K, D, generator=g, dtype=torch.float64) - 0.5
    z = -torch.sign(u) * torch.log1p(-2 * u.abs()) / 2 ** 0.5 * ch
    norms = z.norm(dim=-1).mean(dim=-1)  # mean entry norm per stage
    cb = z * (stage_norms(M) / norms)[:, None, None]
    return cb.float()


def rope_rotate_half(k: torch.Tensor, positions: torch.Tensor, theta: float) -> torch.Tensor:
    """HF rotate-half RoPE of k [..., T, D] at integer positions [T] (float64
    angles, rounded once to float32 like the model's cos/sin tables)."""
    D = k.shape[-1]
    inv = theta ** (-torch.arange(0, D, 2, dtype=torch.float64) / D)
    ang = positions.to(torch.float64)[:, None] * inv[None, :]
    cos = torch.cat([ang.cos(), ang.cos()], -1).float()
    sin = torch.cat([ang.sin(), ang.sin()], -1).float()
    rot = torch.cat([-k[..., D // 2:], k[..., :D // 2]], -1)
    return k * cos + rot * sin


def c3_keys(seed: int, Hkv: int = 8, n_tok: int = 64, D: int = 128,
            first_pos: int = 131008) -> torch.Tensor:
    g = gen(seed)
    k = (torch.randn(Hkv, n_tok, D, generator=g) *
         (torch.rand(D, generator=g) * 3.5 + 0.5)).bfloat16().float()
    pos = torch.arange(first_pos, first_pos + n_tok)
    return rope_rotate_half(k, pos, 500000.0).reshape(-1, D)
