"""The reference's fp32 / CPU PyTorch path, restated — TEST INFRASTRUCTURE ONLY.

Used by bench.py's cpu_baseline leg (timed on the host cores) and by tests
that compare the GPU selection against the fp32 path tie-aware.  It follows
the reference code step by step (no reference code is imported):

  scoring   laprune/llm/aq_kv.py:696-699 (expand KV-group codes to query
            heads) then :614-628 (q_chunk = 512 if N <= 8192 else 64,
            token_chunk = 8192, einsum "mkd,qd->qmk", int64 gather over m,
            sum(dim=1)) in fp32
  select    laprune/llm/modifiers/aq_evaluation.py:166 (cast to the model
            dtype), :185-201 (candidate window, budget, topk(sorted=False))
  encode    laprune/quantizer.py:346-355 (greedy, iters = 0) in fp32
"""
from __future__ import annotations

import torch


def scores_fp32(q: torch.Tensor, codebooks: torch.Tensor, codes_kv: torch.Tensor,
                group: int) -> torch.Tensor:
    """q [Hq, d] fp32, codebooks [M, K, d] fp32, codes_kv [Hkv, N, M] u8 -> [Hq, N] fp32."""
    hkv, n, m = codes_kv.shape
    hq = q.shape[0]
    codes = codes_kv.reshape(hkv, 1, n, m).expand(hkv, group, n, m).reshape(hq, n, m)
    q_chunk = 512 if n <= 8192 else 64
    token_chunk = 8192
    out = torch.empty((hq, n), dtype=q.dtype)
    for start in range(0, hq, q_chunk):
        end = min(start + q_chunk, hq)
        lut_sub = torch.einsum("mkd,qd->qmk", codebooks, q[start:end])
        for ts in range(0, n, token_chunk):
            te = min(ts + token_chunk, n)
            codes_sub = codes[start:end, ts:te, :].to(torch.long)
            gathered = lut_sub.gather(dim=2, index=codes_sub.permute(0, 2, 1))
            out[start:end, ts:te] = gathered.sum(dim=1)
    return out


def select_topk(scores: torch.Tensor, model_dtype: torch.dtype, t_total: int, sink: int = 4,
                local: int = 64, mask_out: float = 0.98, min_remain: int = 20,
                k: int | None = None) -> torch.Tensor:
    """Per-row top-k over the candidate window, indices offset by cand_start."""
    s = scores.to(model_dtype)
    t_codes = s.shape[-1]
    sink_end = min(sink, t_codes) if sink > 0 else 0
    local_start = max(t_total - max(local, 0), 0)
    cs = sink_end
    ce = min(t_codes, local_start) if local > 0 else t_codes
    n = max(0, ce - cs)
    if k is None:
        k = n - int(n * mask_out)
        k = max(min(n, min_remain), k)
        k = max(1, min(k, n))
    idx = torch.topk(s[..., cs:ce], k=min(k, n), dim=-1, sorted=False).indices
    return idx + cs


def encode_fp32(x: torch.Tensor, codebooks: torch.Tensor) -> torch.Tensor:
    """Greedy AQ codes, laprune/quantizer.py:346-355 (iters = 0)."""
    m_cb = codebooks.shape[0]
    norms = [torch.sum(cb ** 2, dim=1) for cb in codebooks]
    cbt = [cb.T.clone() for cb in codebooks]
    codes = torch.zeros(x.shape[0], m_cb, dtype=torch.long)
    residual = x.clone()
    for m in range(m_cb):
        r_norm = torch.sum(residual ** 2, dim=1, keepdim=True)
        dists = r_norm + norms[m].unsqueeze(0) - 2 * (residual @ cbt[m])
        codes[:, m] = torch.argmin(dists, dim=1)
        residual -= codebooks[m][codes[:, m]]
    return codes
