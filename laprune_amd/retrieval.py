"""Decode-step KV retrieval: selection arithmetic, keep set and the fused pipeline.

Mirrors ``_decode_attention`` of laprune/llm/modifiers/aq_evaluation.py:146-253
for one layer and one decode token:

  1. LUT            lut[h,m,k] = q_h . C_m[k]                (lap_lut_build)
  2. score          s[h,t] = sum_m lut[h,m,code[t,m]]         (fused scorer)
  3. select         top-k over the candidate window           (radix top-k)
  4. attend         softmax(q.K_S) V_S over top-k ++ sink ++ local, K/V read
                    in place from the cache                   (sparse decode)

Two selection modes:
  * ``"head"``: one top-k per query head, as the reference
    (aq_evaluation.py:198-202), k from ``mask_out``/``min_remain`` unless a
    fixed budget is given;
  * ``"group"``: one top-k per KV group on the max over its G query-head
    scores (the configs' group-max mode); K/V rows are then read once per
    group.
Every buffer is preallocated so that ``step`` can be captured in a HIP graph
(``torch.cuda.CUDAGraph``); no step allocates.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _native as N


@dataclass
class RetrievalConfig:
    """Hot-path keys of the reference's ``draft_kwargs`` (defaults as in the
    code, aq_evaluation.py:185-188)."""

    mask_out: float = 0.98
    min_remain: int = 20
    sink_size: int = 4
    local_window: int = 64
    topk: int | None = None          # fixed budget; None -> mask_out rule
    select: str = "group"            # "group" | "head"
    score_dtype: torch.dtype = torch.float16  # rank dtype (bf16 = model-dtype cast)

    def __post_init__(self):
        if self.select not in ("group", "head"):
            raise ValueError("select must be 'group' or 'head'")


def candidate_window(t_codes: int, t_total: int, sink: int, local: int) -> tuple[int, int]:
    """Candidate columns [cand_start, cand_end) (aq_evaluation.py:189-193)."""
    sink_end = min(sink, t_codes) if sink > 0 else 0
    local_start = max(t_total - max(local, 0), 0)
    cand_start = sink_end
    cand_end = min(t_codes, local_start) if local > 0 else t_codes
    return cand_start, max(cand_start, cand_end)


def budget_k(n: int, mask_out: float, min_remain: int) -> int:
    """Number of candidates kept (aq_evaluation.py:195-197)."""
    if n <= 0:
        return 0
    k = n - int(n * mask_out)
    k = max(min(n, min_remain), k)
    return max(1, min(k, n))


def keep_segments(t_total: int, sink: int, local: int) -> tuple[int, int, int]:
    """(sink_count, tail_start, tail_count) of the keep set (aq_evaluation.py:211-218).

    The keep set is top-k ++ [0, sink_count) ++ [tail_start, t_total); the
    three parts are disjoint because the candidate window excludes both
    windows."""
    sb = min(sink, t_total) if sink > 0 else 0
    start = max(t_total - local, 0) if local > 0 else t_total
    if start <= 0:
        sb_eff = 0
    else:
        sb_eff = sb
        start = max(start, sb_eff)
    tail_count = t_total - start if (local > 0 and start < t_total) else 0
    return sb_eff, start, tail_count


class SparseDecoder:
    """Preallocated single-layer retrieval + sparse attention for one decode step.

    Args:
      codebooks: [M=32, K=256, D] fp32 (or fp16) AQ codebooks on the GPU.
      batch, num_q_heads, num_kv_heads, head_dim: attention geometry (G = 4).
      max_tokens: largest cache length the step will see (sizes scratch).
      cfg: selection settings.
    """

    M, K = 32, 256

    def __init__(self, codebooks: torch.Tensor, batch: int, num_q_heads: int,
                 num_kv_heads: int, head_dim: int, max_tokens: int,
                 cfg: RetrievalConfig | None = None, dtype: torch.dtype = torch.bfloat16):
        N.lib()
        N.require_cuda(codebooks)
        if tuple(codebooks.shape) != (self.M, self.K, head_dim):
            raise RuntimeError(f"codebooks must be [32, 256, {head_dim}]")
        if num_q_heads != 4 * num_kv_heads:
            raise RuntimeError("the fused scorer serves G = 4 query heads per KV head")
        self.cfg = cfg or RetrievalConfig()
        self.dev = codebooks.device
        self.cb = codebooks.contiguous()
        self.B, self.Hq, self.Hkv, self.D = batch, num_q_heads, num_kv_heads, head_dim
        self.G = num_q_heads // num_kv_heads
        self.T_max = max_tokens
        self.dtype = dtype
        R = batch * num_kv_heads
        self.lut = torch.empty((R, self.M, self.K, 4), dtype=torch.float16, device=self.dev)
        k_cap = self._k_cap(max_tokens)
        rows = num_kv_heads if self.cfg.select == "group" else num_q_heads
        self.idx = torch.empty((batch, rows, max(k_cap, 1)), dtype=torch.int32, device=self.dev)
        self.out = torch.empty((batch, num_q_heads, head_dim), dtype=dtype, device=self.dev)
        self.scores = None
        if self.cfg.select == "head":
            self.scores = torch.empty((batch, num_q_heads, max_tokens), dtype=torch.float16,
                                      device=self.dev)
        ws_r = N.size_query("lap_retrieve_workspace_size", R, max_tokens)
        ws_t = N.size_query("lap_topk_workspace_size", batch * num_q_heads, max_tokens)
        self.ws_sel = torch.empty(max(ws_r, ws_t, 1), dtype=torch.uint8, device=self.dev)
        max_keep = k_cap + self.cfg.sink_size + max(self.cfg.local_window, 0)
        ws_a = N.size_query("lap_attn_decode_workspace_size", batch, num_q_heads, head_dim,
                            max(max_keep, 1))
        self.ws_attn = torch.zeros(max(ws_a, 1), dtype=torch.uint8, device=self.dev)  # counters start at 0
        self.key_mode = N.KEY_BF16 if self.cfg.score_dtype == torch.bfloat16 else N.KEY_F16
        self.last_k = 0

    def _k_cap(self, t: int) -> int:
        cs, ce = candidate_window(t, t, self.cfg.sink_size, self.cfg.local_window)
        n = ce - cs
        if self.cfg.topk is not None:
            return min(self.cfg.topk, n)
        return max(budget_k(n, self.cfg.mask_out, self.cfg.min_remain),
                   budget_k(self.T_max, self.cfg.mask_out, self.cfg.min_remain))

    def plan(self, t_codes: int, t_total: int) -> dict:
        """Host-side selection arithmetic for one step (no device work)."""
        c = self.cfg
        cs, ce = candidate_window(t_codes, t_total, c.sink_size, c.local_window)
        n = ce - cs
        k = min(c.topk, n) if c.topk is not None else budget_k(n, c.mask_out, c.min_remain)
        sink, tail_start, tail_count = keep_segments(t_total, c.sink_size, c.local_window)
        return dict(cand_start=cs, cand_end=ce, k=k, sink=sink, tail_start=tail_start,
                    tail_count=tail_count)

    @torch.no_grad()
    def step(self, q: torch.Tensor, codes: torch.Tensor, keys: torch.Tensor,
             vals: torch.Tensor, t_codes: int | None = None,
             t_total: int | None = None) -> torch.Tensor:
        """One decode step.

        q: [B, Hq, 1, D] (or [B, Hq, D]) post-RoPE query; codes: u8 [B, Hkv, >=t_codes, 32];
        keys/vals: [B, Hkv, >=t_total, D] post-RoPE cache views.  Returns [B, Hq, 1, D].
        """
        if q.dim() == 4:
            q = q[:, :, 0, :]
        B, Hq, Hkv, D = self.B, self.Hq, self.Hkv, self.D
        t_codes = codes.shape[2] if t_codes is None else t_codes
        t_total = keys.shape[2] if t_total is None else t_total
        if t_total > self.T_max or t_codes > t_total:
            raise RuntimeError("cache length exceeds the decoder's max_tokens")
        p = self.plan(t_codes, t_total)
        st = N.stream_of(q)
        qf = q.reshape(B * Hq, D) if q.is_contiguous() else q.contiguous().reshape(B * Hq, D)
        N.call("lap_lut_build", N.ptr(qf), N.dtype_code(qf.dtype), qf.stride(0), N.ptr(self.cb),
               N.dtype_code(self.cb.dtype), B * Hq, D, self.M, self.K, 4, N.LUT_GMKG,
               N.ptr(self.lut), st)
        k = p["k"] if t_codes > 0 else 0
        self.last_k = k
        if k == 0:
            H_idx = Hkv if self.cfg.select == "group" else Hq  # sink + local only
        elif self.cfg.select == "group":
            N.call("lap_retrieve_topk", N.ptr(self.lut), N.ptr(codes), codes.stride(0),
                   codes.stride(1), codes.stride(2), B, Hkv, t_codes, p["cand_start"],
                   p["cand_end"], k, self.key_mode, None, N.ptr(self.idx), N.I32,
                   N.ptr(self.ws_sel), self.ws_sel.numel(), st)
            H_idx = Hkv
        else:
            sc = self.scores
            N.call("lap_retrieve_topk", N.ptr(self.lut), N.ptr(codes), codes.stride(0),
                   codes.stride(1), codes.stride(2), B, Hkv, t_codes, p["cand_start"],
                   p["cand_end"], 0, self.key_mode, N.ptr(sc), N.ptr(self.idx), N.I32,
                   N.ptr(self.ws_sel), self.ws_sel.numel(), st)
            # per-head selection over the fp16 head scores (scores row stride = T_max)
            if B != 1:
                raise RuntimeError("per-head selection serves batch 1")
            N.call("lap_topk_select", N.ptr(sc), sc.stride(1), Hq, 1, t_codes, p["cand_start"],
                   p["cand_end"], k, self.key_mode, N.ptr(self.idx), N.I32,
                   N.ptr(self.ws_sel), self.ws_sel.numel(), st)
            H_idx = Hq
        scale = 1.0 / math.sqrt(D)
        N.call("lap_sparse_attn_decode", N.ptr(q), q.stride(0), q.stride(1), N.ptr(keys),
               N.ptr(vals), N.dtype_code(q.dtype), B, Hq, Hkv, t_total, D, keys.stride(0),
               keys.stride(1), keys.stride(2), vals.stride(0), vals.stride(1), vals.stride(2),
               N.ptr(self.idx), N.I32, H_idx, k, p["sink"], p["tail_start"], p["tail_count"],
               scale, N.ptr(self.out), N.ptr(self.ws_attn), self.ws_attn.numel(), st)
        return self.out.unsqueeze(2)

    @torch.no_grad()
    def step_cached(self, q: torch.Tensor, cache) -> torch.Tensor:
        """One decode step over a ``DecodeKVCache``: candidates are the encoded
        tokens (``encoded_len``), attention covers all ``length`` tokens."""
        return self.step(q, cache.codes, cache.k, cache.v, t_codes=cache.encoded_len,
                         t_total=cache.length)

    def selected(self) -> torch.Tensor:
        """Indices chosen by the last step: [B, rows, k] int32 (ascending)."""
        return self.idx[:, :, :self.last_k]


class DenseDecoder:
    """Preallocated dense single-query decode (the comparator)."""

    def __init__(self, batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                 max_tokens: int, device: torch.device, dtype: torch.dtype = torch.bfloat16):
        N.lib()
        self.B, self.Hq, self.Hkv, self.D = batch, num_q_heads, num_kv_heads, head_dim
        self.out = torch.empty((batch, num_q_heads, head_dim), dtype=dtype, device=device)
        ws = N.size_query("lap_attn_decode_workspace_size", batch, num_q_heads, head_dim,
                          max(max_tokens, 1))
        self.ws = torch.zeros(max(ws, 1), dtype=torch.uint8, device=device)  # counters start at 0

    @torch.no_grad()
    def step(self, q: torch.Tensor, keys: torch.Tensor, vals: torch.Tensor) -> torch.Tensor:
        if q.dim() == 4:
            q = q[:, :, 0, :]
        B, Hq, Hkv, D = self.B, self.Hq, self.Hkv, self.D
        T = keys.shape[2]
        N.call("lap_dense_attn_decode", N.ptr(q), q.stride(0), q.stride(1), N.ptr(keys),
               N.ptr(vals), N.dtype_code(q.dtype), B, Hq, Hkv, T, D, keys.stride(0),
               keys.stride(1), keys.stride(2), vals.stride(0), vals.stride(1), vals.stride(2),
               1.0 / math.sqrt(D), N.ptr(self.out), N.ptr(self.ws), self.ws.numel(),
               N.stream_of(q))
        return self.out.unsqueeze(2)
