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

Ragged batches: ``step`` also takes one length per sequence (lists for
``t_codes`` / ``t_total``).  The reference decodes a batch with one shared
length (aq_evaluation.py:150-155); here every sequence gets the window,
budget and keep set it would get alone, through per-sequence plans
(``lap_row_plan``) uploaded to the device before the kernels that read them.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _native as N
from ._ops import ops


class StepHealthError(RuntimeError):
    """A one-launch decode step ran outside its guarantees: a KV row whose
    workgroups did not all run on one XCD (their exchange through that XCD's
    L2 is then unguaranteed), or a row barrier that gave up waiting.  The
    results of the steps since the workspace was last zeroed are not to be
    trusted; zero the workspace (``SparseDecoder.reset_health``) before the
    next step."""


def check_step_health(split_rows: int, timeouts: int, who: str) -> None:
    """Raise :class:`StepHealthError` naming the counts when either health
    counter of the one-launch step is non-zero (the status words of
    ``lap_decode_step_status``); return quietly when both are zero."""
    if split_rows or timeouts:
        raise StepHealthError(
            f"{who}: the one-launch decode step is unhealthy: {split_rows} KV row(s) ran "
            f"their workgroups on more than one XCD and {timeouts} row barrier(s) timed out; "
            f"the selections and attention outputs since the workspace was zeroed are "
            f"undefined")


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


def keep_plan(k: int, t_total: int, sink: int, local: int) -> tuple[int, int, int]:
    """(sink_count, tail_start, tail_count) of a step that selects k
    candidates.  As keep_segments, except that a step with no selected
    candidate, no sink and no local window keeps the newest token instead of
    nothing (aq_evaluation.py:233-234)."""
    sb, start, tail = keep_segments(t_total, sink, local)
    if k <= 0 and sb == 0 and tail == 0 and t_total > 0:
        return 0, t_total - 1, 1
    return sb, start, tail


PLAN_FIELDS = ("t_codes", "t_total", "cand_start", "cand_end", "k", "sink", "tail_start",
               "tail_count")


class PlanBuffer:
    """Device array of ``lap_row_plan`` [B] written from the host each step.

    Uploads go through a ring of pinned staging buffers; a slot is rewritten
    only after the copy that last read it has completed (its event), so the
    host may run ahead of the device."""

    SLOTS = 4

    def __init__(self, batch: int, device: torch.device):
        self.dev = torch.zeros((batch, len(PLAN_FIELDS)), dtype=torch.int32, device=device)
        self._host = [torch.zeros((batch, len(PLAN_FIELDS)), dtype=torch.int32).pin_memory()
                      for _ in range(self.SLOTS)]
        self._done = [None] * self.SLOTS
        self._i = 0

    def upload(self, rows: list[tuple[int, ...]]) -> torch.Tensor:
        i = self._i
        self._i = (i + 1) % self.SLOTS
        if self._done[i] is not None:
            self._done[i].synchronize()
        h = self._host[i]
        h.copy_(torch.tensor(rows, dtype=torch.int32))
        self.dev.copy_(h, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.dev.device))
        self._done[i] = ev
        return self.dev


def _per_row(v, B: int, name: str) -> list[int] | None:
    """A per-sequence length argument as a list of B ints (None stays None)."""
    if v is None:
        return None
    if isinstance(v, torch.Tensor):
        v = v.tolist()
    if isinstance(v, int):
        return [v] * B
    v = [int(x) for x in v]
    if len(v) != B:
        raise RuntimeError(f"{name} needs one length per sequence ({B}), got {len(v)}")
    return v


class SparseDecoder:
    """Preallocated single-layer retrieval + sparse attention for one decode step.

    Args:
      codebooks: [M=32, K=256, D] fp32 (or fp16) AQ codebooks on the GPU.
      batch, num_q_heads, num_kv_heads, head_dim: attention geometry; G = Hq / Hkv
        from 1 to 8 (G = 4 with D = 128 runs the one-launch step, other
        shapes the kernel chain).
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
        if num_kv_heads <= 0 or num_q_heads % num_kv_heads or \
                not 1 <= num_q_heads // num_kv_heads <= 8:
            raise RuntimeError("the decode step serves G = 1 to 8 query heads per KV head")
        self.cfg = cfg or RetrievalConfig()
        self.dev = codebooks.device
        self.cb = codebooks.contiguous()
        self.B, self.Hq, self.Hkv, self.D = batch, num_q_heads, num_kv_heads, head_dim
        self.G = num_q_heads // num_kv_heads
        self.T_max = max_tokens
        self.dtype = dtype
        R = batch * num_kv_heads
        # G = 4: the interleaved [B * Hkv, M, K, 4] table of the fused scorer;
        # other G: the per-head [B * Hq, M, K] table of the kernel chain
        if self.G == 4:
            self.lut_layout = N.LUT_GMKG
            self.lut = torch.empty((R, self.M, self.K, 4), dtype=torch.float16, device=self.dev)
        else:
            self.lut_layout = N.LUT_HMK
            self.lut = torch.empty((batch * num_q_heads, self.M, self.K), dtype=torch.float16,
                                   device=self.dev)
        k_cap = self._k_cap(max_tokens)
        # selection rows per batch row: KV groups (group max) or query heads
        rows = num_kv_heads if self.cfg.select == "group" else num_q_heads
        self.H_idx = rows
        self.idx = torch.empty((batch, rows, max(k_cap, 1)), dtype=torch.int32, device=self.dev)
        self.out = torch.empty((batch, num_q_heads, head_dim), dtype=dtype, device=self.dev)
        # the tail holds the local window, or the newest token alone when
        # there is none (keep_plan)
        self.max_tail = max(self.cfg.local_window, 1)
        self.max_keep = k_cap + self.cfg.sink_size + self.max_tail
        self.key_mode = N.KEY_BF16 if self.cfg.score_dtype == torch.bfloat16 else N.KEY_F16
        if self.cfg.select == "head":  # the scorer emits one key row per query head
            self.key_mode |= N.SELECT_PER_HEAD
        # one workspace for every step: zero-filled once (the one-launch
        # step's barrier words start at zero and every call leaves them so)
        ws = N.size_query("lap_decode_step_workspace_size", batch, num_q_heads, num_kv_heads,
                          max(max_tokens, 1), head_dim, self.max_keep, self.key_mode)
        self.ws = torch.zeros(max(ws, 1), dtype=torch.uint8, device=self.dev)
        self._ops = ops()
        self.last_k = 0
        self._plans = None
        self._plan_key = None

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
        k = k if t_codes > 0 else 0
        sink, tail_start, tail_count = keep_plan(k, t_total, c.sink_size, c.local_window)
        return dict(cand_start=cs, cand_end=ce, k=k, sink=sink, tail_start=tail_start,
                    tail_count=tail_count)

    def row_plans(self, t_codes: list[int], t_total: list[int]) -> list[dict]:
        """One plan per sequence (the uniform plan of each sequence's lengths)."""
        out = []
        for tc, tt in zip(t_codes, t_total):
            out.append(dict(t_codes=tc, t_total=tt, **self.plan(tc, tt)))
        return out

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
        tc_rows = _per_row(t_codes, B, "t_codes")
        tt_rows = _per_row(t_total, B, "t_total")
        if (tc_rows is not None and len(set(tc_rows)) > 1) or \
                (tt_rows is not None and len(set(tt_rows)) > 1):
            if tc_rows is None or tt_rows is None:
                raise RuntimeError("ragged steps need both t_codes and t_total per sequence")
            return self._step_ragged(q, codes, keys, vals, tc_rows, tt_rows)
        t_codes = codes.shape[2] if tc_rows is None else tc_rows[0]
        t_total = keys.shape[2] if tt_rows is None else tt_rows[0]
        if t_total > self.T_max or t_codes > t_total:
            raise RuntimeError("cache length exceeds the decoder's max_tokens")
        if t_total > keys.shape[2] or t_total > vals.shape[2] or t_codes > codes.shape[2]:
            raise RuntimeError("a sequence length exceeds the cache views")
        p = self.plan(t_codes, t_total)
        qf = q.reshape(B * Hq, D) if q.is_contiguous() else q.contiguous().reshape(B * Hq, D)
        self._ops.lut_build(qf, self.cb, self.G, self.lut_layout, self.lut)
        self.last_k = p["k"]
        self._decode_step(q, codes, keys, vals, max(t_codes, 1), t_total, p, None, 0, 0, 0)
        return self.out.unsqueeze(2)

    def _decode_step(self, q, codes, keys, vals, T, T_kv, p, plans, k_cols, max_sink,
                     max_tail) -> None:
        """lap_decode_step (through the compiled torch op): scoring, top-k
        and sparse attention after the LUT (one launch for group and
        per-head selection at D = 128, the kernel chain otherwise)."""
        if p is None:
            p = dict(cand_start=0, cand_end=0, k=0, sink=0, tail_start=0, tail_count=0)
        keys, vals = keys[:, :, :T_kv], vals[:, :, :T_kv]
        self._ops.decode_step(self.lut, codes, T, p["cand_start"], p["cand_end"], p["k"],
                              p["sink"], p["tail_start"], p["tail_count"], plans, k_cols,
                              max_sink, max_tail, self.key_mode, q, keys, vals,
                              1.0 / math.sqrt(self.D), self.idx, self.out, self.ws)

    def fused_status(self) -> tuple[int, int]:
        """(rows whose workgroups spread over XCDs, barrier time-outs) of
        the one-launch steps run on this decoder's workspace so far
        (synchronises); both stay zero on a healthy device."""
        torch.cuda.synchronize(self.dev)
        a, b = N.u32(), N.u32()
        N.call("lap_decode_step_status", N.ptr(self.ws), self.ws.numel(), N.byref(a),
               N.byref(b))
        return int(a.value), int(b.value)

    def status_words(self) -> torch.Tensor:
        """The two health counters as a device int32 view [2] of the
        workspace (no copy, no synchronisation): callers that watch many
        decoders gather these and copy them to the host once."""
        return self.ws[:8].view(torch.int32)

    def check_health(self) -> None:
        """Raise :class:`StepHealthError` if any one-launch step on this
        decoder's workspace split a row over XCDs or timed out a barrier
        (synchronises)."""
        check_step_health(*self.fused_status(), who="SparseDecoder")

    def reset_health(self) -> None:
        """Zero the workspace (counters, barrier words and histograms) after
        an unhealthy step, so that later steps start from a clean state."""
        self.ws.zero_()

    def _step_ragged(self, q, codes, keys, vals, t_codes: list[int],
                     t_total: list[int]) -> torch.Tensor:
        B, Hq, Hkv, D = self.B, self.Hq, self.Hkv, self.D
        if max(t_total) > self.T_max or any(c > t for c, t in zip(t_codes, t_total)):
            raise RuntimeError("cache length exceeds the decoder's max_tokens")
        if max(t_total) > keys.shape[2] or max(t_codes) > codes.shape[2]:
            raise RuntimeError("a sequence length exceeds the cache views")
        plans = self.row_plans(t_codes, t_total)
        if self._plans is None:
            self._plans = PlanBuffer(B, self.dev)
        key = (tuple(t_codes), tuple(t_total))
        if key != self._plan_key:
            # the device plans change only here; a step with the same lengths
            # (a graph replay) reuses them
            self._plans.upload([tuple(p[f] for f in PLAN_FIELDS) for p in plans])
            self._plan_key = key
        pdev = self._plans.dev
        qf = q.reshape(B * Hq, D) if q.is_contiguous() else q.contiguous().reshape(B * Hq, D)
        self._ops.lut_build(qf, self.cb, self.G, self.lut_layout, self.lut)
        k_cols = max(p["k"] for p in plans)
        T = max(max(t_codes), 1)
        self.last_k = k_cols
        max_sink = max(p["sink"] for p in plans)
        max_tail = max(p["tail_count"] for p in plans)
        self._decode_step(q, codes, keys, vals, T, keys.shape[2], None, pdev, k_cols, max_sink,
                          max_tail)
        return self.out.unsqueeze(2)

    @property
    def k_cols(self) -> int:
        """Index-row width of device-plan steps: the largest budget any step
        within max_tokens can have."""
        return max(self._k_cap(self.T_max), 1)

    @torch.no_grad()
    def step_dev(self, q: torch.Tensor, codes: torch.Tensor, keys: torch.Tensor,
                 vals: torch.Tensor, plans: torch.Tensor) -> torch.Tensor:
        """One decode step driven by device plans (lap_row_plan [B] int32).

        Every launch argument is fixed (columns = the code buffer's
        capacity, index rows k_cols wide, sink/local bounds from the config),
        so the same launches serve every step: capture them once in a graph
        and rewrite ``plans`` before each replay.  Work past a sequence's
        lengths exits early in each kernel."""
        if q.dim() == 4:
            q = q[:, :, 0, :]
        B, Hq, Hkv, D = self.B, self.Hq, self.Hkv, self.D
        T = min(codes.shape[2], self.T_max)
        qf = q.reshape(B * Hq, D) if q.is_contiguous() else q.contiguous().reshape(B * Hq, D)
        self._ops.lut_build(qf, self.cb, self.G, self.lut_layout, self.lut)
        k_cols = self.k_cols
        self.last_k = k_cols
        self._decode_step(q, codes, keys, vals, T, keys.shape[2], None, plans, k_cols,
                          self.cfg.sink_size, self.max_tail)
        return self.out.unsqueeze(2)

    @torch.no_grad()
    def step_cached(self, q: torch.Tensor, cache) -> torch.Tensor:
        """One decode step over a ``DecodeKVCache``: candidates are the encoded
        tokens of each sequence, attention covers all of its cached tokens."""
        return self.step(q, cache.codes, cache.k, cache.v, t_codes=cache.encoded_lens,
                         t_total=cache.lengths)

    def selected(self) -> torch.Tensor:
        """Indices chosen by the last step: [B, rows, k] int32 (ascending; in a
        ragged step, rows past their sequence's k hold -1)."""
        rows = self.idx.shape[1]
        n = self.B * rows * self.last_k
        return self.idx.view(-1)[:n].view(self.B, rows, self.last_k)


class DenseDecoder:
    """Preallocated dense single-query decode (the comparator)."""

    def __init__(self, batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                 max_tokens: int, device: torch.device, dtype: torch.dtype = torch.bfloat16):
        N.lib()
        self.B, self.Hq, self.Hkv, self.D = batch, num_q_heads, num_kv_heads, head_dim
        self.out = torch.empty((batch, num_q_heads, head_dim), dtype=dtype, device=device)
        ws = N.size_query("lap_attn_decode_workspace_size", batch, num_q_heads, head_dim,
                          max(max_tokens, 1))
        self.ws = torch.empty(max(ws, 1), dtype=torch.uint8, device=device)
        self._ops = ops()
        self._plans = None
        self._plan_key = None

    @torch.no_grad()
    def step(self, q: torch.Tensor, keys: torch.Tensor, vals: torch.Tensor,
             lengths=None) -> torch.Tensor:
        """Attention over all cached tokens: keys.shape[2] of them, or
        ``lengths[b]`` for sequence b (ragged batches)."""
        if q.dim() == 4:
            q = q[:, :, 0, :]
        B, Hq, Hkv, D = self.B, self.Hq, self.Hkv, self.D
        T = keys.shape[2]
        rows = _per_row(lengths, B, "lengths")
        if rows is not None and (len(set(rows)) > 1 or rows[0] != T):
            if max(rows) > T or min(rows) < 1:
                raise RuntimeError("lengths must lie in [1, keys.shape[2]]")
            if self._plans is None:
                self._plans = PlanBuffer(B, q.device)
            if tuple(rows) != self._plan_key:
                self._plans.upload([(t, t, 0, 0, 0, 0, 0, t) for t in rows])
                self._plan_key = tuple(rows)
            pdev = self._plans.dev
            self._ops.attn_decode_ragged(q, keys, vals, None, Hkv, 0, pdev, 0, max(rows),
                                         1.0 / math.sqrt(D), self.out, self.ws)
            return self.out.unsqueeze(2)
        return self._dense_uniform(q, keys, vals)

    @torch.no_grad()
    def step_dev(self, q: torch.Tensor, keys: torch.Tensor, vals: torch.Tensor,
                 plans: torch.Tensor) -> torch.Tensor:
        """Dense decode with each sequence's length read from device plans
        (t_total, tail [0, t_total)); fixed launch arguments, as
        SparseDecoder.step_dev."""
        if q.dim() == 4:
            q = q[:, :, 0, :]
        B, Hq, Hkv, D = self.B, self.Hq, self.Hkv, self.D
        T = keys.shape[2]
        self._ops.attn_decode_ragged(q, keys, vals, None, Hkv, 0, plans, 0, T,
                                     1.0 / math.sqrt(D), self.out, self.ws)
        return self.out.unsqueeze(2)

    def _dense_uniform(self, q, keys, vals):
        self._ops.dense_decode(q, keys, vals, 1.0 / math.sqrt(self.D), self.out, self.ws)
        return self.out.unsqueeze(2)
