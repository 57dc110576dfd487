"""LAPrune decode attention inside a transformers Llama model.

Mirrors the reference's model plumbing for the decode path:
  * ``Decoder`` (laprune/llm/modifiers/aq_evaluation.py:496-540) patches
    every attention layer; layers in ``apply_layers`` are LAPrune layers, the
    rest stay dense;
  * ``self_attn_forward`` (:279-322): q/k/v projections, RoPE, append to the
    layer's K/V cache, encode new keys (prefill: all of them; decode: in
    64-token groups), causal SDPA at prefill, sparse retrieval at decode;
  * ``AQGeneration.generate`` (aq_generation.py:114-151): prefill all prompt
    tokens but the last, then greedy decode one token at a time.

Each layer owns a :class:`~laprune_amd.cache.DecodeKVCache`; LAPrune layers
decode through :class:`~laprune_amd.retrieval.SparseDecoder` (LUT -> fused
score -> top-k -> sparse attention, all HIP), dense layers through
:class:`~laprune_amd.retrieval.DenseDecoder`.  Sequences of one batch may have
different lengths (ragged): prefill them one row at a time with
:meth:`LAPruneLlama.prefill_row`, then decode the batch together.

The model is a plain ``transformers`` ``LlamaForCausalLM``; nothing here
downloads anything (build it from a local ``LlamaConfig``).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from .cache import DecodeKVCache
from .retrieval import DenseDecoder, RetrievalConfig, SparseDecoder, check_step_health


@dataclass
class LAPruneSettings:
    """Decode settings (the reference's ``draft_kwargs`` keys on this path)."""

    apply_layers: list[int] = field(default_factory=list)  # LAPrune layers
    retrieval: RetrievalConfig = field(default_factory=RetrievalConfig)
    group_size: int = 64                                   # decode encode buffer

    def __post_init__(self):
        if self.retrieval.local_window < self.group_size - 1:
            raise ValueError("local_window must cover the encode buffer "
                             "(local_window >= group_size - 1)")


class _LayerState:
    def __init__(self, cache: DecodeKVCache, sparse: SparseDecoder | None, dense: DenseDecoder):
        self.cache = cache
        self.sparse = sparse
        self.dense = dense


class LAPruneLlama:
    """A Llama model whose attention layers run the LAPrune decode path.

    Args:
      model: ``transformers`` ``LlamaForCausalLM`` on the GPU (bf16 or fp16).
      codebooks: {layer index: [M=32, K=256, head_dim] fp32 codebooks} for the
        layers in ``settings.apply_layers``.
      settings: which layers are LAPrune layers and the selection settings.
      batch: sequences decoded together.
      capacity: token capacity of every layer's cache (prompt + new tokens).
      health_every: decode steps between reads of the one-launch steps'
        health counters (one synchronisation each; 0 reads only at the end
        of ``generate``).  A non-zero counter raises
        :class:`~laprune_amd.retrieval.StepHealthError`.
    """

    def __init__(self, model, codebooks: dict[int, torch.Tensor], settings: LAPruneSettings,
                 batch: int, capacity: int, health_every: int = 64):
        from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
        self._rope = apply_rotary_pos_emb
        self.model = model
        self.settings = settings
        cfg = model.config
        self.B = batch
        self.Hq = cfg.num_attention_heads
        self.Hkv = cfg.num_key_value_heads
        self.D = getattr(cfg, "head_dim", None) or cfg.hidden_size // self.Hq
        self.capacity = capacity
        p = next(model.parameters())
        self.dev, self.dtype = p.device, p.dtype
        missing = [i for i in settings.apply_layers if i not in codebooks]
        if missing:
            raise RuntimeError(f"no codebooks for LAPrune layers {missing}")
        self.layers = model.model.layers
        self.states: list[_LayerState] = []
        for i, layer in enumerate(self.layers):
            cb = codebooks[i].to(self.dev, torch.float32) if i in settings.apply_layers else None
            cache = DecodeKVCache(cb, batch, self.Hkv, self.D, capacity, dtype=self.dtype,
                                  group_size=settings.group_size, device=self.dev)
            sparse = None
            if cb is not None:
                sparse = SparseDecoder(cb, batch, self.Hq, self.Hkv, self.D, capacity,
                                       settings.retrieval, dtype=self.dtype)
            dense = DenseDecoder(batch, self.Hq, self.Hkv, self.D, capacity, self.dev, self.dtype)
            self.states.append(_LayerState(cache, sparse, dense))
            attn = layer.self_attn
            self._fuse_qkv(attn)
            attn.forward = self._make_forward(i, attn)
        self._row = None  # sequence being prefilled alone (ragged prefill)
        self.health_every = health_every
        self._since_check = 0
        self._dev_mode = False
        self._graph = None
        self._g = None

    # ------------------------------------------------------------ attention
    @staticmethod
    @torch.no_grad()
    def _fuse_qkv(attn) -> None:
        """One [q; k; v] weight per layer, so that a step projects with one
        GEMV instead of three; the modules' own weights become views of it
        (no second copy).  Layers whose biases are mixed keep three GEMVs."""
        mods = (attn.q_proj, attn.k_proj, attn.v_proj)
        has_b = [m.bias is not None for m in mods]
        if any(has_b) and not all(has_b):
            attn._lap_qkv = None
            return
        w = torch.cat([m.weight for m in mods], 0)
        b = torch.cat([m.bias for m in mods], 0) if all(has_b) else None
        sizes = [m.weight.shape[0] for m in mods]
        o = 0
        for m, n in zip(mods, sizes):
            m.weight = torch.nn.Parameter(w[o:o + n], requires_grad=False)
            if b is not None:
                m.bias = torch.nn.Parameter(b[o:o + n], requires_grad=False)
            o += n
        attn._lap_qkv = (w, b, sizes)

    @staticmethod
    def _fused_current(attn) -> bool:
        """Whether the modules' weights (and biases) are still the views of
        the fused tensors.  ``model.to(...)`` or ``load_state_dict(assign=True)``
        replace the parameters; the fused copy is then stale."""
        w, b, sizes = attn._lap_qkv
        mods = (attn.q_proj, attn.k_proj, attn.v_proj)
        off = 0
        for m, n in zip(mods, sizes):
            mw = m.weight
            if (mw.dtype != w.dtype or mw.device != w.device or
                    mw.data_ptr() != w.data_ptr() + off * w.stride(0) * w.element_size()):
                return False
            if b is not None and (m.bias is None or m.bias.dtype != b.dtype or
                                  m.bias.data_ptr() != b.data_ptr() + off * b.element_size()):
                return False
            off += n
        return True

    @classmethod
    def _project(cls, attn, h):
        """q, k, v projections of h [B, T, hidden] as [B, T, n] (views of one
        fused GEMV output when the layer's weights are fused).  A layer whose
        parameters were replaced after wrapping is fused again first."""
        f = getattr(attn, "_lap_qkv", None)
        if f is not None and not cls._fused_current(attn):
            cls._fuse_qkv(attn)
            f = attn._lap_qkv
        if f is None:
            return attn.q_proj(h), attn.k_proj(h), attn.v_proj(h)
        w, b, sizes = f
        return F.linear(h, w, b).split(sizes, dim=-1)

    def _make_forward(self, idx: int, attn):
        def forward(hidden_states, position_embeddings=None, attention_mask=None,
                    past_key_values=None, **kwargs):
            return self._attention(idx, attn, hidden_states, position_embeddings)
        return forward

    def _attention(self, idx, attn, h, position_embeddings):
        B, T, _ = h.shape
        Hq, Hkv, D = self.Hq, self.Hkv, self.D
        cos, sin = position_embeddings
        st = self.states[idx]
        if T == 1 and self._dev_mode:
            # fixed launches, every per-step value in device memory; RoPE and
            # the cache write are one kernel
            qp, kp, vp = self._project(attn, h)
            q = st.cache.rope_append(qp, kp, vp, cos, sin, self._g_pos, self._q_rope)
            if st.sparse is not None:
                if self._g_flush:
                    st.cache.encode_ranges(self._g_ranges)
                o = st.sparse.step_dev(q, st.cache.codes, st.cache.k, st.cache.v,
                                       self._g_plan_sparse)
            else:
                o = st.dense.step_dev(q, st.cache.k, st.cache.v, self._g_plan_dense)
            o = o.transpose(1, 2).reshape(B, T, Hq * D)
            return attn.o_proj(o), None
        qp, kp, vp = self._project(attn, h)
        q = qp.reshape(B, T, Hq, D).transpose(1, 2)
        k = kp.reshape(B, T, Hkv, D).transpose(1, 2)
        v = vp.reshape(B, T, Hkv, D).transpose(1, 2)
        q, k = self._rope(q, k, cos, sin)
        if T > 1:  # prefill: causal attention over the prompt, encode all its keys
            if self._row is None:
                if any(n != 0 for n in st.cache.lengths):
                    raise RuntimeError("batched prefill needs empty caches (use reset())")
                st.cache.append(k, v, prefill=True)
            else:
                st.cache.append_row(self._row, k, v, prefill=True)
            G = Hq // Hkv
            kk = k.repeat_interleave(G, dim=1)
            vv = v.repeat_interleave(G, dim=1)
            # fused kernels only: the math fallback would materialise T x T scores
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                o = F.scaled_dot_product_attention(q, kk, vv, is_causal=True,
                                                   scale=1.0 / math.sqrt(D))
        else:
            if self._row is not None:
                raise RuntimeError("single-token steps decode the whole batch")
            st.cache.append(k, v)  # encodes each sequence's 64-token groups
            if st.sparse is not None:
                o = st.sparse.step_cached(q, st.cache)
            else:
                o = st.dense.step(q, st.cache.k, st.cache.v, lengths=st.cache.lengths)
        o = o.transpose(1, 2).reshape(B, T, Hq * D)
        return attn.o_proj(o), None

    # ------------------------------------------------------------ model calls
    def reset(self) -> None:
        """Forget every sequence (the reference's Decoder.reset)."""
        for st in self.states:
            st.cache.lengths = [0] * self.B
            st.cache.encoded_lens = [0] * self.B

    @property
    def lengths(self) -> list[int]:
        return list(self.states[0].cache.lengths)

    def _check_room(self, new: int, rows=None) -> None:
        """Raise before any layer runs when ``new`` more tokens for the given
        sequences (all by default) would exceed ``capacity``, which sized
        every layer's decoder and workspaces; nothing is appended then, so
        the layers' caches stay consistent."""
        lens = self.lengths
        rows = range(self.B) if rows is None else rows
        need = max(lens[b] for b in rows) + new
        if need > self.capacity:
            raise RuntimeError(f"{need} tokens exceed the capacity of {self.capacity} the "
                               "model was wrapped with (wrap it with a larger capacity)")

    def _forward(self, ids: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        out = self.model(input_ids=ids, position_ids=pos, use_cache=False, logits_to_keep=1)
        return out.logits[:, -1]

    @torch.no_grad()
    def prefill(self, input_ids: torch.Tensor) -> torch.Tensor:
        """Prefill [B, T] prompts of one length; returns last-position logits [B, V]."""
        if input_ids.shape[0] != self.B:
            raise RuntimeError(f"expected {self.B} sequences, got {input_ids.shape[0]}")
        T = input_ids.shape[1]
        if any(n != 0 for n in self.lengths):
            raise RuntimeError("batched prefill needs empty caches (use reset())")
        self._check_room(T)
        pos = torch.arange(T, device=self.dev)[None].expand(self.B, T)
        return self._forward(input_ids.to(self.dev), pos)

    @torch.no_grad()
    def prefill_row(self, b: int, input_ids: torch.Tensor) -> torch.Tensor:
        """Prefill sequence b alone ([1, T_b] prompt); returns its logits [1, V]."""
        T = input_ids.shape[-1]
        if not 0 <= b < self.B:
            raise RuntimeError(f"sequence {b} out of range for batch {self.B}")
        self._check_room(T, rows=[b])
        self._row = b
        try:
            pos = torch.arange(T, device=self.dev)[None]
            return self._forward(input_ids.reshape(1, T).to(self.dev), pos)
        finally:
            self._row = None

    @torch.no_grad()
    def decode(self, tokens: torch.Tensor) -> torch.Tensor:
        """One decode step for all sequences: tokens [B, 1]; returns logits [B, V]."""
        self._check_room(1)
        pos = torch.tensor(self.lengths, device=self.dev)[:, None]
        logits = self._forward(tokens.reshape(self.B, 1).to(self.dev), pos)
        self._count_step()
        return logits

    # ------------------------------------------------------------ health
    def check_health(self) -> None:
        """Read every LAPrune layer's health counters (one gather, one
        synchronising copy) and raise StepHealthError naming the layers
        whose one-launch steps split a row over XCDs or timed out a barrier."""
        self._since_check = 0
        decs = [(i, st.sparse) for i, st in enumerate(self.states) if st.sparse is not None]
        if not decs:
            return
        words = torch.stack([d.status_words() for _, d in decs]).cpu()
        bad = [(i, int(w[0]), int(w[1])) for (i, _), w in zip(decs, words.tolist())
               if w[0] or w[1]]
        if bad:
            check_step_health(sum(b[1] for b in bad), sum(b[2] for b in bad),
                              who=f"LAPruneLlama (layers {[b[0] for b in bad]})")

    def reset_health(self) -> None:
        """Zero every LAPrune layer's step workspace after an unhealthy step."""
        for st in self.states:
            if st.sparse is not None:
                st.sparse.reset_health()

    def _count_step(self) -> None:
        self._since_check += 1
        if self.health_every and self._since_check >= self.health_every:
            self.check_health()

    # ------------------------------------------------------------ captured decode
    # One decode step of the whole model as one HIP graph.  Per-step values
    # (positions, the sequences' plans, encode-flush ranges) live in one
    # device int32 buffer that the host rewrites before each replay; every
    # kernel of the step reads them there, so the captured launches stay
    # valid.  The host keeps the lengths and flush bookkeeping.

    def _graph_buffers(self):
        B, dev = self.B, self.dev
        flat = torch.zeros(19 * B, dtype=torch.int32, device=dev)
        self._g_flat = flat
        self._g_plan_sparse = flat[:8 * B].view(B, 8)
        self._g_plan_dense = flat[8 * B:16 * B].view(B, 8)
        self._g_ranges = flat[16 * B:18 * B].view(B, 2)
        self._g_pos32 = flat[18 * B:].view(B, 1)
        self._g_pos = torch.zeros((B, 1), dtype=torch.long, device=dev)
        self._q_rope = torch.empty((B, self.Hq, self.D), dtype=self.dtype, device=dev)
        self._g_flush = False
        self._g_tok = torch.zeros((B, 1), dtype=torch.long, device=dev)
        self._g_next = torch.zeros((B, 1), dtype=torch.long, device=dev)
        self._g_logits = None
        self._g_host = [torch.zeros(19 * B, dtype=torch.int32).pin_memory() for _ in range(4)]
        self._g_done = [None] * 4
        self._g_slot = 0
        self._g = True

    def _graph_body(self):
        self._g_pos.copy_(self._g_pos32)
        self._dev_mode = True
        try:
            logits = self._forward(self._g_tok, self._g_pos)
        finally:
            self._dev_mode = False
        if self._g_logits is None:
            self._g_logits = torch.empty_like(logits)
        self._g_logits.copy_(logits)
        self._g_next.copy_(logits.argmax(dim=-1, keepdim=True))

    def _upload_step(self) -> None:
        """Advance every layer's bookkeeping by one token and upload the
        step's positions, plans and flush ranges."""
        B = self.B
        pos = self.lengths
        ranges = None
        for st in self.states:
            r = st.cache.advance_decode()
            if st.sparse is not None:
                ranges = r
        # steps on which no sequence fills its encode buffer replay the graph
        # without the encode launches
        self._g_flush = ranges is not None and any(hi > lo for lo, hi in ranges)
        c0 = next((st for st in self.states if st.sparse is not None), self.states[0])
        t_total = c0.cache.lengths
        rows = [0] * (19 * B)
        if c0.sparse is not None:
            from .retrieval import PLAN_FIELDS
            for b, p in enumerate(c0.sparse.row_plans(c0.cache.encoded_lens, t_total)):
                rows[8 * b:8 * b + 8] = [p[f] for f in PLAN_FIELDS]
        for b in range(B):
            t = t_total[b]
            rows[8 * B + 8 * b:8 * B + 8 * b + 8] = [t, t, 0, 0, 0, 0, 0, t]
            if ranges is not None:
                rows[16 * B + 2 * b:16 * B + 2 * b + 2] = list(ranges[b])
            rows[18 * B + b] = pos[b]
        i = self._g_slot
        self._g_slot = (i + 1) % len(self._g_host)
        if self._g_done[i] is not None:
            self._g_done[i].synchronize()
        h = self._g_host[i]
        h.copy_(torch.tensor(rows, dtype=torch.int32))
        self._g_flat.copy_(h, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.dev))
        self._g_done[i] = ev

    @torch.no_grad()
    def decode_graph(self, tokens: torch.Tensor | None = None) -> torch.Tensor:
        """One decode step for all sequences as one graph replay.  tokens
        [B, 1] (device or host); None feeds the previous step's greedy
        tokens.  Returns the logits [B, V] (a buffer the next step reuses)."""
        self._check_room(1)
        if self._g is None:
            self._graph_buffers()
        if tokens is not None:
            self._g_tok.copy_(tokens.reshape(self.B, 1), non_blocking=True)
        else:
            self._g_tok.copy_(self._g_next)
        self._upload_step()
        sig = tuple((st.cache.k.data_ptr(), st.cache.v.data_ptr(), st.cache.codes.data_ptr())
                    for st in self.states)
        if self._graph is not None and sig != self._graph_sig:
            self._graph = None  # a cache was reallocated (grown): capture again
        if self._graph is None:
            self._graph = {}
            self._graph_sig = sig
        g = self._graph.get(self._g_flush)
        if g is None:
            # the first step of each variant (with or without encode flushes)
            # runs eagerly (it also warms up every kernel), then the same body
            # is captured for the following steps
            side = torch.cuda.Stream(self.dev)
            side.wait_stream(torch.cuda.current_stream(self.dev))
            with torch.cuda.stream(side):
                self._graph_body()
            torch.cuda.current_stream(self.dev).wait_stream(side)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._graph_body()
            self._graph[self._g_flush] = g
        else:
            g.replay()
        self._count_step()
        return self._g_logits

    def next_tokens(self) -> torch.Tensor:
        """Greedy tokens [B, 1] of the last captured step (device)."""
        return self._g_next

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int,
                 eos_token_id: int | None = None, graph: bool = False) -> torch.Tensor:
        """Greedy generation as AQGeneration.generate: prefill all prompt
        tokens but the last, then decode from it.  Returns [B, T + n] ids.
        graph=True decodes with captured steps (the cache capacity must hold
        the whole generation)."""
        self.reset()
        ids = input_ids.to(self.dev)
        if ids.shape[1] > 1:
            self.prefill(ids[:, :-1])
        tok = ids[:, -1:]
        new = []
        for i in range(max_new_tokens):
            if graph:
                self.decode_graph(tok if i == 0 else None)
                tok = self._g_next.clone()
            else:
                tok = self.decode(tok).argmax(dim=-1, keepdim=True)
            new.append(tok)
            if eos_token_id is not None and bool((tok == eos_token_id).all()):
                break
        self.check_health()
        return torch.cat([ids] + new, dim=1)


def llama31_8b_config(num_layers: int = 32, max_position_embeddings: int = 131072):
    """A local LlamaConfig with Llama-3.1-8B's public geometry (no download)."""
    from transformers import LlamaConfig
    return LlamaConfig(
        vocab_size=128256, hidden_size=4096, intermediate_size=14336,
        num_hidden_layers=num_layers, num_attention_heads=32, num_key_value_heads=8,
        head_dim=128, max_position_embeddings=max_position_embeddings, rms_norm_eps=1e-5,
        rope_theta=500000.0, tie_word_embeddings=False,
        rope_scaling={"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                      "high_freq_factor": 4.0, "original_max_position_embeddings": 8192},
        attn_implementation="sdpa")


def random_model(config, device, dtype=torch.bfloat16, seed: int = 0, std: float = 0.02):
    """Random-init LlamaForCausalLM: every weight N(0, std), norms at 1."""
    from transformers import LlamaForCausalLM
    torch.manual_seed(seed)
    with torch.device(device):
        model = LlamaForCausalLM(config).to(dtype)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if p.dim() >= 2:
                p.normal_(0.0, std)
            else:
                p.fill_(1.0)
    return model.eval()
