"""Decode-side caches of one attention layer: the growable K/V buffer and the
AQ code cache with its encode buffer.

Mirrors two pieces of laprune/llm/modifiers/aq_evaluation.py:

* ``_kv_cache_append`` (:65-112): a [B, Hkv, capacity, D] K/V buffer that new
  tokens are appended to, growing to max(needed, 2 x capacity);
* the decode branch of ``_prepare_aq_cache`` (:359-422): a u8
  [B, Hkv, capacity, M] code cache and ``encoded_len``.  In decode, the keys
  appended since the last encode are encoded only once there are at least
  ``group_size`` of them (:369-374, ``decode_group_size``); until then they are
  not scoring candidates and are covered by the local window, which must
  therefore span at least ``group_size - 1`` tokens.  Prefill encodes
  everything (:430-447).

The encode goes straight from the strided K buffer into the strided code
buffer with one ``lap_encode_keys`` launch (MFMA search, exact codes).  Growth
allocates (torch); size ``capacity`` up front for HIP-graph capture.

Sequences may have different lengths (ragged batches, which the reference
does not have): each keeps its own ``lengths[b]`` and ``encoded_lens[b]``,
new tokens land at each sequence's own end, and each flushes its encode
buffer by the rule above on its own.
"""
from __future__ import annotations

import torch

from . import _native as N
from ._ops import ops
from .aq_kernels import aq_encode_prepare


def flush_range(length: int, encoded_len: int, group_size: int,
                prefill: bool) -> tuple[int, int] | None:
    """Token range [t0, t1) to encode now, or None (aq_evaluation.py:369-382)."""
    tail = length - encoded_len
    if tail <= 0:
        return None
    if not prefill and group_size > 1 and tail < group_size:
        return None
    return encoded_len, length


def grown_capacity(capacity: int, needed: int) -> int:
    """New capacity when ``needed`` tokens do not fit (aq_evaluation.py:94-95)."""
    return max(needed, capacity * 2)


class DecodeKVCache:
    """K/V buffer + AQ code cache of one layer.

    Args:
      codebooks: [M, K, D] fp32 codebooks of the layer (on the GPU), or None
        for a layer that keeps K/V only (a dense layer: nothing is encoded).
      batch, num_kv_heads, head_dim: cache geometry.
      capacity: initial token capacity (grows by doubling when exceeded).
      dtype: K/V dtype (bf16 or fp16).
      group_size: decode encode buffer (64 in the reference configs).
    """

    def __init__(self, codebooks: torch.Tensor | None, batch: int, num_kv_heads: int,
                 head_dim: int, capacity: int, dtype: torch.dtype = torch.bfloat16,
                 group_size: int = 64, device=None):
        if dtype not in (torch.bfloat16, torch.float16):
            raise RuntimeError("K/V dtype must be bf16 or fp16")
        self.B, self.Hkv, self.D = batch, num_kv_heads, head_dim
        self.dtype = dtype
        self.group_size = int(group_size)
        cap = max(int(capacity), 16)
        if codebooks is None:
            self.dev = torch.device(device if device is not None else "cuda")
            self.cb = self.prep = None
            self.M = self.K = 0
        else:
            N.require_cuda(codebooks)
            if codebooks.dim() != 3 or codebooks.shape[2] != head_dim:
                raise RuntimeError(f"codebooks must be [M, K, {head_dim}]")
            self.dev = codebooks.device
            self.cb = codebooks.to(torch.float32).contiguous()
            self.M, self.K = int(self.cb.shape[0]), int(self.cb.shape[1])
            if self.K > 256:
                raise RuntimeError("K must be <= 256 for uint8 codes")
            self.prep = aq_encode_prepare(self.cb)
        self.k = torch.empty((batch, num_kv_heads, cap, head_dim), dtype=dtype, device=self.dev)
        self.v = torch.empty_like(self.k)
        self.codes = torch.zeros((batch, num_kv_heads, cap, self.M), dtype=torch.uint8,
                                 device=self.dev)
        self.lengths = [0] * batch
        self.encoded_lens = [0] * batch

    @property
    def capacity(self) -> int:
        return int(self.k.shape[2])

    @property
    def ragged(self) -> bool:
        return len(set(self.lengths)) > 1 or len(set(self.encoded_lens)) > 1

    @property
    def length(self) -> int:
        """The common length of all sequences (RuntimeError when they differ)."""
        if len(set(self.lengths)) > 1:
            raise RuntimeError("sequences have different lengths: use .lengths")
        return self.lengths[0]

    @property
    def encoded_len(self) -> int:
        """The common encoded length (RuntimeError when sequences differ)."""
        if len(set(self.encoded_lens)) > 1:
            raise RuntimeError("sequences have different encoded lengths: use .encoded_lens")
        return self.encoded_lens[0]

    def _grow(self, needed: int) -> None:
        cap = grown_capacity(self.capacity, needed)
        k = self.k.new_empty((self.B, self.Hkv, cap, self.D))
        v = self.v.new_empty((self.B, self.Hkv, cap, self.D))
        codes = self.codes.new_zeros((self.B, self.Hkv, cap, self.M))
        n = max(self.lengths)
        if n:
            k[:, :, :n] = self.k[:, :, :n]
            v[:, :, :n] = self.v[:, :, :n]
        e = max(self.encoded_lens)
        if e:
            codes[:, :, :e] = self.codes[:, :, :e]
        self.k, self.v, self.codes = k, v, codes

    def _check_new(self, k_new: torch.Tensor, v_new: torch.Tensor, batch: int) -> int:
        if k_new.shape != v_new.shape or k_new.dim() != 4:
            raise RuntimeError("k_new and v_new must both be [B, Hkv, Tn, D]")
        B, H, Tn, D = k_new.shape
        if (B, H, D) != (batch, self.Hkv, self.D):
            raise RuntimeError(f"expected [{batch}, {self.Hkv}, Tn, {self.D}], got "
                               f"{list(k_new.shape)}")
        return Tn

    def append(self, k_new: torch.Tensor, v_new: torch.Tensor, prefill: bool = False) -> None:
        """Append [B, Hkv, Tn, D] keys/values, Tn to every sequence at its own
        end; encode the tails the policy says to."""
        Tn = self._check_new(k_new, v_new, self.B)
        ends = [n + Tn for n in self.lengths]
        if max(ends) > self.capacity:
            self._grow(max(ends))
        if len(set(self.lengths)) == 1:
            n = self.lengths[0]
            self.k[:, :, n:n + Tn] = k_new.to(self.dtype)
            self.v[:, :, n:n + Tn] = v_new.to(self.dtype)
        else:
            # one scatter per buffer: row b's tokens go to [lengths[b], +Tn)
            pos = torch.tensor([[n + i for i in range(Tn)] for n in self.lengths],
                               device=self.dev)
            bidx = torch.arange(self.B, device=self.dev)[:, None]
            self.k[bidx, :, pos] = k_new.to(self.dtype).permute(0, 2, 1, 3)
            self.v[bidx, :, pos] = v_new.to(self.dtype).permute(0, 2, 1, 3)
        self.lengths = ends
        self.encode(prefill=prefill)

    def append_row(self, b: int, k_new: torch.Tensor, v_new: torch.Tensor,
                   prefill: bool = True) -> None:
        """Append [1, Hkv, Tn, D] keys/values to sequence b alone (a ragged
        prefill fills each sequence this way); encode its tail by the policy."""
        Tn = self._check_new(k_new, v_new, 1)
        n = self.lengths[b]
        if n + Tn > self.capacity:
            self._grow(n + Tn)
        self.k[b:b + 1, :, n:n + Tn] = k_new.to(self.dtype)
        self.v[b:b + 1, :, n:n + Tn] = v_new.to(self.dtype)
        self.lengths[b] = n + Tn
        self._encode_rows([b], prefill, None)

    @torch.no_grad()
    def encode(self, prefill: bool = False, resid_norm: torch.Tensor | None = None) -> int:
        """Encode each sequence's [encoded_len, length) if the policy allows;
        returns rows encoded.  ``resid_norm`` ([B, Hkv, t1 - t0] fp32) needs
        every sequence to flush the same range."""
        return self._encode_rows(list(range(self.B)), prefill, resid_norm)

    def _encode_rows(self, rows: list[int], prefill: bool, resid_norm) -> int:
        if self.cb is None:  # K/V-only layer: the whole cache counts as encoded
            for b in rows:
                self.encoded_lens[b] = self.lengths[b]
            return 0
        todo = {}
        for b in rows:
            rng = flush_range(self.lengths[b], self.encoded_lens[b], self.group_size, prefill)
            if rng is not None:
                todo.setdefault(rng, []).append(b)
        if not todo:
            return 0
        if resid_norm is not None and (len(todo) != 1 or len(rows) != self.B
                                       or len(next(iter(todo.values()))) != self.B):
            raise RuntimeError("resid_norm needs every sequence to flush the same range")
        done = 0
        for (t0, t1), bs in todo.items():
            if len(bs) == self.B:
                self._launch(0, self.B, t0, t1, resid_norm)
            else:
                for b in bs:
                    self._launch(b, 1, t0, t1, None)
            for b in bs:
                self.encoded_lens[b] = t1
            done += len(bs) * self.Hkv * (t1 - t0)
        return done

    def _launch(self, b0: int, nb: int, t0: int, t1: int, resid_norm) -> None:
        k, c = self.k[b0:b0 + nb], self.codes[b0:b0 + nb]
        N.call("lap_encode_keys", N.ptr(k), N.dtype_code(k.dtype), k.stride(0), k.stride(1),
               k.stride(2), nb, self.Hkv, t0, t1, self.D, N.ptr(self.cb), self.M, self.K,
               N.ptr(self.prep), self.prep.numel(), N.ptr(c), c.stride(0), c.stride(1),
               c.stride(2), N.ptr(resid_norm), N.stream_of(k))

    # ---- device-resident decode steps (one captured graph per step) ------
    # The positions and flush ranges of a step live in device tensors, so the
    # same launches serve every step; the host only advances its bookkeeping
    # (advance_decode) and uploads the step's values.  Capacity cannot grow
    # here: size it for the whole generation.

    def advance_decode(self) -> list[tuple[int, int]]:
        """Host bookkeeping of one decode token per sequence: lengths grow by
        one and each sequence whose encode buffer is full flushes it.  Returns
        the per-sequence flush ranges ((0, 0) for none)."""
        if max(self.lengths) + 1 > self.capacity:
            raise RuntimeError("decode step past the cache capacity")
        ranges = []
        for b in range(self.B):
            self.lengths[b] += 1
            if self.cb is None:
                self.encoded_lens[b] = self.lengths[b]
                ranges.append((0, 0))
                continue
            rng = flush_range(self.lengths[b], self.encoded_lens[b], self.group_size, False)
            if rng is None:
                ranges.append((0, 0))
            else:
                ranges.append(rng)
                self.encoded_lens[b] = rng[1]
        return ranges

    def append_at(self, k_new: torch.Tensor, v_new: torch.Tensor, pos: torch.Tensor,
                  bidx: torch.Tensor) -> None:
        """Write one token per sequence ([B, Hkv, 1, D]) at device positions
        pos [B, 1] (int64); bidx is arange(B)[:, None] on the device."""
        self.k[bidx, :, pos] = k_new.to(self.dtype).permute(0, 2, 1, 3)
        self.v[bidx, :, pos] = v_new.to(self.dtype).permute(0, 2, 1, 3)

    def rope_append(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
                    sin: torch.Tensor, pos: torch.Tensor, q_out: torch.Tensor) -> torch.Tensor:
        """Rotate one decode token per sequence and append it, in one launch.

        q [B, 1, Hq*D], k and v [B, 1, Hkv*D] (projection outputs, heads
        contiguous), cos/sin [B, 1, D] (the model's rotary tables in its
        dtype), pos [B, 1] int64 device positions.  rope(k) and v go to the
        capacity buffers at pos; rope(q) to q_out [B, Hq, D], returned as
        [B, Hq, 1, D].  Bit-identical to apply_rotary_pos_emb + append_at."""
        D, B = self.D, self.B
        Hq = q.shape[-1] // D
        if any(t.stride(-1) != 1 for t in (q, k, v, cos, sin)):
            raise RuntimeError("rope_append: rows must be contiguous")
        if any(t.dtype != self.dtype for t in (q, k, v, cos, sin)):
            raise RuntimeError("rope_append: q, k, v, cos and sin must be in the cache dtype")
        if sin.stride(0) != cos.stride(0) or cos.shape[-1] != D or sin.shape[-1] != D:
            raise RuntimeError("rope_append: cos and sin must be [B, 1, D] with equal strides")
        if (q.shape[0] != B or k.shape[0] != B or v.shape[0] != B or cos.shape[0] != B
                or k.shape[-1] != self.Hkv * D or v.shape[-1] != self.Hkv * D
                or q.shape[-1] % D != 0):
            raise RuntimeError("rope_append: q [B,1,Hq*D], k/v [B,1,Hkv*D] expected")
        if pos.dtype != torch.int64 or pos.numel() != B:
            raise RuntimeError("rope_append: pos must be int64 with one position per sequence")
        if q_out.shape != (B, Hq, D) or not q_out.is_contiguous() or q_out.dtype != self.dtype:
            raise RuntimeError("rope_append: q_out must be a contiguous [B, Hq, D] tensor")
        ops().rope_append(q, k, v, cos, sin, pos, self.k, self.v, self.capacity, q_out)
        return q_out.unsqueeze(2)

    def encode_ranges(self, ranges: torch.Tensor) -> None:
        """Encode each sequence's device range ([B, 2] int32, at most
        group_size tokens; empty ranges cost a workgroup exit)."""
        if self.cb is None:
            return
        if self.k.shape[:2] != (self.B, self.Hkv) or self.k.shape[3] != self.D:
            raise RuntimeError("encode_ranges: key cache shape changed")
        ops().encode_keys_ranges(self.k, ranges, self.group_size, self.capacity, self.cb,
                                 self.prep, self.codes)

    def keys(self) -> torch.Tensor:
        return self.k[:, :, :self.length]

    def values(self) -> torch.Tensor:
        return self.v[:, :, :self.length]

    def encoded_codes(self) -> torch.Tensor:
        """[B, Hkv, encoded_len, M] view (strided in the capacity buffer)."""
        return self.codes[:, :, :self.encoded_len]
