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
"""
from __future__ import annotations

import torch

from . import _native as N
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
      codebooks: [M, K, D] fp32 codebooks of the layer (on the GPU).
      batch, num_kv_heads, head_dim: cache geometry.
      capacity: initial token capacity (grows by doubling when exceeded).
      dtype: K/V dtype (bf16 or fp16).
      group_size: decode encode buffer (64 in the reference configs).
    """

    def __init__(self, codebooks: torch.Tensor, batch: int, num_kv_heads: int, head_dim: int,
                 capacity: int, dtype: torch.dtype = torch.bfloat16, group_size: int = 64):
        N.require_cuda(codebooks)
        if codebooks.dim() != 3 or codebooks.shape[2] != head_dim:
            raise RuntimeError(f"codebooks must be [M, K, {head_dim}]")
        if dtype not in (torch.bfloat16, torch.float16):
            raise RuntimeError("K/V dtype must be bf16 or fp16")
        self.dev = codebooks.device
        self.cb = codebooks.to(torch.float32).contiguous()
        self.M, self.K = int(self.cb.shape[0]), int(self.cb.shape[1])
        if self.K > 256:
            raise RuntimeError("K must be <= 256 for uint8 codes")
        self.B, self.Hkv, self.D = batch, num_kv_heads, head_dim
        self.dtype = dtype
        self.group_size = int(group_size)
        self.prep = aq_encode_prepare(self.cb)
        cap = max(int(capacity), 16)
        self.k = torch.empty((batch, num_kv_heads, cap, head_dim), dtype=dtype, device=self.dev)
        self.v = torch.empty_like(self.k)
        self.codes = torch.zeros((batch, num_kv_heads, cap, self.M), dtype=torch.uint8,
                                 device=self.dev)
        self.length = 0
        self.encoded_len = 0

    @property
    def capacity(self) -> int:
        return int(self.k.shape[2])

    def _grow(self, needed: int) -> None:
        cap = grown_capacity(self.capacity, needed)
        k = self.k.new_empty((self.B, self.Hkv, cap, self.D))
        v = self.v.new_empty((self.B, self.Hkv, cap, self.D))
        codes = self.codes.new_zeros((self.B, self.Hkv, cap, self.M))
        if self.length:
            k[:, :, :self.length] = self.k[:, :, :self.length]
            v[:, :, :self.length] = self.v[:, :, :self.length]
        if self.encoded_len:
            codes[:, :, :self.encoded_len] = self.codes[:, :, :self.encoded_len]
        self.k, self.v, self.codes = k, v, codes

    def append(self, k_new: torch.Tensor, v_new: torch.Tensor, prefill: bool = False) -> None:
        """Append [B, Hkv, Tn, D] keys/values; encode the tail when the policy says so."""
        if k_new.shape != v_new.shape or k_new.dim() != 4:
            raise RuntimeError("k_new and v_new must both be [B, Hkv, Tn, D]")
        B, H, Tn, D = k_new.shape
        if (B, H, D) != (self.B, self.Hkv, self.D):
            raise RuntimeError(f"expected [{self.B}, {self.Hkv}, Tn, {self.D}], got "
                               f"{list(k_new.shape)}")
        end = self.length + Tn
        if end > self.capacity:
            self._grow(end)
        self.k[:, :, self.length:end] = k_new.to(self.dtype)
        self.v[:, :, self.length:end] = v_new.to(self.dtype)
        self.length = end
        self.encode(prefill=prefill)

    @torch.no_grad()
    def encode(self, prefill: bool = False, resid_norm: torch.Tensor | None = None) -> int:
        """Encode [encoded_len, length) if the policy allows; returns rows encoded."""
        rng = flush_range(self.length, self.encoded_len, self.group_size, prefill)
        if rng is None:
            return 0
        t0, t1 = rng
        k, c = self.k, self.codes
        N.call("lap_encode_keys", N.ptr(k), N.dtype_code(k.dtype), k.stride(0), k.stride(1),
               k.stride(2), self.B, self.Hkv, t0, t1, self.D, N.ptr(self.cb), self.M, self.K,
               N.ptr(self.prep), self.prep.numel(), N.ptr(c), c.stride(0), c.stride(1),
               c.stride(2), N.ptr(resid_norm), N.stream_of(k))
        self.encoded_len = t1
        return self.B * self.Hkv * (t1 - t0)

    def keys(self) -> torch.Tensor:
        return self.k[:, :, :self.length]

    def values(self) -> torch.Tensor:
        return self.v[:, :, :self.length]

    def encoded_codes(self) -> torch.Tensor:
        """[B, Hkv, encoded_len, M] view (strided in the capacity buffer)."""
        return self.codes[:, :, :self.encoded_len]
