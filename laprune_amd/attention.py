"""Drop-in ``do_sdpa_attn`` (laprune/attention.py:21-73).

Same signature, argument meaning and errors as the reference: post-RoPE
query/key/value ``[B, H, T, D]``, optional down-projections, an optional
mask, native GQA, output ``[B, T, H*D]`` through ``out_proj`` when given.

A single query without a mask or down-projections (decode; the reference's
``num_queries == 1`` branch, :62-65) runs the split-K flash-decode kernel
(``lap_dense_attn_decode``): fp16/bf16, head dim 64/128/256, 1/2/4/8 query
heads per KV head, K/V rows 16-byte aligned.  Every other case (prefill with
the causal or tail-causal mask, an explicit mask, down-projections, shapes
outside the kernel's contract) runs ``scaled_dot_product_attention`` exactly
as the reference does.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _tail_causal_mask(num_queries: int, num_keys: int, dtype, device) -> torch.Tensor:
    """Additive mask for queries at the last positions of the cache
    (laprune/attention.py:6-18): query i sees keys up to num_keys - nq + i."""
    if num_queries > num_keys:
        raise ValueError(f"num_queries={num_queries} exceeds num_keys={num_keys}")
    allowed = torch.ones(num_queries, num_keys, dtype=torch.bool, device=device).tril(
        diagonal=num_keys - num_queries)
    mask = torch.zeros(1, 1, num_queries, num_keys, dtype=torch.float32, device=device)
    mask.masked_fill_(~allowed, torch.finfo(dtype).min)
    return mask.to(dtype=dtype)


def _decode_kernel_fits(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        return False
    if q.dim() != 4 or k.dim() != 4 or v.shape != k.shape or q.shape[2] != 1:
        return False
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype or v.dtype != q.dtype:
        return False
    B, Hq, _, D = q.shape
    Hkv = k.shape[1]
    if k.shape[0] != B or k.shape[3] != D or D not in (64, 128, 256) or k.shape[2] < 1:
        return False
    if Hq % Hkv or not 1 <= Hq // Hkv <= 8:
        return False
    if q.stride(3) != 1 or k.stride(3) != 1 or v.stride(3) != 1:
        return False
    for t in (k, v):  # rows are read as 16-byte vectors
        if t.data_ptr() % 16 or any(s % 8 for s in t.stride()[:3]):
            return False
    return True


def do_sdpa_attn(query, key, value, cos=None, sin=None, out_proj=None, query_down_proj=None,
                 key_down_proj=None, mask=None, already_rope: bool = False):
    """Attention over post-RoPE Q/K with native GQA caches."""
    if not already_rope:
        raise ValueError("LAPrune attention expects post-RoPE query and key tensors")
    q, k, v = query, key, value
    num_heads = int(q.shape[1])
    num_queries = int(q.shape[-2])
    if query_down_proj is not None:
        q = q.transpose(1, 2).flatten(2) @ query_down_proj
        q = q.unflatten(-1, (num_heads, -1)).transpose(1, 2)
    if key_down_proj is not None:
        k = k.transpose(1, 2).flatten(2) @ key_down_proj
        k = k.unflatten(-1, (num_heads, -1)).transpose(1, 2)
    enable_gqa = int(q.shape[1]) != int(k.shape[1])
    if enable_gqa and int(q.shape[1]) % int(k.shape[1]) != 0:
        raise ValueError(f"invalid GQA head counts: Hq={q.shape[1]}, Hkv={k.shape[1]}")

    if (mask is None and num_queries == 1 and query_down_proj is None
            and key_down_proj is None and _decode_kernel_fits(q, k, v)):
        from .aq_kernels import _impl
        output = _impl.dense_attn_decode(q, k, v)
    elif mask is not None:
        output = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, is_causal=False,
                                                enable_gqa=enable_gqa)
    else:
        num_keys = int(k.shape[-2])
        if num_keys == num_queries:
            output = F.scaled_dot_product_attention(q, k, v, attn_mask=None, is_causal=True,
                                                    enable_gqa=enable_gqa)
        elif num_queries == 1:
            output = F.scaled_dot_product_attention(q, k, v, attn_mask=None, is_causal=False,
                                                    enable_gqa=enable_gqa)
        else:
            causal = _tail_causal_mask(num_queries, num_keys, q.dtype, q.device)
            output = F.scaled_dot_product_attention(q, k, v, attn_mask=causal, is_causal=False,
                                                    enable_gqa=enable_gqa)
    output = output.transpose(1, 2).flatten(2)
    return out_proj(output) if out_proj is not None else output
