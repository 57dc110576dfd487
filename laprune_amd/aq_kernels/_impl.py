"""Torch-facing implementations of the ``aq_kernels`` names over the C ABI.

Each function validates its arguments the way the reference host function
does (the TORCH_CHECKs cited per function), allocates outputs with torch on
the input's device, and launches on the current torch stream.  No function
here computes anything on the CPU.
"""
from __future__ import annotations

import math
import threading

import torch

from .. import _native as N
from .._ops import ops

_ws_lock = threading.Lock()
_ws_cache: dict = {}


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A per-device scratch buffer of at least ``nbytes`` (grown on demand)."""
    key = (device.type, device.index)
    with _ws_lock:
        buf = _ws_cache.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            _ws_cache[key] = buf
        return buf


def _device_guard(t: torch.Tensor):
    return torch.cuda.device(t.device)


# --------------------------------------------------------------------- A1

def aq_lut_build(q: torch.Tensor, codebooks: torch.Tensor, G: int = 1,
                 layout: str = "hmk") -> torch.Tensor:
    """fp16 LUT ``lut[h,m,k] = q[h] . codebooks[m,k]`` (fp32 fmaf chain over d).

    ``layout="hmk"`` returns [Hq, M, K] (the reference's layout,
    laprune/llm/aq_kv.py:681-682); ``layout="gmkg"`` returns
    [Hq/G, M, K, G] (query heads of one KV group interleaved).
    """
    N.require_cuda(q, codebooks)
    _check(q.dim() == 2 and codebooks.dim() == 3, "expected q [Hq, d] and codebooks [M, K, d]")
    Hq, D = q.shape
    M, K, Dc = codebooks.shape
    _check(D == Dc, "q and codebooks last dim must match")
    _check(q.stride(1) == 1, "q rows must be contiguous")
    if q.data_ptr() % 16 or q.stride(0) % 4:  # the kernels read q four elements at a time
        q = q.clone(memory_format=torch.contiguous_format)
    cb = codebooks.contiguous()
    if cb.data_ptr() % 16:
        cb = cb.clone()
    lay = N.LUT_HMK if layout == "hmk" else N.LUT_GMKG
    if lay == N.LUT_HMK:
        out = torch.empty((Hq, M, K), dtype=torch.float16, device=q.device)
    else:
        _check(G > 0 and Hq % G == 0, f"Hq={Hq} not divisible by G={G}")
        out = torch.empty((Hq // G, M, K, G), dtype=torch.float16, device=q.device)
    with _device_guard(q):
        ops().lut_build(q, cb, G, lay, out)
    return out


# --------------------------------------------------------------------- A2

def aq_lut_gather_grouped(lut: torch.Tensor, codes: torch.Tensor, G: int,
                          grid_y_cap: int = 48) -> torch.Tensor:
    """Reference: aq_kernels/aq_lut_gqa.cu:460-534 (``aq_lut_gather_grouped``)."""
    _check(lut.is_cuda and codes.is_cuda, "tensors must be CUDA")
    _check(lut.dtype == torch.float16 and codes.dtype == torch.uint8,
           "grouped LUT requires fp16 LUT and uint8 codes")
    _check(lut.dim() == 3 and codes.dim() == 3, "expected lut [H,M,K] and codes [Hkv,T,M]")
    _check(codes.stride(2) == 1, "codes M dimension must be contiguous")
    lut_c = lut.contiguous()
    H, M, K = lut_c.shape
    Hkv, T, Mc = codes.shape
    _check(H == Hkv * G, "H must equal Hkv*G")
    _check(0 < G <= 4, "grouped kernel supports G<=4")
    _check(Mc >= M, "codes M dimension smaller than the LUT's")
    out = torch.empty((H, T), dtype=torch.float16, device=lut.device)
    if T == 0:
        return out
    _check(grid_y_cap > 0, "grid_y_cap must be positive")
    with _device_guard(lut):
        ops().score_grouped(lut_c, N.LUT_HMK, codes, G, M, K, out)
    return out


def aq_lut_gather(lut: torch.Tensor, codes: torch.Tensor, G: int, M_start: int, M_end: int,
                  indices: torch.Tensor | None = None) -> torch.Tensor:
    """Reference: aq_kernels/aq_lut_gqa.cu:350-422 (``aq_lut_gather``, exported as
    ``aq_lut_gather_gqa``)."""
    _check(lut.is_cuda and codes.is_cuda, "tensors must be on CUDA")
    _check(lut.dtype == torch.float16, "lut must be fp16")
    _check(codes.dtype == torch.uint8, "codes must be uint8")
    _check(lut.dim() == 3 and codes.dim() == 3, "lut and codes must be 3-D")
    lut_c = lut.contiguous()
    _check(codes.stride(2) == 1, "codes M dimension must be contiguous")
    H, M_stride, K = lut_c.shape
    Hkv, T, _ = codes.shape
    _check(H == Hkv * G, "H must equal Hkv * G")
    _check(M_end <= M_stride and M_start >= 0 and M_end - M_start > 0, "invalid M range")
    idx = None
    n = T
    if indices is not None:
        idx = indices.contiguous().to(torch.int64)
        _check(idx.size(0) == H, "indices must have H rows")
        n = idx.size(1)
    out = torch.empty((H, n), dtype=torch.float16, device=lut.device)
    if n == 0:
        return out
    with _device_guard(lut):
        N.call("lap_lut_score_gqa", N.ptr(lut_c), N.ptr(codes), codes.stride(0), codes.stride(1),
               Hkv, G, T, M_stride, K, M_start, M_end, N.ptr(idx), n, N.ptr(out),
               N.stream_of(lut))
    return out


def aq_lut_gather_forward(lut: torch.Tensor, codes: torch.Tensor) -> torch.Tensor:
    """Reference: aq_kernels/aq_lut.cu:641-738 (``aq_lut_gather_forward``)."""
    _check(lut.is_cuda, "lut must be a CUDA tensor")
    _check(codes.is_cuda, "codes must be a CUDA tensor")
    _check(lut.device == codes.device, "lut and codes must be on the same CUDA device")
    _check(lut.dim() == 2, "lut must be of shape [Q, M*K]")
    _check(codes.dim() == 3, "codes must be of shape [Q, N, M]")
    _check(lut.dtype in (torch.float16, torch.float32), "lut must be fp16 or fp32")
    _check(codes.dtype in (torch.int64, torch.uint8, torch.int8),
           "codes must be int64 (Long) or uint8 (Byte) or int8 (Char)")
    lut = lut.contiguous()
    codes = codes.contiguous()
    Q, MK = lut.shape
    Qc, n, M = codes.shape
    _check(Qc == Q, "codes Q dimension must match lut Q")
    _check(M > 0, "codes M dimension must be > 0")
    _check(MK % M == 0, "lut second dim must be divisible by M (expect M*K)")
    K = MK // M
    out = torch.empty((Q, n), dtype=lut.dtype, device=lut.device)
    if n == 0 or Q == 0:
        return out
    with _device_guard(lut):
        N.call("lap_lut_score_mha", N.ptr(lut), N.dtype_code(lut.dtype), N.ptr(codes),
               N.dtype_code(codes.dtype), Q, n, M, K, N.ptr(out), N.stream_of(lut))
    return out


def aq_lut_forward(q: torch.Tensor, codebooks: torch.Tensor, codes: torch.Tensor) -> torch.Tensor:
    """Reference: aq_kernels/aq_lut.cu:445-574 (``aq_lut_forward``)."""
    _check(q.is_cuda, "q must be a CUDA tensor")
    _check(codebooks.is_cuda, "codebooks must be a CUDA tensor")
    _check(codes.is_cuda, "codes must be a CUDA tensor")
    _check(q.device == codebooks.device, "q and codebooks must be on the same CUDA device")
    _check(q.device == codes.device, "q and codes must be on the same CUDA device")
    _check(q.dim() == 2, "q must be of shape [Q, d]")
    _check(codebooks.dim() == 3, "codebooks must be of shape [M, K, d]")
    _check(codes.dim() == 3, "codes must be of shape [Q, N, M]")
    _check(q.dtype == codebooks.dtype, "q and codebooks must have the same dtype")
    _check(codes.dtype in (torch.int64, torch.uint8, torch.int8),
           "codes must be int64 (Long) or uint8 (Byte) or int8 (Char)")
    _check(q.dtype in (torch.float32, torch.float16),
           "aq_lut_forward on the HIP path serves fp32 and fp16")
    q = q.contiguous()
    codebooks = codebooks.contiguous()
    codes = codes.contiguous()
    Q, d = q.shape
    M, K, d_cb = codebooks.shape
    _check(d == d_cb, "q and codebooks last dim must match")
    Qc, n, Mc = codes.shape
    _check(Qc == Q, "codes Q dimension must match q")
    _check(Mc == M, "codes M dimension must match codebooks")
    out = torch.empty((Q, n), dtype=q.dtype, device=q.device)
    if n == 0 or Q == 0:
        return out
    with _device_guard(q):
        N.call("lap_aq_lut_direct", N.ptr(q), N.ptr(codebooks), N.dtype_code(q.dtype),
               N.ptr(codes), N.dtype_code(codes.dtype), Q, n, M, K, d, N.ptr(out),
               N.stream_of(q))
    return out


# --------------------------------------------------------------------- A3

def _key_mode(key_dtype: torch.dtype) -> int:
    if key_dtype == torch.float16:
        return N.KEY_F16
    if key_dtype == torch.bfloat16:
        return N.KEY_BF16
    raise RuntimeError("key_dtype must be torch.float16 or torch.bfloat16")


def aq_topk(scores: torch.Tensor, k: int, group: int = 1, cand_start: int = 0,
            cand_end: int | None = None, key_dtype: torch.dtype = torch.float16,
            index_dtype: torch.dtype = torch.int64) -> torch.Tensor:
    """Top-k column indices of fp16 ``scores`` [R*group, T] over [cand_start, cand_end).

    The key of row r is the max over its ``group`` consecutive score rows,
    ranked as ``key_dtype`` (bfloat16 reproduces the model-dtype cast before
    ``torch.topk`` at aq_evaluation.py:166).  Returns [R, min(k, n)] indices in
    ascending order; ties at the threshold keep the lowest columns.
    """
    N.require_cuda(scores)
    _check(scores.dtype == torch.float16 and scores.dim() == 2, "scores must be fp16 [rows, T]")
    _check(scores.stride(1) == 1, "scores columns must be contiguous")
    rows, T = scores.shape
    _check(group > 0 and rows % group == 0, "rows must be a multiple of group")
    R = rows // group
    ce = T if cand_end is None else cand_end
    _check(0 <= cand_start <= ce <= T, "candidate window outside [0, T)")
    n = ce - cand_start
    ke = min(int(k), n)
    _check(k >= 0, "k must be non-negative")
    _check(index_dtype in (torch.int32, torch.int64), "index dtype must be int32/int64")
    out = torch.empty((R, ke), dtype=index_dtype, device=scores.device)
    if ke == 0:
        return out
    ws_bytes = N.size_query("lap_topk_workspace_size", R, n)
    ws = _workspace(scores.device, ws_bytes)
    with _device_guard(scores):
        N.call("lap_topk_select", N.ptr(scores), scores.stride(0), R, group, T, cand_start, ce,
               ke, _key_mode(key_dtype), N.ptr(out), N.dtype_code(index_dtype), N.ptr(ws),
               ws.numel(), N.stream_of(scores))
    return out


def aq_retrieve_topk(lut_gmkg: torch.Tensor, codes: torch.Tensor, k: int, cand_start: int = 0,
                     cand_end: int | None = None, key_dtype: torch.dtype = torch.float16,
                     index_dtype: torch.dtype = torch.int32, return_scores: bool = False,
                     per_head: bool = False):
    """Fused LUT scoring + top-k for G=4, M=32, K=256.

    ``lut_gmkg`` [B*Hkv, 32, 256, 4] fp16 (from ``aq_lut_build(..., layout="gmkg")``),
    ``codes`` u8 [B, Hkv, T, 32] (any T/H/B strides, M contiguous).  Returns
    indices [B, Hkv, min(k, n)] (ascending; one top-k per KV group on the max
    of its 4 query-head scores) or, with ``per_head``, [B, Hkv*4, min(k, n)]
    (one top-k per query head, the reference's selection), and optionally the
    per-head fp16 scores [B, Hkv*4, T].
    """
    N.require_cuda(lut_gmkg, codes)
    _check(lut_gmkg.dtype == torch.float16 and codes.dtype == torch.uint8,
           "fused retrieval requires fp16 LUT and uint8 codes")
    _check(codes.dim() == 4 and codes.shape[-1] == 32 and codes.stride(3) == 1,
           "codes must be [B, Hkv, T, 32] with M contiguous")
    B, Hkv, T, _ = codes.shape
    _check(tuple(lut_gmkg.shape) == (B * Hkv, 32, 256, 4) and lut_gmkg.is_contiguous(),
           "lut must be contiguous [B*Hkv, 32, 256, 4]")
    ce = T if cand_end is None else cand_end
    _check(0 <= cand_start <= ce <= T, "candidate window outside [0, T)")
    ke = min(int(k), ce - cand_start)
    _check(k >= 0, "k must be non-negative")
    rows = Hkv * 4 if per_head else Hkv
    out = torch.empty((B, rows, ke), dtype=index_dtype, device=codes.device)
    scores = (torch.empty((B, Hkv * 4, T), dtype=torch.float16, device=codes.device)
              if return_scores else None)
    ws_bytes = N.size_query("lap_retrieve_workspace_size", B * rows, T)
    ws = _workspace(codes.device, ws_bytes)
    mode = _key_mode(key_dtype) | (N.SELECT_PER_HEAD if per_head else 0)
    with _device_guard(codes):
        N.call("lap_retrieve_topk", N.ptr(lut_gmkg), N.ptr(codes), codes.stride(0),
               codes.stride(1), codes.stride(2), B, Hkv, T, cand_start, ce, ke, mode,
               N.ptr(scores), N.ptr(out), N.dtype_code(index_dtype), N.ptr(ws), ws.numel(),
               N.stream_of(codes))
    return (out, scores) if return_scores else out


# --------------------------------------------------------------------- A4

def _gather_checks(keys, vals, indices, threads, vector_width):
    _check(keys.is_cuda and vals.is_cuda and indices.is_cuda,
           "keys, vals and indices must be CUDA tensors")
    _check(keys.dtype in (torch.float16, torch.bfloat16) and vals.dtype == keys.dtype,
           "gqa_gather_kv supports fp16/bf16 K/V of one dtype")
    _check(indices.dtype == torch.int64, "indices must be int64")
    _check(keys.dim() == 4 and vals.dim() == 4 and indices.dim() == 3,
           "expected K/V [B,Hkv,T,D] and indices [B,Hq,N]")
    _check(keys.shape == vals.shape, "K/V shapes must match")
    _check(keys.stride(3) == 1 and vals.stride(3) == 1, "K/V head dimension must be contiguous")
    _check(vector_width in (2, 8), "vector_width must be 2 or 8 half elements")
    D = keys.shape[3]
    _check(D > 0 and D % 2 == 0, "D must be positive and even")
    _check(D % vector_width == 0, "D must be divisible by vector_width")
    dvec = D // vector_width
    _check(threads in (256, 512, 1024) and dvec <= threads and threads % dvec == 0,
           "threads must be 256/512/1024 and divisible by D/vector_width")


def _gather(keys, vals, idx, G, explicit_n, tail_start, tail_count):
    B, Hkv, T, D = keys.shape
    Hq = idx.shape[1]
    n = explicit_n + tail_count
    out_k = torch.empty((B, Hq, n, D), dtype=keys.dtype, device=keys.device)
    out_v = torch.empty((B, Hq, n, D), dtype=vals.dtype, device=vals.device)
    if n == 0:
        return [out_k, out_v]
    with _device_guard(keys):
        N.call("lap_gqa_gather_kv", N.ptr(keys), N.ptr(vals), N.dtype_code(keys.dtype), B, Hkv,
               T, D, keys.stride(0), keys.stride(1), keys.stride(2), vals.stride(0),
               vals.stride(1), vals.stride(2), N.ptr(idx), Hq, explicit_n, tail_start,
               tail_count, N.ptr(out_k), N.ptr(out_v), N.stream_of(keys))
    return [out_k, out_v]


def gqa_gather_kv(keys: torch.Tensor, vals: torch.Tensor, indices: torch.Tensor, G: int,
                  threads: int = 256, vector_width: int = 8):
    """Reference: aq_kernels/aq_lut_gqa.cu:536-604 (``gqa_gather_kv``)."""
    _gather_checks(keys, vals, indices, threads, vector_width)
    B, Hkv, T, D = keys.shape
    _check(indices.size(0) == B, "indices batch mismatch")
    _check(indices.size(1) == Hkv * G, "Hq must equal Hkv * G")
    idx = indices.contiguous()
    return _gather(keys, vals, idx, G, idx.size(2), -1, 0)


def gqa_gather_kv_with_tail(keys: torch.Tensor, vals: torch.Tensor, indices: torch.Tensor,
                            G: int, tail_start: int, tail_count: int, threads: int = 256,
                            vector_width: int = 8):
    """Reference: aq_kernels/aq_lut_gqa.cu:606-664 (``gqa_gather_kv_with_tail``)."""
    _gather_checks(keys, vals, indices, threads, vector_width)
    B, Hkv, T, D = keys.shape
    _check(indices.size(0) == B and indices.size(1) == Hkv * G, "GQA shape mismatch")
    _check(tail_count >= 0 and tail_start >= 0 and tail_start + tail_count <= T,
           "invalid implicit tail range")
    idx = indices.contiguous()
    return _gather(keys, vals, idx, G, idx.size(2), tail_start, tail_count)


# --------------------------------------------------------------------- A5

def _attn_common(q, keys, vals):
    N.require_cuda(q, keys, vals)
    _check(q.dtype in (torch.float16, torch.bfloat16), "attention decode supports fp16/bf16")
    _check(keys.dtype == q.dtype and vals.dtype == q.dtype, "q/k/v must have same dtype")
    _check(keys.dim() == 4 and vals.shape == keys.shape, "K/V must be [B,Hkv,T,D] of one shape")
    if q.dim() == 4:
        _check(q.size(2) == 1, "q must have Q=1 when dim==4")
        q = q[:, :, 0, :]
    _check(q.dim() == 3 and q.stride(2) == 1, "q must be [B,H,D] or [B,H,1,D]")
    _check(keys.stride(3) == 1 and vals.stride(3) == 1, "K/V head dimension must be contiguous")
    B, Hq, D = q.shape
    _check(keys.shape[0] == B and keys.shape[3] == D, "q must match K/V batch and head dim")
    return q


def sparse_attn_decode(q: torch.Tensor, keys: torch.Tensor, vals: torch.Tensor,
                       indices: torch.Tensor | None, sink: int = 0, tail_start: int = -1,
                       tail_count: int = 0, scale: float | None = None) -> torch.Tensor:
    """Single-query attention over a keep list, reading K/V rows in place.

    ``q`` [B,Hq,D] or [B,Hq,1,D]; ``keys``/``vals`` [B,Hkv,T,D] (strided cache
    views are fine); ``indices`` int32/int64 [B, Hq or Hkv, n] (per query head,
    or one list per KV group).  Keep list = indices ++ [0,sink) ++
    [tail_start, tail_start+tail_count).  Returns [B,Hq,1,D].
    Replaces the gather + ``scaled_dot_product_attention`` at
    laprune/llm/modifiers/aq_evaluation.py:243-251.
    """
    q3 = _attn_common(q, keys, vals)
    B, Hq, D = q3.shape
    Hkv, T = keys.shape[1], keys.shape[2]
    if indices is not None:
        N.require_cuda(indices)
        _check(indices.dim() == 3 and indices.shape[0] == B, "indices must be [B, H, n]")
        _check(indices.dtype in (torch.int32, torch.int64), "idx must be int64 or int32")
        idx = indices.contiguous()
        H_idx, n_idx = idx.shape[1], idx.shape[2]
        idx_code = N.dtype_code(idx.dtype)
    else:
        idx, H_idx, n_idx, idx_code = None, Hkv, 0, N.I32
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    out = torch.empty((B, Hq, D), dtype=q.dtype, device=q.device)
    L = n_idx + sink + tail_count
    ws_bytes = N.size_query("lap_attn_decode_workspace_size", B, Hq, D, max(L, 1))
    ws = _workspace(q.device, ws_bytes)
    with _device_guard(q):
        N.call("lap_sparse_attn_decode", N.ptr(q3), q3.stride(0), q3.stride(1), N.ptr(keys),
               N.ptr(vals), N.dtype_code(q.dtype), B, Hq, Hkv, T, D, keys.stride(0),
               keys.stride(1), keys.stride(2), vals.stride(0), vals.stride(1), vals.stride(2),
               N.ptr(idx), idx_code, H_idx, n_idx, sink, tail_start, tail_count, sc,
               N.ptr(out), N.ptr(ws), ws.numel(), N.stream_of(q))
    return out.unsqueeze(2)


def dense_attn_decode(q: torch.Tensor, keys: torch.Tensor, vals: torch.Tensor,
                      scale: float | None = None) -> torch.Tensor:
    """Single-query attention over all T cached tokens (split-K flash-decode).

    Same result as ``F.scaled_dot_product_attention(q, K, V, enable_gqa=True)``
    for one query (laprune/attention.py:62-65).  Returns [B,Hq,1,D].
    """
    q3 = _attn_common(q, keys, vals)
    B, Hq, D = q3.shape
    Hkv, T = keys.shape[1], keys.shape[2]
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    out = torch.empty((B, Hq, D), dtype=q.dtype, device=q.device)
    ws_bytes = N.size_query("lap_attn_decode_workspace_size", B, Hq, D, max(T, 1))
    ws = _workspace(q.device, ws_bytes)
    with _device_guard(q):
        N.call("lap_dense_attn_decode", N.ptr(q3), q3.stride(0), q3.stride(1), N.ptr(keys),
               N.ptr(vals), N.dtype_code(q.dtype), B, Hq, Hkv, T, D, keys.stride(0),
               keys.stride(1), keys.stride(2), vals.stride(0), vals.stride(1), vals.stride(2),
               sc, N.ptr(out), N.ptr(ws), ws.numel(), N.stream_of(q))
    return out.unsqueeze(2)


# --------------------------------------------------------------------- A6

def aq_encode_prepare(codebooks: torch.Tensor) -> torch.Tensor:
    """Per-codebook encode tables (transposed codebook + entry norms), uint8 bytes."""
    N.require_cuda(codebooks)
    _check(codebooks.dim() == 3, "codebooks must be [M, K, d]")
    cb = codebooks.to(torch.float32).contiguous()
    M, K, D = cb.shape
    nbytes = N.size_query("lap_encode_prep_size", M, K, D)
    prep = torch.empty(nbytes, dtype=torch.uint8, device=cb.device)
    with _device_guard(cb):
        N.call("lap_encode_prepare", N.ptr(cb), M, K, D, N.ptr(prep), nbytes, N.stream_of(cb))
    return prep


def aq_encode_greedy(x: torch.Tensor, codebooks: torch.Tensor,
                     prep: torch.Tensor | None = None):
    """Greedy AQ codes (uint8 [N, M]) and final residual norms (fp32 [N]).

    Follows laprune/quantizer.py:346-355 (iters = 0) in fp32 with the dot16
    summation order stated in include/laprune_hip.h.
    """
    N.require_cuda(x, codebooks)
    _check(x.dim() == 2 and codebooks.dim() == 3, "expected x [N, d] and codebooks [M, K, d]")
    cb = codebooks.to(torch.float32).contiguous()
    if cb.data_ptr() % 16:  # rows are read as 16-byte vectors
        cb = cb.clone()
    M, K, D = cb.shape
    _check(x.shape[1] == D, "x and codebooks last dim must match")
    _check(K <= 256, "K must be <= 256 for uint8 codes")
    xf = x.to(torch.float32)
    if xf.stride(1) != 1:
        xf = xf.contiguous()
    if prep is None:
        prep = aq_encode_prepare(cb)
    n = xf.shape[0]
    codes = torch.empty((n, M), dtype=torch.uint8, device=x.device)
    rnorm = torch.empty((n,), dtype=torch.float32, device=x.device)
    if n == 0:
        return codes, rnorm
    with _device_guard(x):
        N.call("lap_encode_greedy", N.ptr(xf), xf.stride(0), n, D, N.ptr(cb), M, K, N.ptr(prep),
               prep.numel(), N.ptr(codes), codes.stride(0), N.ptr(rnorm), N.stream_of(x))
    return codes, rnorm


def aq_reconstruct(codebooks: torch.Tensor, codes: torch.Tensor) -> torch.Tensor:
    """Approximate keys fp32 [N, d] from codes [N, M]: the sum over m ascending
    of ``codebooks[m, codes[:, m]]`` in fp32 from 0 (laprune/llm/aq_kv.py:431-457,
    ``AQLayerCodebookManager.reconstruct``).  Codes may be uint8, int8 or
    int64; the low 8 bits are read as the code, clamped to K - 1."""
    N.require_cuda(codebooks, codes)
    _check(codebooks.dim() == 3, "codebooks must be of shape [M, K, d]")
    _check(codes.dim() == 2, "codes must be of shape [N, M]")
    _check(codes.dtype in (torch.int64, torch.uint8, torch.int8),
           "codes must be int64 (Long) or uint8 (Byte) or int8 (Char)")
    _check(codes.device == codebooks.device, "codes and codebooks must be on the same device")
    cb = codebooks.to(torch.float32).contiguous()
    if cb.data_ptr() % 16:  # rows are read as 16-byte vectors
        cb = cb.clone()
    M, K, D = cb.shape
    _check(codes.shape[1] == M, "codes M dimension must match codebooks")
    _check(D % 4 == 0, "d must be a multiple of 4")
    if codes.stride(1) != 1:
        codes = codes.contiguous()
    n = codes.shape[0]
    out = torch.empty((n, D), dtype=torch.float32, device=codebooks.device)
    if n == 0:
        return out
    with _device_guard(codebooks):
        N.call("lap_aq_reconstruct", N.ptr(cb), M, K, D, N.ptr(codes), N.dtype_code(codes.dtype),
               codes.stride(0), n, N.ptr(out), N.stream_of(codebooks))
    return out


_prep_lock = threading.Lock()
_prep_cache: dict = {}


def _cached_prep(codebooks: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    key = (codebooks.data_ptr(), tuple(codebooks.shape), codebooks.dtype,
           str(codebooks.device), codebooks._version)
    with _prep_lock:
        hit = _prep_cache.get(key)
        if hit is None:
            cb = codebooks.to(torch.float32).contiguous()
            hit = (cb, aq_encode_prepare(cb))
            _prep_cache.clear()
            _prep_cache[key] = hit
        return hit


def fused_linear_encode_forward(x: torch.Tensor, weight_t: torch.Tensor, bias: torch.Tensor,
                                codebooks: torch.Tensor, fp32_residual: bool = True,
                                tile_n: int = 0) -> torch.Tensor:
    """Reference: aq_kernels/fused_linear_encode.cu:168-234.

    ``weight_t`` [M, d, K] and ``bias`` [M, K] are what the reference derives
    from ``codebooks`` (laprune/llm/aq_kv.py:69-71); they are shape-checked and
    the codes follow the fp32 greedy argmin over ``codebooks``.
    """
    _check(x.is_cuda, "x must be CUDA")
    _check(x.dim() == 2 and weight_t.dim() == 3 and bias.dim() == 2 and codebooks.dim() == 3,
           "expected x [N,d], weight_t [M,d,K], bias [M,K], codebooks [M,K,d]")
    M, d, K = weight_t.shape
    _check(tuple(codebooks.shape) == (M, K, d), "codebooks must be [M, K, d] matching weight_t")
    _check(tuple(bias.shape) == (M, K), "bias must be [M, K]")
    _check(x.shape[1] == d, "x and weight_t inner dims must match")
    cb, prep = _cached_prep(codebooks)
    codes, _ = aq_encode_greedy(x, cb, prep)
    return codes
