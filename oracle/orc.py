"""CPU oracle for the decode-time retrieval path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module.  The product (``laprune_amd``) never does.

Two layers:
  * ``aq_oracle.c`` (loaded here through ctypes) restates each hot-path
    function in scalar C with the explicit arithmetic order the gfx950
    kernels promise, so GPU results can be compared bit for bit;
  * numpy / float64 helpers here give independent truths (exact rational
    arithmetic, float64 closed forms, stable sorts) that pin the C
    restatement itself.

What pins each function (tests/test_oracle_pins.py):
  f2h / h2f      all 65536 fp16 patterns round-trip; 200k random floats
                 against numpy's float32->float16 (IEEE RNE) conversion.
  lut_build      exact-rational fmaf chain on small shapes (bit-exact);
                 float64 matmul within the fp32 error bound; one-hot
                 codebooks return q entries; linearity in q.
  score_*        independent numpy float32 sequential sum (bit-exact);
                 all-zero codes = sum of column 0; one-hot LUT counts codes;
                 grouped == per-head == expanded-MHA (reference fallback
                 identity, laprune/llm/aq_kv.py:695-699).
  topk           numpy lexsort on (-key, index); closed-form budgets
                 (n=131008 -> 2621, n=8128 -> 163); all-equal rows; k >= n.
  reconstruct    numpy float32 sequential sum (bit-exact); a crafted case
                 where the m order changes the fp32 result; one-hot
                 codebooks give the code pattern; float64 sum within the
                 fp32 bound.
  encode         exact-rational dot16 on small shapes; float64 argmin with
                 teacher forcing (codes equal except documented near-ties);
                 constructed codebooks (exact recovery, zero input chain).
  attention      float64 softmax.V; all-tokens keep list equals torch's CPU
                 scaled_dot_product_attention; single key returns V row.
No function is "parity unpinned": the reference ships no tests or golden
vectors, so every pin above is mathematical or an independent restatement.
"""
from __future__ import annotations

import ctypes as C
import math
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle.so"

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            from . import build as _b
            _b.build()
        L = C.CDLL(str(LIB))
        vp, i32, i64 = C.c_void_p, C.c_int, C.c_int64
        L.orc_h2f.argtypes = [C.c_uint16]
        L.orc_h2f.restype = C.c_float
        L.orc_f2h.argtypes = [C.c_float]
        L.orc_f2h.restype = C.c_uint16
        L.orc_f2bf.argtypes = [C.c_float]
        L.orc_f2bf.restype = C.c_uint16
        L.orc_lut_build.argtypes = [vp, vp, i32, i32, i32, i32, vp]
        L.orc_score_grouped.argtypes = [vp, vp, i64, i64, i32, i32, i32, i32, i32, vp]
        L.orc_score_gqa.argtypes = [vp, vp, i64, i64, i32, i32, i32, i32, i32, i32, i32, vp, i32, vp]
        L.orc_score_mha.argtypes = [vp, i32, vp, i32, i32, i32, i32, vp]
        L.orc_aq_direct.argtypes = [vp, vp, i32, vp, i32, i32, i32, i32, i32, vp]
        L.orc_reconstruct.argtypes = [vp, vp, i32, i32, i32, i32, vp]
        L.orc_topk.argtypes = [vp, i64, i32, i32, i32, i32, i32, i32, vp]
        L.orc_topk.restype = C.c_int
        L.orc_dot16.argtypes = [vp, vp, i32]
        L.orc_dot16.restype = C.c_float
        L.orc_encode.argtypes = [vp, vp, i32, i32, i32, i32, vp, vp, vp]
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else C.c_void_p(a.ctypes.data)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ------------------------------------------------------------- conversions

def f2h_scalar(x: float) -> int:
    return int(lib().orc_f2h(float(x)))


def h2f_scalar(h: int) -> float:
    return float(lib().orc_h2f(int(h)))


def h_bits(a) -> np.ndarray:
    """fp16 values (numpy float16 or torch tensor converted) -> uint16 bits."""
    return np.ascontiguousarray(np.asarray(a, dtype=np.float16)).view(np.uint16)


def h_vals(bits: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def f2bf_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits (RNE), vectorised, same rule as the C oracle."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf_vals(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# --------------------------------------------------------------------- A1

def lut_build(q: np.ndarray, cb: np.ndarray) -> np.ndarray:
    """fp16 bits [Hq, M, K]: fmaf chain over d, RNE to fp16."""
    q = _c(q, np.float32)
    cb = _c(cb, np.float32)
    Hq, D = q.shape
    M, K, _ = cb.shape
    out = np.empty((Hq, M, K), dtype=np.uint16)
    lib().orc_lut_build(_p(q), _p(cb), Hq, D, M, K, _p(out))
    return out


def lut_to_gmkg(lut_hmk: np.ndarray, G: int) -> np.ndarray:
    Hq, M, K = lut_hmk.shape
    return np.ascontiguousarray(lut_hmk.reshape(Hq // G, G, M, K).transpose(0, 2, 3, 1))


# --------------------------------------------------------------------- A2

def score_grouped(lut: np.ndarray, codes: np.ndarray, G: int) -> np.ndarray:
    """lut fp16 bits [H, M, K]; codes uint8 [Hkv, T, M] (any strides, M unit)."""
    lut = _c(lut, np.uint16)
    assert codes.dtype == np.uint8 and codes.strides[2] == 1
    H, M, K = lut.shape
    Hkv, T, _ = codes.shape
    out = np.empty((H, T), dtype=np.uint16)
    lib().orc_score_grouped(_p(lut), C.c_void_p(codes.ctypes.data), codes.strides[0],
                            codes.strides[1], Hkv, G, T, M, K, _p(out))
    return out


def score_gqa(lut: np.ndarray, codes: np.ndarray, G: int, M_start: int, M_end: int,
              indices: np.ndarray | None = None) -> np.ndarray:
    lut = _c(lut, np.uint16)
    assert codes.dtype == np.uint8 and codes.strides[2] == 1
    H, Ms, K = lut.shape
    Hkv, T, _ = codes.shape
    idx = None if indices is None else _c(indices, np.int64)
    n = T if idx is None else idx.shape[1]
    out = np.empty((H, n), dtype=np.uint16)
    lib().orc_score_gqa(_p(lut), C.c_void_p(codes.ctypes.data), codes.strides[0],
                        codes.strides[1], Hkv, G, T, Ms, K, M_start, M_end, _p(idx), n, _p(out))
    return out


def score_mha(lut: np.ndarray, codes: np.ndarray, f32: bool) -> np.ndarray:
    """lut [Q, M*K] (float32 values or fp16 bits); codes any int dtype [Q, N, M]."""
    lut = _c(lut, np.float32 if f32 else np.uint16)
    codes64 = _c(codes.astype(np.int64), np.int64)
    Q, n, M = codes64.shape
    K = lut.shape[1] // M
    out = np.empty((Q, n), dtype=np.float32 if f32 else np.uint16)
    lib().orc_score_mha(_p(lut), 1 if f32 else 0, _p(codes64), Q, n, M, K, _p(out))
    return out


def reconstruct(cb: np.ndarray, codes: np.ndarray) -> np.ndarray:
    """float32 [N, D]: sum over m ascending of cb[m, codes[:, m]] (fp32, from 0)."""
    cb = _c(cb, np.float32)
    codes64 = _c(codes.astype(np.int64), np.int64)
    n, M = codes64.shape
    Mc, K, D = cb.shape
    assert Mc == M
    out = np.empty((n, D), dtype=np.float32)
    lib().orc_reconstruct(_p(cb), _p(codes64), n, M, K, D, _p(out))
    return out


def aq_direct(q: np.ndarray, cb: np.ndarray, codes: np.ndarray, f16: bool) -> np.ndarray:
    """q [Q,D], cb [M,K,D] as float32 values or fp16 bits (f16=True)."""
    dt = np.uint16 if f16 else np.float32
    q = _c(q, dt)
    cb = _c(cb, dt)
    codes64 = _c(codes.astype(np.int64), np.int64)
    Q, n, M = codes64.shape
    _, K, D = cb.shape
    out = np.empty((Q, n), dtype=np.uint16 if f16 else np.float32)
    lib().orc_aq_direct(_p(q), _p(cb), 1 if f16 else 0, _p(codes64), Q, n, M, K, D, _p(out))
    return out


# --------------------------------------------------------------------- A3

def topk(scores: np.ndarray, k: int, group: int = 1, cand_start: int = 0,
         cand_end: int | None = None, key_bf16: bool = False) -> np.ndarray:
    """scores fp16 bits [R*group, T] -> int64 [R, min(k, n)] ascending."""
    scores = _c(scores, np.uint16)
    rows, T = scores.shape
    R = rows // group
    ce = T if cand_end is None else cand_end
    ke = max(0, min(k, ce - cand_start))
    out = np.zeros((R, max(k, 1)), dtype=np.int64)
    lib().orc_topk(_p(scores), T, R, group, cand_start, ce, k, 1 if key_bf16 else 0, _p(out))
    return out[:, :ke].copy()


def key16(bits: np.ndarray) -> np.ndarray:
    """Orderable key of fp16 bits (numpy restatement, independent of the C)."""
    b = np.asarray(bits, dtype=np.uint32)
    b = np.where((b & 0x7FFF) == 0, 0, b)
    return np.where(b & 0x8000, (~b) & 0xFFFF, b | 0x8000).astype(np.uint32)


def topk_numpy(scores: np.ndarray, k: int, group: int = 1, cand_start: int = 0,
               cand_end: int | None = None, key_bf16: bool = False) -> np.ndarray:
    """Independent restatement by lexsort on (-key, index)."""
    rows, T = scores.shape
    R = rows // group
    ce = T if cand_end is None else cand_end
    n = ce - cand_start
    ke = max(0, min(k, n))
    out = np.zeros((R, ke), dtype=np.int64)
    for r in range(R):
        blk = scores[r * group:(r + 1) * group, cand_start:ce]
        if key_bf16:
            blk = f2bf_bits(h_vals(blk.reshape(-1))).reshape(blk.shape)
        key = key16(blk).max(axis=0)
        order = np.lexsort((np.arange(n), -key.astype(np.int64)))
        out[r] = np.sort(order[:ke]) + cand_start
    return out


def candidate_window(t_codes: int, t_total: int, sink: int, local: int):
    """(cand_start, cand_end) of laprune/llm/modifiers/aq_evaluation.py:189-193."""
    sink_end = min(sink, t_codes) if sink > 0 else 0
    local_start = max(t_total - max(local, 0), 0)
    cand_start = sink_end
    cand_end = min(t_codes, local_start) if local > 0 else t_codes
    return cand_start, max(cand_start, cand_end)


def budget_k(n: int, mask_out: float = 0.98, min_remain: int = 20) -> int:
    """Top-k budget of aq_evaluation.py:195-197."""
    if n <= 0:
        return 0
    k = n - int(n * mask_out)
    k = max(min(n, min_remain), k)
    return max(1, min(k, n))


# --------------------------------------------------------------------- A6

def dot16(a: np.ndarray, b: np.ndarray) -> np.float32:
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    return np.float32(lib().orc_dot16(_p(a), _p(b), a.shape[0]))


def encode(x: np.ndarray, cb: np.ndarray, trace: bool = False):
    """codes uint8 [N, M], rnorm float32 [N] (and dists [N, M, K] if trace)."""
    x = _c(x, np.float32)
    cb = _c(cb, np.float32)
    n, D = x.shape
    M, K, _ = cb.shape
    codes = np.empty((n, M), dtype=np.uint8)
    rnorm = np.empty((n,), dtype=np.float32)
    tr = np.empty((n, M, K), dtype=np.float32) if trace else None
    lib().orc_encode(_p(x), _p(cb), n, M, K, D, _p(codes), _p(rnorm), _p(tr))
    return (codes, rnorm, tr) if trace else (codes, rnorm)


# --------------------------------------------------------------------- A4/A5

def keep_list(topk_idx: np.ndarray, t_total: int, sink: int, local: int) -> np.ndarray:
    """Keep set of aq_evaluation.py:210-237 (explicit-parts form): top-k ++ sinks ++ local."""
    sb = min(sink, t_total) if sink > 0 else 0
    start = max(t_total - local, 0) if local > 0 else t_total
    if start <= 0:
        sb_eff = 0
    else:
        sb_eff = sb
        if start < sb_eff:
            start = sb_eff
    parts = [np.asarray(topk_idx, dtype=np.int64)]
    if sb_eff > 0:
        parts.append(np.arange(sb_eff, dtype=np.int64))
    if local > 0 and start < t_total:
        parts.append(np.arange(start, t_total, dtype=np.int64))
    keep = np.concatenate(parts)
    if keep.size == 0 and t_total > 0:  # nothing kept: the newest token (:233-234)
        keep = np.array([t_total - 1], dtype=np.int64)
    return keep


def gather_rows(kv: np.ndarray, idx: np.ndarray, G: int) -> np.ndarray:
    """out[b,hq,n] = kv[b, hq//G, idx[b,hq,n]] (rows outside [0,T) -> NaN marker)."""
    B, Hkv, T, D = kv.shape
    _, Hq, n = idx.shape
    out = np.full((B, Hq, n, D), np.nan, dtype=np.float64)
    for b in range(B):
        for h in range(Hq):
            ii = idx[b, h]
            ok = (ii >= 0) & (ii < T)
            out[b, h, ok] = kv[b, h // G, ii[ok]]
    return out


def attn_decode_f64(q: np.ndarray, K: np.ndarray, V: np.ndarray, keep, scale: float | None = None):
    """float64 single-query attention.  q [B,Hq,D]; K,V [B,Hkv,T,D];
    keep(b, h) -> int array of token ids (ids outside [0,T) are skipped)."""
    B, Hq, D = q.shape
    Hkv, T = K.shape[1], K.shape[2]
    G = Hq // Hkv
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    out = np.zeros((B, Hq, D), dtype=np.float64)
    for b in range(B):
        for h in range(Hq):
            ids = np.asarray(keep(b, h), dtype=np.int64)
            ids = ids[(ids >= 0) & (ids < T)]
            if ids.size == 0:
                continue
            kk = K[b, h // G, ids].astype(np.float64)
            vv = V[b, h // G, ids].astype(np.float64)
            s = kk @ q[b, h].astype(np.float64) * sc
            w = np.exp(s - s.max())
            out[b, h] = (w @ vv) / w.sum()
    return out
