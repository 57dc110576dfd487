"""Drop-in ``aq_kernels`` package backed by the gfx950 C ABI.

Mirrors the seven names the reference package exports
(aq_kernels/__init__.py:1-23 of the LAPrune tree) with the same positional
and keyword signatures, argument meaning and ``RuntimeError`` on invalid
input.  As in the reference, every name is ``None`` when the native library
cannot be loaded, so callers written against the reference keep their
``is not None`` gating; code in this package that *needs* the kernels calls
``laprune_amd._native.lib()`` and fails loudly instead.

Differences from the reference (all supersets):
  * K/V gathers accept bf16 as well as fp16;
  * launch-tuning arguments (``threads``, ``vector_width``, ``grid_y_cap``) are
    validated as in the reference and otherwise ignored;
  * ``fused_linear_encode_forward`` follows the fp32 greedy contract of
    laprune/quantizer.py:346-355 on ``codebooks`` (``weight_t`` and ``bias``,
    which the reference derives from the same codebooks, are shape-checked).
New names: ``aq_lut_build``, ``aq_topk``, ``aq_retrieve_topk``,
``sparse_attn_decode``, ``dense_attn_decode``, ``aq_encode_prepare``,
``aq_encode_greedy``.
"""
from __future__ import annotations

from . import _impl

try:
    _impl.N.lib()
    _OK = True
except Exception:  # the reference's contract: names become None
    _OK = False

if _OK:
    aq_lut_forward = _impl.aq_lut_forward
    aq_lut_gather_forward = _impl.aq_lut_gather_forward
    fused_linear_encode_forward = _impl.fused_linear_encode_forward
    aq_lut_gather_gqa = _impl.aq_lut_gather
    aq_lut_gather_grouped = _impl.aq_lut_gather_grouped
    gqa_gather_kv = _impl.gqa_gather_kv
    gqa_gather_kv_with_tail = _impl.gqa_gather_kv_with_tail
    # superset
    aq_lut_build = _impl.aq_lut_build
    aq_topk = _impl.aq_topk
    aq_retrieve_topk = _impl.aq_retrieve_topk
    sparse_attn_decode = _impl.sparse_attn_decode
    dense_attn_decode = _impl.dense_attn_decode
    aq_encode_prepare = _impl.aq_encode_prepare
    aq_encode_greedy = _impl.aq_encode_greedy
else:
    aq_lut_forward = None
    aq_lut_gather_forward = None
    fused_linear_encode_forward = None
    aq_lut_gather_gqa = None
    aq_lut_gather_grouped = None
    gqa_gather_kv = None
    gqa_gather_kv_with_tail = None
    aq_lut_build = None
    aq_topk = None
    aq_retrieve_topk = None
    sparse_attn_decode = None
    dense_attn_decode = None
    aq_encode_prepare = None
    aq_encode_greedy = None

REFERENCE_NAMES = (
    "aq_lut_forward",
    "aq_lut_gather_forward",
    "fused_linear_encode_forward",
    "aq_lut_gather_gqa",
    "aq_lut_gather_grouped",
    "gqa_gather_kv",
    "gqa_gather_kv_with_tail",
)
