"""Codebook manager: the serving surface of the reference's
``AQLayerCodebookManager`` (laprune/llm/aq_kv.py:79-699) on the gfx950 kernels.

* ``approx_inner_product_multihead_gqa`` (:633-699), the decode scorer that
  ``_decode_attention`` calls (aq_evaluation.py:165): the fp16 LUT from
  ``lap_lut_build`` (fp32 fmaf chain over d, RNE to fp16) summed by the
  grouped scorer (``lap_lut_score_grouped``, sequential fp32 over m, fp16
  out) for G <= 4, or by the per-head GQA scorer for larger groups.
* ``approx_inner_product_multihead`` (:519-630): per-head codes, the same LUT
  summed by the MHA scorer; ``approx_inner_product`` (:459-520) is its
  one-query form with the head's group codebooks.
* ``reconstruct`` (:431-457): approximate keys from codes
  (``lap_aq_reconstruct``, fp32 sum over m in the reference's order).
* ``encode_keys`` / ``encode_keys_batch`` (:347-428): the greedy fp32 encode
  (``lap_encode_greedy``), which is the reference's decode setting
  (``aq_encode_icm_iters_decode`` = 0, aq_evaluation.py:383-396).
* ``load`` / ``save`` (:243-342): the torch-zip files of
  ``laprune_amd.codebooks`` (read with ``weights_only=True``).

ICM refinement (``icm_iters > 0``) and codebook training (``fit_layer``) are
the reference's offline paths; they raise ``NotImplementedError`` here.
Everything served runs on the GPU and fails loudly without the HIP library.
"""
from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import torch

from . import _native as N
from . import codebooks as cbio


@dataclass
class AQLayerConfig:
    """Codebook shape of one layer (aq_kv.py:79-93): M sub-codebooks of K
    entries of dimension d, shared by ``heads_per_group`` heads."""

    M: int
    K: int
    d: int
    heads_per_group: int = 2
    num_heads: Optional[int] = None


class AQLayerCodebookManager:
    """Per-(layer, head-group) codebooks and the LUT scoring / greedy encode
    that serve decode (aq_kv.py:96-125)."""

    def __init__(self, layer_cfgs: Dict[int, AQLayerConfig],
                 device: Optional[torch.device] = None, dtype: torch.dtype = torch.float32):
        self.layer_cfgs = dict(layer_cfgs)
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.dtype = dtype
        self._cb: Dict[Tuple[int, int], torch.Tensor] = {}
        self._prep: Dict[Tuple[int, int], torch.Tensor] = {}

    # ------------------------------------------------------------ storage
    def set_codebooks(self, layer_idx: int, group_idx: int, codebooks: torch.Tensor) -> None:
        """Install [M, K, d] codebooks for (layer, group) (fp32 on the device)."""
        cfg = self.layer_cfgs[layer_idx]
        if codebooks.dim() != 3 or tuple(codebooks.shape) != (cfg.M, cfg.K, cfg.d):
            raise ValueError(f"codebooks {tuple(codebooks.shape)} do not match layer {layer_idx}'s "
                             f"config ({cfg.M}, {cfg.K}, {cfg.d})")
        self._cb[(layer_idx, group_idx)] = codebooks.to(self.device, torch.float32).contiguous()
        self._prep.pop((layer_idx, group_idx), None)

    def codebooks(self, layer_idx: int, group_idx: int = 0) -> torch.Tensor:
        try:
            return self._cb[(layer_idx, group_idx)]
        except KeyError:
            raise KeyError(f"no codebooks for layer {layer_idx}, group {group_idx}") from None

    def load(self, save_dir: str) -> None:
        """Read ``layer_{L}_group_{G}.pt`` files for the configured layers
        (aq_kv.py:277-342): unparsable names and unconfigured layers are
        ignored, group files the layer's grouping cannot use are skipped,
        and a file's M/K/d replace the layer's configured shape."""
        if not os.path.isdir(save_dir):
            raise FileNotFoundError(save_dir)
        found = cbio.load_dir(save_dir, layers=list(self.layer_cfgs))
        for (layer, group), lc in found.items():
            cfg = self.layer_cfgs[layer]
            if cfg.num_heads is not None and cfg.heads_per_group > 0:
                expected = int(cfg.num_heads) // int(cfg.heads_per_group)
                if expected > 0 and group >= expected:
                    continue
            if (cfg.M, cfg.K, cfg.d) != (lc.M, lc.K, lc.d):
                self.layer_cfgs[layer] = AQLayerConfig(M=lc.M, K=lc.K, d=lc.d,
                                                       heads_per_group=cfg.heads_per_group,
                                                       num_heads=cfg.num_heads)
            self.set_codebooks(layer, group, lc.codebooks)

    def save(self, save_dir: str) -> None:
        """Write every installed (layer, group) in the reference's format."""
        os.makedirs(save_dir, exist_ok=True)
        for (layer, group), cb in sorted(self._cb.items()):
            cbio.save_file(os.path.join(save_dir, f"layer_{layer}_group_{group}.pt"), cb)

    # ------------------------------------------------------------ encode
    def _prepared(self, layer_idx: int, group_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        key = (layer_idx, group_idx)
        cb = self.codebooks(layer_idx, group_idx)
        prep = self._prep.get(key)
        if prep is None:
            from .aq_kernels import _impl
            prep = _impl.aq_encode_prepare(cb)
            self._prep[key] = prep
        return cb, prep

    @torch.no_grad()
    def encode_keys_batch(self, layer_idx: int, group_idx: int, keys: torch.Tensor,
                          batch_size: int = 3_000_000, icm_iters: int = 2) -> torch.Tensor:
        """uint8 codes [N, M] of keys [N, d] for one (layer, group)
        (aq_kv.py:389-428; greedy, first index on ties)."""
        if icm_iters != 0:
            raise NotImplementedError("ICM refinement (icm_iters > 0) is an offline path; "
                                      "decode encodes greedily (icm_iters=0)")
        if batch_size <= 0:
            raise ValueError("batch_size must be positive")
        from .aq_kernels import _impl
        cb, prep = self._prepared(layer_idx, group_idx)
        x = keys.to(self.device)
        if x.dim() != 2 or x.shape[1] != cb.shape[2]:
            raise ValueError(f"keys must be [N, {cb.shape[2]}], got {tuple(keys.shape)}")
        codes, _ = _impl.aq_encode_greedy(x, cb, prep)
        return codes

    @torch.no_grad()
    def encode_keys(self, layer_idx: int, head_idx: int, keys: torch.Tensor,
                    batch_size: int = 3_000_000, icm_iters: int = 2) -> torch.Tensor:
        """Codes of one head's keys: its group's codebooks (aq_kv.py:347-387)."""
        cfg = self.layer_cfgs[layer_idx]
        return self.encode_keys_batch(layer_idx, head_idx // cfg.heads_per_group, keys,
                                      batch_size, icm_iters)

    # ------------------------------------------------------------ scoring
    def _lut(self, layer_idx: int, q: torch.Tensor, m_codes: int) -> torch.Tensor:
        from .aq_kernels import _impl
        cb = self.codebooks(layer_idx, 0)
        M, K, d = cb.shape
        if q.dim() == 1:
            q = q[None, :]
        q = q.to(self.device)
        if q.dim() != 2 or q.shape[1] != d or m_codes != M:
            raise ValueError(f"AQ shape mismatch: codebook={tuple(cb.shape)}, q={tuple(q.shape)}, "
                             f"codes M={m_codes}")
        if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            q = q.float()
        return _impl.aq_lut_build(q.contiguous(), cb, 1, "hmk")

    @torch.no_grad()
    def approx_inner_product_multihead_gqa(self, layer_idx: int, q: torch.Tensor,
                                           codes: torch.Tensor, num_kv_group: int,
                                           scoring_m: int = 32) -> torch.Tensor:
        """fp16 scores [B*Hq, N] of q [B*Hq, d] against codes [B*Hkv, N, M]
        without expanding the codes to query heads (aq_kv.py:633-699)."""
        from .aq_kernels import _impl
        q2 = q[None, :] if q.dim() == 1 else q
        if codes.dim() != 3:
            raise ValueError(f"codes must be [B*Hkv, N, M], got {tuple(codes.shape)}")
        kv_heads, n_tokens, m_codes = codes.shape
        group = int(num_kv_group)
        if q2.shape[0] != kv_heads * group:
            raise ValueError(f"Invalid GQA score heads: Hq={q2.shape[0]}, Hkv={kv_heads}, "
                             f"G={group}")
        if int(scoring_m) != 32:
            raise ValueError(f"aq_scoring_m must be 32, got {scoring_m}")
        N.require_cuda(codes)
        if codes.dtype != torch.uint8:
            raise ValueError("codes must be uint8")
        lut = self._lut(layer_idx, q2, m_codes)
        if codes.stride(2) != 1:
            codes = codes.contiguous()
        if group <= 4:
            return _impl.aq_lut_gather_grouped(lut, codes, group)
        return _impl.aq_lut_gather(lut, codes, group, 0, m_codes, None)

    @torch.no_grad()
    def approx_inner_product_multihead(self, layer_idx: int, q: torch.Tensor,
                                       codes: torch.Tensor) -> torch.Tensor:
        """Scores [Q, N] of q [Q, d] against per-query codes [Q, N, M]
        (aq_kv.py:519-630); fp16 out."""
        from .aq_kernels import _impl
        if codes.dim() != 3:
            raise ValueError(f"codes must be [Q, N, M], got {tuple(codes.shape)}")
        N.require_cuda(codes)
        lut = self._lut(layer_idx, q, codes.shape[2])
        Q, M, K = lut.shape
        return _impl.aq_lut_gather_forward(lut.reshape(Q, M * K), codes.contiguous())

    @torch.no_grad()
    def reconstruct(self, layer_idx: int, head_idx: int, codes: torch.Tensor) -> torch.Tensor:
        """Approximate keys [N, d] from codes [N, M] with the head's group
        codebooks (aq_kv.py:431-457): fp32, the sum over m ascending of
        C_m[codes[:, m]], as the reference's loop adds them."""
        from .aq_kernels import _impl
        cfg = self.layer_cfgs[layer_idx]
        cb = self.codebooks(layer_idx, head_idx // cfg.heads_per_group)
        codes = codes.to(cb.device)
        if codes.dim() != 2 or codes.shape[1] != cb.shape[0]:
            raise ValueError(f"codes must be [N, {cb.shape[0]}], got {tuple(codes.shape)}")
        return _impl.aq_reconstruct(cb, codes)

    @torch.no_grad()
    def approx_inner_product(self, layer_idx: int, head_idx: int, q: torch.Tensor,
                             codes: torch.Tensor) -> torch.Tensor:
        """Scores [N] of one query q ([d] or [1, d]) against codes [N, M] with
        the head's group codebooks (aq_kv.py:459-520): the LUT q . C_m[k] and
        its gather-sum over m, under this path's contract (fp16 LUT from an
        fp32 fmaf chain over d, sequential fp32 sum over m, fp16 out; the
        reference sums an fp32 LUT in torch's order in the manager's dtype)."""
        from .aq_kernels import _impl
        cfg = self.layer_cfgs[layer_idx]
        cb = self.codebooks(layer_idx, head_idx // cfg.heads_per_group)
        if q.dim() == 2:
            if q.shape[0] != 1:
                raise ValueError(f"q must be [d] or [1, d], got {tuple(q.shape)}")
            q = q[0]
        M, K, d = cb.shape
        if q.dim() != 1 or q.shape[0] != d:
            raise ValueError(f"q must have {d} elements, got {tuple(q.shape)}")
        codes = codes.to(cb.device)
        if codes.dim() != 2 or codes.shape[1] != M:
            raise ValueError(f"codes must be [N, {M}], got {tuple(codes.shape)}")
        N.require_cuda(codes)
        qv = q.to(cb.device)
        if qv.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            qv = qv.float()
        lut = _impl.aq_lut_build(qv[None, :].contiguous(), cb, 1, "hmk")  # fp16 [1, M, K]
        return _impl.aq_lut_gather_forward(lut.reshape(1, M * K), codes[None].contiguous())[0]

    def fit_layer(self, *args, **kwargs):
        raise NotImplementedError("codebook training is an offline path (the reference's "
                                  "training/ scripts); load trained codebooks with load()")
