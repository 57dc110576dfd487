"""On-disk AQ codebooks: one torch-zip file per layer and head group.

Format (written by the reference's training/train_llama31_codebooks.py:
345-362, read by AQLayerCodebookManager.load, laprune/llm/aq_kv.py:277-342):
``layer_{L}_group_{G}.pt`` holds a dict with ints ``M``, ``K``, ``d`` and a
float32 tensor ``codebooks`` of shape [M, K, d], plus optional entries
(``metadata`` dict, ``d_sub``, ``method``) that are carried along unread.

Files are read with ``torch.load(..., weights_only=True)``, which executes
nothing from the file; a file that loader refuses is reported, not opened
another way.  The directory rules follow the reference loader: names that do
not parse as ``layer_{int}_group_{int}`` are ignored, and when the head
grouping is known (``num_heads`` / ``heads_per_group``) group files the
grouping cannot use are skipped.
"""
from __future__ import annotations

import os
import re
from dataclasses import dataclass, field

import torch

_NAME = re.compile(r"^layer_(\d+)_group_(\d+)\.pt$")


@dataclass
class LayerCodebook:
    """Codebooks of one (layer, group): [M, K, d] float32 plus the stored extras."""

    layer: int
    group: int
    M: int
    K: int
    d: int
    codebooks: torch.Tensor
    extras: dict = field(default_factory=dict)


def parse_name(fname: str) -> tuple[int, int] | None:
    """(layer, group) of ``layer_{L}_group_{G}.pt``, else None."""
    m = _NAME.match(fname)
    return (int(m.group(1)), int(m.group(2))) if m else None


def load_file(path: str, device: torch.device | str | None = None,
              dtype: torch.dtype = torch.float32) -> LayerCodebook:
    """Read and check one codebook file."""
    try:
        ck = torch.load(path, map_location="cpu", weights_only=True)
    except Exception as e:  # the safe loader refused the file
        raise RuntimeError(f"{path}: not readable with torch.load(weights_only=True): {e}") from e
    if not isinstance(ck, dict):
        raise RuntimeError(f"{path}: expected a dict, found {type(ck).__name__}")
    for key in ("M", "K", "d", "codebooks"):
        if key not in ck:
            raise RuntimeError(f"{path}: missing '{key}'")
    M, K, d = int(ck["M"]), int(ck["K"]), int(ck["d"])
    cb = ck["codebooks"]
    if not torch.is_tensor(cb) or tuple(cb.shape) != (M, K, d):
        shape = tuple(cb.shape) if torch.is_tensor(cb) else type(cb).__name__
        raise RuntimeError(f"{path}: codebooks {shape} do not match M={M}, K={K}, d={d}")
    if not cb.is_floating_point():
        raise RuntimeError(f"{path}: codebooks must be floating point, found {cb.dtype}")
    if K > 256:
        raise RuntimeError(f"{path}: K={K} does not fit uint8 codes")
    parsed = parse_name(os.path.basename(path)) or (-1, -1)
    extras = {k: v for k, v in ck.items() if k not in ("M", "K", "d", "codebooks")}
    cb = cb.to(dtype=dtype).contiguous()
    if device is not None:
        cb = cb.to(device)
    return LayerCodebook(parsed[0], parsed[1], M, K, d, cb, extras)


def load_dir(save_dir: str, layers=None, num_heads: int | None = None,
             heads_per_group: int | None = None, device=None,
             dtype: torch.dtype = torch.float32) -> dict[tuple[int, int], LayerCodebook]:
    """All usable codebook files of a directory, keyed by (layer, group).

    ``layers`` (an iterable of layer indices) restricts the set; with
    ``num_heads`` and ``heads_per_group`` given, groups at or past
    num_heads // heads_per_group are skipped as stale (aq_kv.py:300-307)."""
    if not os.path.isdir(save_dir):
        raise FileNotFoundError(save_dir)
    want = None if layers is None else set(int(x) for x in layers)
    max_groups = None
    if num_heads is not None and heads_per_group:
        max_groups = int(num_heads) // int(heads_per_group)
    out = {}
    for fname in sorted(os.listdir(save_dir)):
        lg = parse_name(fname)
        if lg is None:
            continue
        layer, group = lg
        if want is not None and layer not in want:
            continue
        if max_groups is not None and max_groups > 0 and group >= max_groups:
            continue
        out[lg] = load_file(os.path.join(save_dir, fname), device=device, dtype=dtype)
    return out


def save_file(path: str, codebooks: torch.Tensor, metadata: dict | None = None) -> None:
    """Write one file in the reference's format (training writer, :345-362)."""
    if codebooks.dim() != 3:
        raise RuntimeError("codebooks must be [M, K, d]")
    M, K, d = (int(x) for x in codebooks.shape)
    payload = {"M": M, "K": K, "d": d,
               "codebooks": codebooks.detach().to("cpu", torch.float32).contiguous()}
    if metadata is not None:
        payload["metadata"] = metadata
    torch.save(payload, path)
