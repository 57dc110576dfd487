"""Scores round to fp32 at every add and then to fp16, as the contract says
(acc += (float)lut[m][code_m]; score = fp16_rne(acc)), also where a fused
rounding would differ.

The table is built so that a token's exact sum lies just above an fp16
midpoint while its fp32 sum lands on the midpoint:

  type X: 1 + 2^-11 (exact in fp32), then + 2^-24: the fp32 add ties to
          even and stays at 1 + 2^-11, the midpoint of 1 and 1 + 2^-10,
          whose fp16 rounding ties to even: 1.0 (0x3C00).  Rounding the exact
          sum once (v_fma_mixlo_f16) gives 1 + 2^-10 (0x3C01) instead.
  type Y: 1 + 2^-10 exactly (0x3C01).
  other:  0.5.

With k = the number of Y tokens and the X tokens at lower columns, the
contract selects every Y token; a single rounding would make X and Y tie and
the lower-column X tokens win.  Keys are fp16 (bf16 keys would merge the two
values).  Checked through the fused scorer's fp16 scores and selection
(group and per-head keys) and through the one-launch decode step (group and
per-head selection), against the oracle."""
import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

HKV, G, M, K, D = 8, 4, 32, 256, 128
T = 8192
X_COLS = np.arange(100, 600)
Y_COLS = np.arange(4000, 4500)
NK = len(Y_COLS)


def _f16_bits(x):
    return int(np.array(x, dtype=np.float16).view(np.uint16))


def _inputs():
    lut = np.zeros((HKV, M, K, G), dtype=np.uint16)  # GMKG, fp16 bits
    lut[:, 0, 0, :] = _f16_bits(0.5)
    lut[:, 0, 1, :] = _f16_bits(1.0)
    lut[:, 0, 2, :] = _f16_bits(1.0)
    lut[:, 1, 1, :] = _f16_bits(2.0 ** -11)
    lut[:, 1, 2, :] = _f16_bits(2.0 ** -10)
    lut[:, 31, 1, :] = _f16_bits(2.0 ** -24)  # the smallest fp16 subnormal
    codes = np.zeros((1, HKV, T, M), dtype=np.uint8)
    codes[0, :, X_COLS, 0] = 1
    codes[0, :, X_COLS, 1] = 1
    codes[0, :, X_COLS, 31] = 1
    codes[0, :, Y_COLS, 0] = 2
    codes[0, :, Y_COLS, 1] = 2
    return lut, codes


def _oracle(orc, lut, codes):
    lut_hmk = np.ascontiguousarray(lut.transpose(0, 3, 1, 2).reshape(HKV * G, M, K))
    want_s = orc.score_grouped(lut_hmk, codes[0], G)
    assert (want_s[:, X_COLS] == 0x3C00).all() and (want_s[:, Y_COLS] == 0x3C01).all()
    return want_s


@pytest.mark.parametrize("per_head", [False, True])
def test_scorer_rounds_to_fp32_then_fp16(dev, orc, per_head):
    from laprune_amd import aq_kernels as AK
    lut, codes = _inputs()
    want_s = _oracle(orc, lut, codes)
    cs, ce = orc.candidate_window(T, T, 4, 64)
    lut_d = torch.from_numpy(lut.view(np.int16)).to(dev).view(torch.float16)
    codes_d = torch.from_numpy(codes).to(dev)
    print(f"crafted scorer, per_head={per_head}", flush=True)
    idx, scores = AK.aq_retrieve_topk(lut_d, codes_d, NK, cs, ce, key_dtype=torch.float16,
                                      return_scores=True, per_head=per_head)
    torch.cuda.synchronize()
    got_s = scores[0].cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got_s, want_s)
    want_i = orc.topk(want_s, NK, group=1 if per_head else G, cand_start=cs, cand_end=ce)
    assert np.array_equal(idx[0].cpu().numpy().astype(np.int64), want_i)
    assert (want_i == Y_COLS[None, :]).all()


@pytest.mark.parametrize("select", ["group", "head"])
def test_step_rounds_to_fp32_then_fp16(dev, orc, select):
    from laprune_amd import _native as N
    lut, codes = _inputs()
    want_s = _oracle(orc, lut, codes)
    cs, ce = orc.candidate_window(T, T, 4, 64)
    want_i = orc.topk(want_s, NK, group=G if select == "group" else 1, cand_start=cs,
                      cand_end=ce)
    assert (want_i == Y_COLS[None, :]).all()
    g = torch.Generator().manual_seed(5)
    B, HQ = 1, HKV * G
    lut_d = torch.from_numpy(lut.view(np.int16)).to(dev)
    codes_d = torch.from_numpy(codes).to(dev)
    q = torch.randn(B, HQ, D, generator=g).bfloat16().to(dev)
    kc = torch.randn(B, HKV, T, D, generator=g).bfloat16().to(dev)
    vc = torch.randn(B, HKV, T, D, generator=g).bfloat16().to(dev)
    key_mode = N.KEY_F16 | (N.SELECT_PER_HEAD if select == "head" else 0)
    rows = HQ if select == "head" else HKV
    sink, tail_start, tail_count = 4, T - 64, 64
    keep_max = NK + sink + tail_count
    ws_bytes = N.size_query("lap_decode_step_workspace_size", B, HQ, HKV, T, D, keep_max,
                            key_mode)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
    idx = torch.full((B, rows, NK), -3, dtype=torch.int32, device=dev)
    out = torch.empty(B, HQ, D, dtype=torch.bfloat16, device=dev)
    print(f"crafted one-launch step, select={select}", flush=True)
    N.call("lap_decode_step", N.ptr(lut_d), N.ptr(codes_d), codes_d.stride(0),
           codes_d.stride(1), codes_d.stride(2), T, cs, ce, NK, sink, tail_start, tail_count,
           None, 0, 0, 0, key_mode, N.ptr(q), q.stride(0), q.stride(1), N.ptr(kc), N.ptr(vc),
           N.dtype_code(q.dtype), B, HQ, HKV, T, D, kc.stride(0), kc.stride(1), kc.stride(2),
           vc.stride(0), vc.stride(1), vc.stride(2), 1.0 / math.sqrt(D), N.ptr(idx), N.I32,
           N.ptr(out), N.ptr(ws), ws.numel(), N.stream_of(q))
    torch.cuda.synchronize()
    assert np.array_equal(idx[0].cpu().numpy().astype(np.int64), want_i)
    assert torch.isfinite(out.float()).all()
