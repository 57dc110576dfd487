"""One lap_decode_step workspace shared by calls of different batch sizes.

The workspace's persistent head (status words, row barriers, row
histograms) has a call-independent layout, so a workspace sized for B = 2
serves a B = 1 call and then B = 2 again.  Each call must equal, bit for
bit, the same call on a fresh workspace, and the health counters must stay
zero.  Without the fixed layout the B = 1 call reads row 1's barrier words
as row 0's histogram and selects the wrong keys.
"""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu

Hq, Hkv, D = 32, 8, 128


def _inputs(seed, B, T, dev):
    g = torch.Generator().manual_seed(seed)
    cb = torch.randn(32, 256, D, generator=g) * 0.02
    codes = torch.randint(0, 256, (B, Hkv, T, 32), generator=g, dtype=torch.uint8).to(dev)
    q = torch.randn(B, Hq, 1, D, generator=g).bfloat16().to(dev)
    gd = torch.Generator(device=dev).manual_seed(seed + 1)
    kk = torch.randn((B, Hkv, T, D), generator=gd, device=dev).bfloat16()
    vv = torch.randn((B, Hkv, T, D), generator=gd, device=dev).bfloat16()
    return cb.to(dev), codes, kk, vv, q


def _decoder(cb, B, T, select):
    from laprune_amd.retrieval import RetrievalConfig, SparseDecoder
    cfg = RetrievalConfig(topk=1024, sink_size=4, local_window=64, select=select,
                          score_dtype=torch.bfloat16)
    return SparseDecoder(cb, B, Hq, Hkv, D, T, cfg, dtype=torch.bfloat16)


def _step_on(ws, dec, q, codes, kk, vv):
    """lap_decode_step of dec's shape and LUT (built by dec.step) on `ws`."""
    from laprune_amd import _native as N
    T = codes.shape[2]
    p = dec.plan(T, T)
    idx = torch.full_like(dec.idx, -7)
    out = torch.zeros_like(dec.out)
    q3 = q[:, :, 0, :]
    N.call("lap_decode_step", N.ptr(dec.lut), N.ptr(codes), codes.stride(0), codes.stride(1),
           codes.stride(2), T, p["cand_start"], p["cand_end"], p["k"], p["sink"],
           p["tail_start"], p["tail_count"], None, 0, 0, 0, dec.key_mode, N.ptr(q3),
           q3.stride(0), q3.stride(1), N.ptr(kk), N.ptr(vv), N.BF16, dec.B, Hq, Hkv, T, D,
           kk.stride(0), kk.stride(1), kk.stride(2), vv.stride(0), vv.stride(1), vv.stride(2),
           1.0 / math.sqrt(D), N.ptr(idx), N.I32, N.ptr(out), ws.data_ptr(), ws.numel(),
           N.stream_of(q3))
    torch.cuda.synchronize()
    return idx, out


@pytest.mark.parametrize("select", ["group", "head"])
def test_workspace_serves_smaller_batch(dev, select):
    T = 32768
    print(f"workspace reuse: B=2 then B=1 then B=2, {select} selection", flush=True)
    cb, codes2, kk2, vv2, q2 = _inputs(300, 2, T, dev)
    dec2 = _decoder(cb, 2, T, select)
    dec1 = _decoder(cb, 1, T, select)
    want2 = dec2.step(q2, codes2, kk2, vv2)[:, :, 0].clone()
    want2_idx = dec2.selected().clone()
    # a B = 1 step on the B = 2 workspace against a fresh B = 1 workspace
    q1, codes1, kk1, vv1 = q2[1:2], codes2[1:2], kk2[1:2], vv2[1:2]
    want1 = dec1.step(q1, codes1, kk1, vv1)[:, :, 0].clone()
    want1_idx = dec1.selected().clone()
    assert dec2.ws.numel() >= dec1.ws.numel()
    got1_idx, got1 = _step_on(dec2.ws, dec1, q1, codes1, kk1, vv1)
    n1 = want1_idx.numel()
    assert torch.equal(got1_idx.view(-1)[:n1], want1_idx.view(-1))
    assert torch.equal(got1, want1)
    # B = 2 again on the shared workspace, against its first (fresh) call
    again = dec2.step(q2, codes2, kk2, vv2)[:, :, 0]
    assert torch.equal(dec2.selected(), want2_idx)
    assert torch.equal(again, want2)
    assert dec2.fused_status() == (0, 0) and dec1.fused_status() == (0, 0)
