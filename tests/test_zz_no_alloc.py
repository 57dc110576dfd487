"""lap_decode_step_noalloc (the decode step on the library's static scratch)
against lap_decode_step on a caller workspace.

Both entry points run the same kernels, so indices and attention outputs
must be identical bit for bit.  Calls in a row shrink the input: the C2
shape (one launch, 32 workgroups per KV row), then a shorter partial row,
then ragged device plans over B = 2 (fewer workgroups per row, more rows),
then per-head selection at 8192 columns (the one-launch per-head kernel),
then head_dim 64, which only the kernel chain serves (the scratch past the
persistent head: the retrieve and attention workspaces).  After every call
the scratch's health counters (lap_decode_step_noalloc_status) are zero.
Shapes beyond the scratch are refused before any launch.
"""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu

Hq, Hkv, D = 32, 8, 128


def _inputs(seed, B, T, dev, D=D):
    g = torch.Generator().manual_seed(seed)
    cb = torch.randn(32, 256, D, generator=g) * 0.02
    codes = torch.randint(0, 256, (B, Hkv, T, 32), generator=g, dtype=torch.uint8).to(dev)
    q = torch.randn(B, Hq, 1, D, generator=g).bfloat16().to(dev)
    gd = torch.Generator(device=dev).manual_seed(seed + 1)
    kk = torch.randn((B, Hkv, T, D), generator=gd, device=dev).bfloat16()
    vv = torch.randn((B, Hkv, T, D), generator=gd, device=dev).bfloat16()
    return cb.to(dev), codes, kk, vv, q


def _decoder(cb, B, T, topk, select="group"):
    from laprune_amd.retrieval import RetrievalConfig, SparseDecoder
    cfg = RetrievalConfig(topk=topk, sink_size=4, local_window=64, select=select,
                          score_dtype=torch.bfloat16)
    return SparseDecoder(cb, B, Hq, Hkv, cb.shape[2], T, cfg, dtype=torch.bfloat16)


def _scratch_status():
    from laprune_amd import _native as N
    a, b = N.u32(), N.u32()
    N.call("lap_decode_step_noalloc_status", N.byref(a), N.byref(b))
    return int(a.value), int(b.value)


def _noalloc(dec, q, codes, kk, vv, T, T_kv, p, plans=None, k_cols=0, max_sink=0, max_tail=0):
    from laprune_amd import _native as N
    idx = torch.full_like(dec.idx, -7)
    out = torch.zeros_like(dec.out)
    q = q[:, :, 0, :]
    if p is None:
        p = dict(cand_start=0, cand_end=0, k=0, sink=0, tail_start=0, tail_count=0)
    N.call("lap_decode_step_noalloc", N.ptr(dec.lut), N.ptr(codes), codes.stride(0),
           codes.stride(1), codes.stride(2), T, p["cand_start"], p["cand_end"], p["k"],
           p["sink"], p["tail_start"], p["tail_count"], N.ptr(plans), k_cols, max_sink, max_tail,
           dec.key_mode, N.ptr(q), q.stride(0), q.stride(1), N.ptr(kk), N.ptr(vv),
           N.dtype_code(q.dtype), dec.B, Hq, Hkv, T_kv, dec.D, kk.stride(0), kk.stride(1),
           kk.stride(2), vv.stride(0), vv.stride(1), vv.stride(2), 1.0 / math.sqrt(dec.D),
           N.ptr(idx), N.I32, N.ptr(out), N.stream_of(q))
    torch.cuda.synchronize()
    assert _scratch_status() == (0, 0)
    return idx, out


def _uniform(dev, seed, B, T, tc, topk, select="group", D=D):
    cb, codes, kk, vv, q = _inputs(seed, B, T, dev, D)
    dec = _decoder(cb, B, T, topk, select)
    want = dec.step(q, codes[:, :, :tc], kk, vv, t_codes=tc, t_total=T)
    torch.cuda.synchronize()
    want_idx, want_out = dec.selected().clone(), want[:, :, 0].clone()
    n = want_idx.numel()  # uniform steps write [B][rows][k] densely
    p = dec.plan(tc, T)
    idx, out = _noalloc(dec, q, codes[:, :, :tc], kk, vv, tc, T, p)
    assert torch.equal(idx.view(-1)[:n], want_idx.view(-1))
    assert torch.equal(out, want_out)
    assert dec.fused_status() == (0, 0)


def test_noalloc_matches_workspace_step_shrinking(dev):
    print("noalloc: C2 131072, top-2048", flush=True)
    _uniform(dev, 900, 1, 131072, 131072, 2048)
    print("noalloc: 40003 (39936 encoded), top-700", flush=True)
    _uniform(dev, 901, 1, 40003, 39936, 700)
    print("noalloc: ragged B=2", flush=True)
    from laprune_amd.retrieval import PLAN_FIELDS
    B, T = 2, 16384
    cb, codes, kk, vv, q = _inputs(902, B, T, dev)
    dec = _decoder(cb, B, T, 512)
    t_total = [16384, 9001]
    t_codes = [t - t % 64 for t in t_total]
    dec.step(q, codes, kk, vv, t_codes=t_codes, t_total=t_total)
    torch.cuda.synchronize()
    want_idx, want_out = dec.idx.clone(), dec.out.clone()
    plans = dec.row_plans(t_codes, t_total)
    pdev = torch.tensor([[pl[f] for f in PLAN_FIELDS] for pl in plans], dtype=torch.int32,
                        device=dev)
    k_cols = max(pl["k"] for pl in plans)
    idx, out = _noalloc(dec, q, codes, kk, vv, max(t_codes), kk.shape[2], None, pdev, k_cols,
                        max(pl["sink"] for pl in plans), max(pl["tail_count"] for pl in plans))
    assert torch.equal(idx[..., :k_cols], want_idx[..., :k_cols])
    assert torch.equal(out, want_out)
    print("noalloc: per-head selection 8192 (one-launch per-head kernel)", flush=True)
    _uniform(dev, 903, 1, 8192, 8192, None, select="head")
    print("noalloc: head_dim 64, 8192 (kernel chain)", flush=True)
    _uniform(dev, 905, 1, 8192, 8192, 512, D=64)
    print("noalloc: head_dim 64, per-head selection 4096 (kernel chain)", flush=True)
    _uniform(dev, 906, 1, 4096, 4096, None, select="head", D=64)


def test_noalloc_refuses_oversized_shapes(dev):
    from laprune_amd import _native as N
    cb, codes, kk, vv, q = _inputs(904, 1, 256, dev)
    dec = _decoder(cb, 1, 256, 16)
    dec.step(q, codes, kk, vv)
    torch.cuda.synchronize()
    # more KV rows than the scratch's persistent head serves
    with pytest.raises(N.NativeError) as e:
        N.call("lap_decode_step_noalloc", N.ptr(dec.lut), N.ptr(codes), 0, 0, 32, 256, 0, 192,
               16, 4, 192, 64, None, 0, 0, 0, dec.key_mode, N.ptr(q), 0, D, N.ptr(kk),
               N.ptr(vv), N.BF16, 33, Hq, Hkv, 256, D, 0, 0, D, 0, 0, D, 0.088,
               N.ptr(dec.idx), N.I32, N.ptr(dec.out), N.stream_of(q))
    assert e.value.status == N.LAP_ERR_WORKSPACE and "static scratch" in str(e.value)
    # a kernel-chain shape whose buffers exceed the 64 MiB scratch
    # (B = 32 per-head rows at T = 65536: about 140 MB of score rows)
    with pytest.raises(N.NativeError) as e:
        N.call("lap_decode_step_noalloc", N.ptr(dec.lut), N.ptr(codes), 0, 0, 32, 65536, 4,
               65472, 16, 4, 65472, 64, None, 0, 0, 0, dec.key_mode | N.SELECT_PER_HEAD,
               N.ptr(q), 0, D, N.ptr(kk), N.ptr(vv), N.BF16, 32, Hq, Hkv, 65536, D, 0, 0, D,
               0, 0, D, 0.088, N.ptr(dec.idx), N.I32, N.ptr(dec.out), N.stream_of(q))
    assert e.value.status == N.LAP_ERR_WORKSPACE and "static scratch" in str(e.value)
