"""GPU parity of every kernel against the CPU oracle (bit-exact unless stated).

All calls go through the C ABI (via the torch-facing wrappers of
laprune_amd.aq_kernels, which only marshal pointers).  Inputs are seeded.
"""
import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _np_u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.fixture(scope="module")
def K(dev):
    from laprune_amd import aq_kernels as K
    for name in K.REFERENCE_NAMES:
        assert getattr(K, name) is not None, name
    return K


# ------------------------------------------------------------------ A1 LUT

@pytest.fixture(params=["mfma", "dpp"])
def lut_impl(request, monkeypatch):
    """The LUT builder's two forms for D = 64 and 128: fp32 MFMA (default) and
    DPP-broadcast VALU (LAPRUNE_LUT_IMPL=dpp, read at every call)."""
    monkeypatch.setenv("LAPRUNE_LUT_IMPL", request.param)
    return request.param


@pytest.mark.parametrize("qdt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("layout", ["hmk", "gmkg"])
def test_lut_build_bit_exact(dev, K, orc, qdt, layout, lut_impl):
    g = _gen(1)
    q = torch.randn(32, 128, generator=g).to(qdt)
    cb = torch.randn(32, 256, 128, generator=g) * 0.02
    lut = K.aq_lut_build(q.to(dev), cb.to(dev), G=4, layout=layout)
    torch.cuda.synchronize()
    want = orc.lut_build(q.float().numpy(), cb.numpy())
    if layout == "gmkg":
        want = orc.lut_to_gmkg(want, 4)
    got = _np_u16(lut)
    assert got.shape == want.shape
    assert np.array_equal(got, want)


@pytest.mark.parametrize("Hq,D,M,Kc,G,layout,cdt", [
    (512, 128, 32, 256, 4, "gmkg", "f32"),  # batch 16 x 32 heads: pipelined 64-head tiles
    (512, 128, 32, 256, 4, "gmkg", "f16"),  # ... fp16 codebooks
    (520, 128, 32, 256, 4, "gmkg", "f32"),  # ... with a partial last head tile
    (448, 128, 40, 206, 4, "gmkg", "f32"),  # ... last workgroup: one partial row tile
    (200, 64, 32, 256, 4, "hmk", "f32"),    # ... D = 64, reference layout
    (40, 128, 32, 256, 4, "gmkg", "f32"),   # partial head tile
    (24, 128, 5, 100, 2, "gmkg", "f32"),    # G = 2, M*K not a multiple of the row tile
    (64, 256, 8, 64, 4, "hmk", "f32"),      # D = 256
])
def test_lut_build_tiles(dev, K, orc, Hq, D, M, Kc, G, layout, cdt, lut_impl):
    from laprune_amd import _native as N
    print("device info (CUs, LDS per block, wave):", N.device_info(), flush=True)
    g = _gen(3 + Hq + D)
    q = torch.randn(Hq, D, generator=g).bfloat16()
    cb = torch.randn(M, Kc, D, generator=g) * 0.05
    cb_dev = cb.to(dev)
    if cdt == "f16":
        cb_dev = cb_dev.half()
        cb = cb.half().float()
    lut = K.aq_lut_build(q.to(dev), cb_dev, G=G, layout=layout)
    torch.cuda.synchronize()
    want = orc.lut_build(q.float().numpy(), cb.numpy())
    if layout == "gmkg":
        want = orc.lut_to_gmkg(want, G)
    assert np.array_equal(_np_u16(lut), want)


@pytest.mark.parametrize("tpw", [2, 3, 5])
@pytest.mark.parametrize("Hq,D,M,Kc,layout,cdt", [
    (512, 128, 32, 256, "gmkg", "f32"),  # C5's LUT
    (448, 128, 40, 206, "gmkg", "f32"),  # partial last row tile, groups cut short
    (520, 128, 32, 256, "hmk", "f16"),   # partial head tile, reference layout, fp16 codebooks
    (200, 64, 32, 256, "gmkg", "f32"),   # D = 64
])
def test_lut_build_pipelined(dev, K, orc, monkeypatch, Hq, D, M, Kc, layout, cdt, tpw):
    """The 64 x 64 MFMA form over several row tiles per workgroup (the next
    tile's rows fetched during the current tile's chain): bit-exact at forced
    tiles per workgroup, including groups that run past the last row tile."""
    monkeypatch.setenv("LAPRUNE_LUT_MFMA_TPW", str(tpw))
    g = _gen(11 + Hq + D + tpw)
    q = torch.randn(Hq, D, generator=g).bfloat16()
    cb = torch.randn(M, Kc, D, generator=g) * 0.05
    cb_dev = cb.to(dev)
    if cdt == "f16":
        cb_dev = cb_dev.half()
        cb = cb.half().float()
    print(f"lut pipelined: Hq={Hq} D={D} M={M} K={Kc} tpw={tpw}", flush=True)
    lut = K.aq_lut_build(q.to(dev), cb_dev, G=4, layout=layout)
    torch.cuda.synchronize()
    want = orc.lut_build(q.float().numpy(), cb.numpy())
    if layout == "gmkg":
        want = orc.lut_to_gmkg(want, 4)
    assert np.array_equal(_np_u16(lut), want)


@pytest.mark.parametrize("cdt", [torch.float32, torch.float16])
def test_lut_build_wide_range(dev, K, orc, lut_impl, cdt):
    """Operands spread over many binades, exact zeros, signed zeros and
    products below the fp32 normal range: the per-d rounding order shows in
    the fp16 outputs (many land near a rounding boundary or in overflow)."""
    g = _gen(11)
    Hq, D, M, Kc = 64, 128, 4, 64

    def spread(*shape):  # per-element spread of 8 binades
        return torch.randn(*shape, generator=g) * torch.exp2(
            torch.randint(-8, 1, shape, generator=g).float())
    # per-head and per-row scales: sums from far below fp16's subnormals
    # (fp32-subnormal products) through overflow to inf
    head_e = torch.cat([torch.linspace(-95, -60, 16), torch.linspace(-45, 14, Hq - 16)]).round()
    row_e = torch.randint(-35, 5, (M, Kc, 1), generator=g).float()
    q = spread(Hq, D) * torch.exp2(head_e)[:, None]
    q[:, ::7] = 0.0
    q[::5, 3::11] = -0.0
    q = q.bfloat16()
    cb = spread(M, Kc, D) * torch.exp2(row_e)
    if cdt == torch.float16:
        cb = (spread(M, Kc, D) * torch.exp2(row_e.clamp(min=-14) / 2)).to(cdt).float()
    cb_dev = cb.to(cdt).to(dev)
    lut = K.aq_lut_build(q.to(dev), cb_dev, G=4, layout="gmkg")
    torch.cuda.synchronize()
    want = orc.lut_to_gmkg(orc.lut_build(q.float().numpy(), cb.numpy()), 4)
    assert np.array_equal(_np_u16(lut), want)


def test_lut_build_odd_shapes(dev, K, orc):
    g = _gen(2)
    q = torch.randn(5, 64, generator=g)
    cb = torch.randn(3, 37, 64, generator=g) * 0.1
    lut = K.aq_lut_build(q.to(dev), cb.to(dev))
    assert np.array_equal(_np_u16(lut), orc.lut_build(q.numpy(), cb.numpy()))


# --------------------------------------------------------------- A2 scores

def _codes_view(g, Hkv, T, M=32, cap=0):
    buf = torch.randint(0, 256, (Hkv, T + cap, M), generator=g, dtype=torch.uint8)
    return buf, buf[:, :T, :]


@pytest.mark.parametrize("T,cap", [(1, 0), (1000, 0), (8192, 128), (20000, 64)])
@pytest.mark.parametrize("layout", ["hmk", "gmkg"])
def test_score_grouped_fast_path(dev, K, orc, T, cap, layout):
    from laprune_amd import _native as N
    g = _gen(3 + T)
    lut16 = (torch.randn(32, 32, 256, generator=g) * 0.3).half()
    buf, view = _codes_view(g, 8, T, cap=cap)
    dbuf = buf.to(dev)
    dview = dbuf[:, :T, :]
    if layout == "hmk":
        out = K.aq_lut_gather_grouped(lut16.to(dev), dview, 4)
    else:
        lut_il = lut16.view(8, 4, 32, 256).permute(0, 2, 3, 1).contiguous().to(dev)
        out = torch.empty(32, T, dtype=torch.float16, device=dev)
        N.call("lap_lut_score_grouped", N.ptr(lut_il), N.LUT_GMKG, N.ptr(dview), dview.stride(0),
               dview.stride(1), 8, 4, T, 32, 256, N.ptr(out), N.stream_of(out))
    torch.cuda.synchronize()
    want = orc.score_grouped(_np_u16(lut16), view.numpy(), 4)
    assert np.array_equal(_np_u16(out), want)


@pytest.mark.parametrize("G,M,Kc", [(2, 32, 256), (3, 16, 128), (4, 24, 256), (1, 8, 64)])
def test_score_grouped_generic(dev, K, orc, G, M, Kc):
    g = _gen(10 + G)
    Hkv, T = 3, 777
    lut16 = (torch.randn(Hkv * G, M, Kc, generator=g) * 0.3).half()
    codes = torch.randint(0, Kc, (Hkv, T, M), generator=g, dtype=torch.uint8)
    out = K.aq_lut_gather_grouped(lut16.to(dev), codes.to(dev), G)
    torch.cuda.synchronize()
    assert np.array_equal(_np_u16(out), orc.score_grouped(_np_u16(lut16), codes.numpy(), G))


@pytest.mark.parametrize("with_idx", [False, True])
@pytest.mark.parametrize("mrange", [(0, 32), (8, 24)])
def test_score_gqa(dev, K, orc, with_idx, mrange):
    g = _gen(20)
    Hkv, G, T = 2, 4, 3000
    lut16 = (torch.randn(Hkv * G, 32, 256, generator=g) * 0.3).half()
    buf, view = _codes_view(g, Hkv, T, cap=50)
    idx = None
    if with_idx:
        idx = torch.randint(-5, T + 5, (Hkv * G, 300), generator=g, dtype=torch.int64)
    out = K.aq_lut_gather_gqa(lut16.to(dev), buf.to(dev)[:, :T, :], G, mrange[0], mrange[1],
                              None if idx is None else idx.to(dev))
    torch.cuda.synchronize()
    want = orc.score_gqa(_np_u16(lut16), view.numpy(), G, mrange[0], mrange[1],
                         None if idx is None else idx.numpy())
    assert np.array_equal(_np_u16(out), want)


@pytest.mark.parametrize("lut_dt", [torch.float16, torch.float32])
@pytest.mark.parametrize("code_dt", [torch.uint8, torch.int8, torch.int64])
def test_score_mha(dev, K, orc, lut_dt, code_dt):
    g = _gen(30)
    Q, n, M, Kc = 5, 999, 32, 200
    lut = (torch.randn(Q, M * Kc, generator=g) * 0.3).to(lut_dt)
    if code_dt == torch.int64:
        codes = torch.randint(-300, 600, (Q, n, M), generator=g, dtype=torch.int64)
    else:
        codes = torch.randint(-128 if code_dt == torch.int8 else 0,
                              128 if code_dt == torch.int8 else 256, (Q, n, M), generator=g,
                              dtype=torch.int64).to(code_dt)
    out = K.aq_lut_gather_forward(lut.to(dev), codes.to(dev))
    torch.cuda.synchronize()
    f32 = lut_dt == torch.float32
    want = orc.score_mha(lut.numpy() if f32 else _np_u16(lut), codes.numpy(), f32)
    got = out.cpu().numpy() if f32 else _np_u16(out)
    assert np.array_equal(got.view(np.uint32) if f32 else got, want.view(np.uint32) if f32 else want)


@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
def test_aq_lut_direct(dev, K, orc, dt):
    g = _gen(40)
    Q, n, M, Kc, D = 3, 300, 8, 64, 128
    q = torch.randn(Q, D, generator=g).to(dt)
    cb = (torch.randn(M, Kc, D, generator=g) * 0.05).to(dt)
    codes = torch.randint(0, 80, (Q, n, M), generator=g, dtype=torch.int64)
    out = K.aq_lut_forward(q.to(dev), cb.to(dev), codes.to(dev))
    torch.cuda.synchronize()
    if dt == torch.float32:
        want = orc.aq_direct(q.numpy(), cb.numpy(), codes.numpy(), False)
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))
    else:
        want = orc.aq_direct(_np_u16(q), _np_u16(cb), codes.numpy(), True)
        assert np.array_equal(_np_u16(out), want)


# ---------------------------------------------------------- reconstruction

@pytest.mark.parametrize("code_dt", [torch.uint8, torch.int8, torch.int64])
@pytest.mark.parametrize("Kc,D", [(256, 128), (100, 64), (37, 4)])
def test_aq_reconstruct(dev, K, orc, code_dt, Kc, D):
    """Approximate keys from codes (aq_kv.py:431-457) bit for bit against the
    oracle's ascending-m fp32 sum: every code dtype (low 8 bits, clamped to
    K - 1), rows a strided view (the M codes of each row inside a wider row)."""
    from laprune_amd.aq_kernels import _impl
    g = _gen(60 + Kc)
    M, n = 32, 1000
    cb = torch.randn(M, Kc, D, generator=g) * 0.05
    wide = torch.randint(-300 if code_dt == torch.int64 else 0, 600 if code_dt == torch.int64
                         else 256, (n, M + 5), generator=g, dtype=torch.int64).to(code_dt)
    codes = wide[:, 2:2 + M]  # row stride M + 5
    out = _impl.aq_reconstruct(cb.to(dev), codes.to(dev))
    torch.cuda.synchronize()
    want = orc.reconstruct(cb.numpy(), codes.numpy().astype(np.int64))
    assert out.shape == (n, D) and out.dtype == torch.float32
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_aq_reconstruct_grid_stride(dev, K, orc):
    """40003 rows at D = 128: more quads than one pass of the grid, so
    threads loop; first and last 128 rows and 512 random rows checked."""
    from laprune_amd.aq_kernels import _impl
    g = _gen(66)
    M, Kc, D, n = 32, 256, 128, 40003
    cb = torch.randn(M, Kc, D, generator=g) * 0.05
    codes = torch.randint(0, Kc, (n, M), generator=g, dtype=torch.int64).to(torch.uint8)
    out = _impl.aq_reconstruct(cb.to(dev), codes.to(dev)).cpu().numpy()
    pick = torch.randperm(n - 256, generator=g)[:512].numpy() + 128
    rows = np.unique(np.concatenate([np.arange(128), np.arange(n - 128, n), pick]))
    want = orc.reconstruct(cb.numpy(), codes.numpy()[rows])
    assert np.array_equal(out[rows].view(np.uint32), want.view(np.uint32))


def test_manager_reconstruct_and_inner_product(dev, K, orc):
    """AQLayerCodebookManager.reconstruct / approx_inner_product pick the
    head's group codebooks (head // heads_per_group) and match the oracle:
    reconstruction bit-exact; inner products bit-exact to the fp16 LUT and
    sequential fp32 sum of this path, and close to q . reconstruct(codes)."""
    from laprune_amd.aq_kv import AQLayerCodebookManager, AQLayerConfig
    g = _gen(70)
    M, Kc, D, n = 32, 256, 128, 3000
    mgr = AQLayerCodebookManager({5: AQLayerConfig(M=M, K=Kc, d=D, heads_per_group=2,
                                                   num_heads=8)}, device=dev)
    cbs = [torch.randn(M, Kc, D, generator=g) * 0.05 for _ in range(4)]
    for gi, cb in enumerate(cbs):
        mgr.set_codebooks(5, gi, cb)
    codes = torch.randint(0, Kc, (n, M), generator=g, dtype=torch.uint8)
    q = torch.randn(D, generator=g)
    for head in (0, 3, 7):
        cb = cbs[head // 2]
        rec = mgr.reconstruct(5, head, codes.to(dev))
        want = orc.reconstruct(cb.numpy(), codes.numpy())
        assert np.array_equal(rec.cpu().numpy().view(np.uint32), want.view(np.uint32))
        s = mgr.approx_inner_product(5, head, q.to(dev)[None, :], codes)
        torch.cuda.synchronize()
        lut = orc.lut_build(q.numpy()[None, :], cb.numpy())  # fp16 bits [1, M, K]
        want_s = orc.score_mha(lut.reshape(1, M * Kc), codes.numpy()[None].astype(np.int64),
                               False)[0]
        assert s.shape == (n,) and np.array_equal(_np_u16(s), want_s)
        exact = want.astype(np.float64) @ q.numpy().astype(np.float64)
        got = s.float().cpu().numpy()
        assert np.max(np.abs(got - exact)) < 2e-2 * max(1.0, float(np.max(np.abs(exact))))


# ---------------------------------------------------------------- A3 top-k

@pytest.mark.parametrize("group,key_dt", [(1, torch.float16), (4, torch.float16),
                                          (4, torch.bfloat16), (1, torch.bfloat16)])
@pytest.mark.parametrize("T,cs,ce,k", [(8192, 0, 8128, 163), (8192, 4, 8128, 2048),
                                       (5000, 10, 4990, 5000), (70000, 0, 70000, 1),
                                       (3000, 0, 3000, 2999)])
def test_topk(dev, K, orc, group, key_dt, T, cs, ce, k):
    g = _gen(50 + T + k)
    R = 3
    # coarse values to force many ties
    s = (torch.randn(R * group, T, generator=g) * 4).round().half() / 4
    idx = K.aq_topk(s.to(dev), k, group=group, cand_start=cs, cand_end=ce, key_dtype=key_dt)
    torch.cuda.synchronize()
    bits = _np_u16(s)
    want = orc.topk(bits, k, group, cs, ce, key_bf16=key_dt == torch.bfloat16)
    want2 = orc.topk_numpy(bits, k, group, cs, ce, key_bf16=key_dt == torch.bfloat16)
    assert np.array_equal(want, want2)
    assert np.array_equal(idx.cpu().numpy(), want)


def test_topk_all_equal_and_int32(dev, K, orc):
    s = torch.zeros(2, 4096, dtype=torch.float16)
    s[1] = -0.0
    idx = K.aq_topk(s.to(dev), 100, cand_start=7, cand_end=4000, index_dtype=torch.int32)
    torch.cuda.synchronize()
    assert idx.dtype == torch.int32
    assert np.array_equal(idx.cpu().numpy(), np.tile(np.arange(7, 107), (2, 1)))


@pytest.mark.parametrize("B,T,k,key_dt", [(2, 8192, 163, torch.bfloat16),
                                          (2, 30000, 1024, torch.float16),
                                          (1, 131072, 2621, torch.bfloat16)])
def test_retrieve_topk_per_head(dev, K, orc, B, T, k, key_dt):
    """One top-k per query head from the fused scorer (LAP_SELECT_PER_HEAD):
    the reference's own selection (k = 2621 of 131004 candidates on bf16-cast
    scores at 128k).  Rows are b * 32 + h; the split form (score, then
    lap_retrieve_select_heads) gives the same indices."""
    from laprune_amd import _native as N
    g = _gen(70 + T + B)
    Hkv, Hq, cap = 8, 32, 64
    q = torch.randn(B * Hq, 128, generator=g).bfloat16()
    cb = torch.randn(32, 256, 128, generator=g) * 0.02
    buf = torch.randint(0, 256, (B, Hkv, T + cap, 32), generator=g, dtype=torch.uint8)
    codes = buf.to(dev)[:, :, :T, :]
    lut = K.aq_lut_build(q.to(dev), cb.to(dev), G=4, layout="gmkg")
    cs, ce = orc.candidate_window(T, T, 4, 64)
    idx, scores = K.aq_retrieve_topk(lut, codes, k, cs, ce, key_dtype=key_dt,
                                     return_scores=True, per_head=True)
    # the split form
    kmode = (N.KEY_BF16 if key_dt == torch.bfloat16 else N.KEY_F16) | N.SELECT_PER_HEAD
    ws = torch.empty(N.size_query("lap_retrieve_workspace_size", B * Hq, T), dtype=torch.uint8,
                     device=dev)
    idx2 = torch.full((B, Hq, k), -3, dtype=torch.int32, device=dev)
    N.call("lap_retrieve_score", N.ptr(lut), N.ptr(codes), codes.stride(0), codes.stride(1),
           codes.stride(2), B, Hkv, T, cs, ce, kmode, None, N.ptr(ws), ws.numel(),
           N.stream_of(idx2))
    N.call("lap_retrieve_select_heads", B, Hkv, T, cs, ce, k, N.ptr(idx2), N.I32, N.ptr(ws),
           ws.numel(), N.stream_of(idx2))
    torch.cuda.synchronize()
    assert tuple(idx.shape) == (B, Hq, k)
    assert np.array_equal(idx.cpu().numpy(), idx2.cpu().numpy())
    lut_hmk = orc.lut_build(q.float().numpy(), cb.numpy())
    for b in range(B):
        want_s = orc.score_grouped(lut_hmk[b * Hq:(b + 1) * Hq], buf[b, :, :T, :].numpy(), 4)
        assert np.array_equal(_np_u16(scores[b]), want_s)
        want_i = orc.topk(want_s, k, group=1, cand_start=cs, cand_end=ce,
                          key_bf16=key_dt == torch.bfloat16)
        assert np.array_equal(idx[b].cpu().numpy().astype(np.int64), want_i), b


@pytest.mark.parametrize("T,k", [(32768, 1024), (3001, 2933), (20000, 1), (9000, 8000)])
def test_retrieve_topk_all_equal(dev, K, orc, T, k):
    """Every token scores the same: each key of the window is a candidate
    (the selection's candidate lists run full) and all of them tie, so the
    result is the k lowest columns of the window."""
    Hkv, cap = 8, 64
    g = _gen(61)
    q = torch.randn(32, 128, generator=g).bfloat16()
    cb = torch.randn(32, 256, 128, generator=g) * 0.02
    codes = torch.full((1, Hkv, T + cap, 32), 17, dtype=torch.uint8, device=dev)[:, :, :T, :]
    lut = K.aq_lut_build(q.to(dev), cb.to(dev), G=4, layout="gmkg")
    cs, ce = orc.candidate_window(T, T, 4, 64)
    k = min(k, ce - cs)
    idx = K.aq_retrieve_topk(lut, codes, k, cs, ce)
    torch.cuda.synchronize()
    want = np.tile(np.arange(cs, cs + k), (Hkv, 1))
    assert np.array_equal(idx[0].cpu().numpy().astype(np.int64), want)


@pytest.mark.parametrize("T,k,key_dt", [(8192, 2048, torch.float16), (131072, 2048, torch.float16),
                                        (131072, 2621, torch.bfloat16), (4096, 5000, torch.float16)])
def test_retrieve_topk_fused(dev, K, orc, T, k, key_dt):
    g = _gen(60 + T)
    Hkv, cap = 8, 128
    q = torch.randn(32, 128, generator=g).bfloat16()
    cb = torch.randn(32, 256, 128, generator=g) * 0.02
    buf = torch.randint(0, 256, (1, Hkv, T + cap, 32), generator=g, dtype=torch.uint8)
    dbuf = buf.to(dev)
    codes = dbuf[:, :, :T, :]
    lut = K.aq_lut_build(q.to(dev), cb.to(dev), G=4, layout="gmkg")
    cs, ce = orc.candidate_window(T, T, 4, 64)
    idx, scores = K.aq_retrieve_topk(lut, codes, k, cs, ce, key_dtype=key_dt, return_scores=True)
    torch.cuda.synchronize()
    lut_hmk = orc.lut_build(q.float().numpy(), cb.numpy())
    want_s = orc.score_grouped(lut_hmk, buf[0, :, :T, :].numpy(), 4)
    assert np.array_equal(_np_u16(scores[0]), want_s)
    want_i = orc.topk(want_s, k, group=4, cand_start=cs, cand_end=ce,
                      key_bf16=key_dt == torch.bfloat16)
    assert np.array_equal(idx[0].cpu().numpy().astype(np.int64), want_i)


# --------------------------------------------------------------- A4 gather

@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("tail", [None, (40, 24)])
def test_gqa_gather_kv(dev, K, orc, dt, tail):
    g = _gen(70)
    B, Hkv, T, D, G, n = 2, 2, 100, 128, 4, 17
    buf_k = torch.randn(B, Hkv, T + 28, D, generator=g).to(dt)
    buf_v = torch.randn(B, Hkv, T + 28, D, generator=g).to(dt)
    idx = torch.randint(0, T, (B, Hkv * G, n), generator=g, dtype=torch.int64)
    dk, dv = buf_k.to(dev)[:, :, :T], buf_v.to(dev)[:, :, :T]
    if tail is None:
        ok, ov = K.gqa_gather_kv(dk, dv, idx.to(dev), G)
        full = idx.numpy()
    else:
        ok, ov = K.gqa_gather_kv_with_tail(dk, dv, idx.to(dev), G, tail[0], tail[1])
        t_idx = np.broadcast_to(np.arange(tail[0], tail[0] + tail[1]), (B, Hkv * G, tail[1]))
        full = np.concatenate([idx.numpy(), t_idx], axis=2)
    torch.cuda.synchronize()
    want_k = orc.gather_rows(buf_k[:, :, :T].float().numpy(), full, G)
    want_v = orc.gather_rows(buf_v[:, :, :T].float().numpy(), full, G)
    assert np.array_equal(ok.float().cpu().numpy(), want_k)
    assert np.array_equal(ov.float().cpu().numpy(), want_v)


def test_gqa_gather_out_of_range_rows_untouched(dev, K):
    B, Hkv, T, D = 1, 1, 10, 64
    k = torch.randn(B, Hkv, T, D, device=dev, dtype=torch.float16)
    idx = torch.tensor([[[0, -1, 10, 3]]], dtype=torch.int64, device=dev)
    ok, ov = K.gqa_gather_kv(k, k, idx, 1)
    torch.cuda.synchronize()
    assert torch.equal(ok[0, 0, 0], k[0, 0, 0]) and torch.equal(ok[0, 0, 3], k[0, 0, 3])


# ---------------------------------------------------------- A5 attention

def _rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-6))


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("per_head", [False, True])
@pytest.mark.parametrize("D", [128, 64, 256])
def test_sparse_attn_decode(dev, K, orc, dt, per_head, D):
    g = _gen(80 + D)
    B, Hq, Hkv, T, n = 2, 8, 2, 3000, 300
    q = torch.randn(B, Hq, 1, D, generator=g).to(dt)
    kk = torch.randn(B, Hkv, T + 16, D, generator=g).to(dt)
    vv = torch.randn(B, Hkv, T + 16, D, generator=g).to(dt)
    H_idx = Hq if per_head else Hkv
    idx = torch.randint(4, T - 64, (B, H_idx, n), generator=g, dtype=torch.int64)
    out = K.sparse_attn_decode(q.to(dev), kk.to(dev)[:, :, :T], vv.to(dev)[:, :, :T],
                               idx.to(dev), sink=4, tail_start=T - 64, tail_count=64)
    torch.cuda.synchronize()
    G = Hq // Hkv

    def keep(b, h):
        row = h if per_head else h // G
        return np.concatenate([idx[b, row].numpy(), np.arange(4), np.arange(T - 64, T)])

    want = orc.attn_decode_f64(q[:, :, 0].double().numpy(), kk[:, :, :T].double().numpy(),
                               vv[:, :, :T].double().numpy(), keep)
    assert _rel(out[:, :, 0].double().cpu().numpy(), want) < 1e-2


@pytest.mark.parametrize("T", [1, 63, 64, 5000, 131072])
def test_dense_attn_decode(dev, K, orc, T):
    g = _gen(90 + T)
    B, Hq, Hkv, D = 1, 32, 8, 128
    q = torch.randn(B, Hq, 1, D, generator=g).bfloat16()
    kk = torch.randn(B, Hkv, T, D, generator=g).bfloat16()
    vv = torch.randn(B, Hkv, T, D, generator=g).bfloat16()
    out = K.dense_attn_decode(q.to(dev), kk.to(dev), vv.to(dev))
    torch.cuda.synchronize()
    want = orc.attn_decode_f64(q[:, :, 0].double().numpy(), kk.double().numpy(),
                               vv.double().numpy(), lambda b, h: np.arange(T))
    assert _rel(out[:, :, 0].double().cpu().numpy(), want) < 1e-2


# --------------------------------------------------------------- A6 encode

# 20000 and 40000 rows take the 32- and 64-row workgroup tiles (two and four
# row groups sharing each codebook fragment) on a 256-CU device; 40003 leaves a
# partial last tile.
@pytest.mark.parametrize("N,D", [(512, 128), (37, 64), (3, 256), (20000, 128), (40003, 128),
                                 (40000, 64)])
def test_encode_bit_exact(dev, K, orc, N, D):
    g = _gen(100 + N)
    M, Kc = 32, 256
    x = torch.randn(N, D, generator=g) * (torch.rand(D, generator=g) * 3.5 + 0.5)
    cb = torch.randn(M, Kc, D, generator=g) * 0.02
    codes, rn = K.aq_encode_greedy(x.to(dev), cb.to(dev))
    torch.cuda.synchronize()
    # rows are encoded independently: large launches are checked on the first
    # and last 128 rows (the partial last tile included) and 512 random rows
    rows = np.arange(N)
    if N > 4096:
        pick = torch.randperm(N - 256, generator=g)[:512].numpy() + 128
        rows = np.unique(np.concatenate([np.arange(128), np.arange(N - 128, N), pick]))
    want_c, want_r = orc.encode(x.numpy()[rows], cb.numpy())
    assert np.array_equal(codes.cpu().numpy()[rows], want_c)
    assert np.array_equal(rn.cpu().numpy()[rows].view(np.uint32), want_r.view(np.uint32))


def test_encode_c3_config(dev, K, orc, encode_rows):
    """BASELINE config C3 exactly: 8 KV heads x 64 post-RoPE keys (pre-RoPE
    bf16 N(0,1) x per-channel U(0.5, 4), rotate-half RoPE with theta 500000
    at positions 131008..131071), 32 x 256 fp32 codebooks N(0, 0.02):
    codes and residual norms bit-exact against the oracle."""
    g = _gen(303)
    Hkv, n_tok, D = 8, 64, 128
    k = (torch.randn(Hkv, n_tok, D, generator=g) *
         (torch.rand(D, generator=g) * 3.5 + 0.5)).bfloat16().float()
    pos = torch.arange(131008, 131008 + n_tok, dtype=torch.float64)
    inv = 500000.0 ** (-torch.arange(0, D, 2, dtype=torch.float64) / D)
    ang = pos[:, None] * inv[None, :]
    cos = torch.cat([ang.cos(), ang.cos()], -1).float()
    sin = torch.cat([ang.sin(), ang.sin()], -1).float()
    x = (k * cos + torch.cat([-k[..., D // 2:], k[..., :D // 2]], -1) * sin).reshape(-1, D)
    cb = torch.randn(32, 256, D, generator=g) * 0.02
    codes, rn = K.aq_encode_greedy(x.to(dev), cb.to(dev))
    torch.cuda.synchronize()
    want_c, want_r = orc.encode(x.numpy(), cb.numpy())
    assert codes.shape == (Hkv * n_tok, 32)
    assert np.array_equal(codes.cpu().numpy(), want_c)
    assert np.array_equal(rn.cpu().numpy().view(np.uint32), want_r.view(np.uint32))


@pytest.fixture(params=["4", "16", "x1", "x2"])
def encode_rows(request, monkeypatch):
    """Runs a test on the 4-row and the 16-row MFMA workgroup kernels and on
    the exact-distance kernel at 1 and 2 rows per workgroup (flushes take
    the exact kernel by default)."""
    if request.param.startswith("x"):
        monkeypatch.setenv("LAPRUNE_ENCODE_EXACT", "1")
        monkeypatch.setenv("LAPRUNE_ENCODE_EXACT_ROWS", request.param[1:])
        return int(request.param[1:])
    monkeypatch.setenv("LAPRUNE_ENCODE_ROWS", request.param)
    return int(request.param)


@pytest.mark.parametrize("N,D", [(512, 128), (37, 64), (2048, 128)])
def test_encode_both_small_kernels(dev, K, orc, N, D, encode_rows):
    g = _gen(150 + N)
    M, Kc = 32, 256
    x = torch.randn(N, D, generator=g) * (torch.rand(D, generator=g) * 3.5 + 0.5)
    cb = torch.randn(M, Kc, D, generator=g) * 0.02
    codes, rn = K.aq_encode_greedy(x.to(dev), cb.to(dev))
    torch.cuda.synchronize()
    want_c, want_r = orc.encode(x.numpy(), cb.numpy())
    assert np.array_equal(codes.cpu().numpy(), want_c)
    assert np.array_equal(rn.cpu().numpy().view(np.uint32), want_r.view(np.uint32))


@pytest.mark.parametrize("Kc,D", [(60, 64), (48, 128), (16, 64), (240, 128)])
def test_encode_bit_exact_entry_counts(dev, K, orc, Kc, D, encode_rows):
    """K % 16 != 0 takes the all-VALU search, the rest the MFMA search with
    fewer entry tiles than waves."""
    g = _gen(120 + Kc)
    M, N = 8, 45
    x = torch.randn(N, D, generator=g) * 2.0
    cb = torch.randn(M, Kc, D, generator=g) * 0.05
    codes, rn = K.aq_encode_greedy(x.to(dev), cb.to(dev))
    torch.cuda.synchronize()
    want_c, want_r = orc.encode(x.numpy(), cb.numpy())
    assert np.array_equal(codes.cpu().numpy(), want_c)
    assert np.array_equal(rn.cpu().numpy().view(np.uint32), want_r.view(np.uint32))


def test_encode_more_stages_than_staged_codes(dev, K, orc, encode_rows):
    """M = 80 stages: codes of stages 64 and up are stored as they are
    chosen, the first 64 staged in LDS and stored at the end."""
    g = _gen(125)
    M, Kc, D, N = 80, 32, 64, 45
    x = torch.randn(N, D, generator=g) * 2.0
    cb = torch.randn(M, Kc, D, generator=g) * 0.05
    codes, rn = K.aq_encode_greedy(x.to(dev), cb.to(dev))
    torch.cuda.synchronize()
    want_c, want_r = orc.encode(x.numpy(), cb.numpy())
    assert codes.shape == (N, M)
    assert np.array_equal(codes.cpu().numpy(), want_c)
    assert np.array_equal(rn.cpu().numpy().view(np.uint32), want_r.view(np.uint32))


def test_encode_ties_and_near_ties(dev, K, orc, encode_rows):
    """Duplicate entries (exact ties: the lowest index must win) and entries a
    few ulps apart, far inside the bf16 coarse error, so the exact recheck
    decides."""
    g = _gen(130)
    M, Kc, D, N = 6, 64, 128, 80
    cb = torch.randn(M, Kc, D, generator=g) * 0.05
    cb[:, 40] = cb[:, 7]                       # exact duplicate of an earlier entry
    cb[:, 41] = cb[:, 7] * (1 + 2 ** -20)      # a hair away from it
    cb[:, 63] = cb[:, 12].clone()
    cb[:, 63, 0] = torch.nextafter(cb[:, 12, 0], torch.tensor(1.0))
    # rows built from the duplicated entries so that they are the likely winners
    x = torch.zeros(N, D)
    for i in range(N):
        k = [7, 40, 41, 12, 63][i % 5]
        x[i] = sum(cb[m, k] for m in range(M)) + torch.randn(D, generator=g) * 1e-3
    codes, rn = K.aq_encode_greedy(x.to(dev), cb.to(dev))
    torch.cuda.synchronize()
    want_c, want_r = orc.encode(x.numpy(), cb.numpy())
    assert np.array_equal(codes.cpu().numpy(), want_c)
    assert np.array_equal(rn.cpu().numpy().view(np.uint32), want_r.view(np.uint32))
    assert 40 not in set(codes.cpu().numpy().ravel().tolist())  # ties go to entry 7


def test_encode_non_finite_rows(dev, K, orc, encode_rows):
    """Rows whose norms overflow or hold NaN take the full exact scan and
    follow the contract (NaN and +inf distances never win; no finite
    distance gives code 0)."""
    g = _gen(140)
    M, Kc, D, N = 4, 32, 64, 20
    cb = torch.randn(M, Kc, D, generator=g) * 0.05
    x = torch.randn(N, D, generator=g)
    x[3, 5] = float("nan")
    x[7] = 3e19            # rn overflows to +inf
    x[11, 0] = float("inf")
    codes, rn = K.aq_encode_greedy(x.to(dev), cb.to(dev))
    torch.cuda.synchronize()
    want_c, want_r = orc.encode(x.numpy(), cb.numpy())
    assert np.array_equal(codes.cpu().numpy(), want_c)
    got_r = rn.cpu().numpy()
    assert np.array_equal(np.isnan(got_r), np.isnan(want_r))
    fin = ~np.isnan(want_r)
    assert np.array_equal(got_r[fin].view(np.uint32), want_r[fin].view(np.uint32))


def test_fused_linear_encode_dropin(dev, K, orc):
    g = _gen(110)
    M, Kc, D, N = 32, 256, 128, 64
    cb = torch.randn(M, Kc, D, generator=g) * 0.02
    x = torch.randn(N, D, generator=g)
    cbh = cb.half()
    weight_t = cbh.transpose(1, 2).contiguous()
    bias = (-0.5 * cbh.float().pow(2).sum(-1)).half()
    codes = K.fused_linear_encode_forward(x.half().to(dev), weight_t.to(dev), bias.to(dev),
                                          cbh.to(dev), True, 0)
    torch.cuda.synchronize()
    want, _ = orc.encode(x.half().float().numpy(), cbh.float().numpy())
    assert codes.dtype == torch.uint8 and np.array_equal(codes.cpu().numpy(), want)


# ------------------------------------------------- decode caches (A2/A6 callers)

def test_encode_keys_strided_matches_flat(dev, K, orc):
    """lap_encode_keys on a token range of a strided [B][H][Tcap][D] bf16 cache
    writes the same codes and residual norms as the flat encode of those rows."""
    from laprune_amd import _native as Nn
    g = _gen(150)
    B, H, Tcap, D, M, Kc = 2, 3, 120, 128, 32, 256
    t0, t1 = 37, 81
    keys = (torch.randn(B, H, Tcap, D, generator=g) * 2).bfloat16()
    cb = torch.randn(M, Kc, D, generator=g) * 0.02
    kd, cbd = keys.to(dev), cb.to(dev)
    prep = K.aq_encode_prepare(cbd)
    codes = torch.zeros(B, H, Tcap + 8, M, dtype=torch.uint8, device=dev)
    rn = torch.empty(B * H * (t1 - t0), dtype=torch.float32, device=dev)
    Nn.call("lap_encode_keys", Nn.ptr(kd), Nn.BF16, kd.stride(0), kd.stride(1), kd.stride(2),
            B, H, t0, t1, D, Nn.ptr(cbd), M, Kc, Nn.ptr(prep), prep.numel(), Nn.ptr(codes),
            codes.stride(0), codes.stride(1), codes.stride(2), Nn.ptr(rn), Nn.stream_of(kd))
    torch.cuda.synchronize()
    flat = keys[:, :, t0:t1].float().reshape(-1, D)
    want_c, want_r = orc.encode(flat.numpy(), cb.numpy())
    got = codes[:, :, t0:t1].reshape(-1, M).cpu().numpy()
    assert np.array_equal(got, want_c)
    assert np.array_equal(rn.cpu().numpy().view(np.uint32), want_r.view(np.uint32))
    # untouched outside the range
    assert int(codes[:, :, :t0].abs().sum()) == 0 and int(codes[:, :, t1:].abs().sum()) == 0


def test_decode_cache_growth_flushes_and_codes(dev, K, orc):
    """Prefill, then single-token appends through capacity growth: views hold
    what was appended, encodes follow the 64-token rule, codes are exact."""
    from laprune_amd.cache import DecodeKVCache
    g = _gen(160)
    B, H, D, M, Kc = 1, 2, 128, 32, 256
    cb = torch.randn(M, Kc, D, generator=g) * 0.02
    cache = DecodeKVCache(cb.to(dev), B, H, D, capacity=64, group_size=64)
    k_all = (torch.randn(B, H, 300 + 140, D, generator=g) * 1.5).bfloat16()
    v_all = torch.randn(B, H, 300 + 140, D, generator=g).bfloat16()
    cache.append(k_all[:, :, :300].to(dev), v_all[:, :, :300].to(dev), prefill=True)
    assert cache.length == 300 and cache.encoded_len == 300 and cache.capacity >= 300
    enc_points = []
    for t in range(300, 440):
        cache.append(k_all[:, :, t:t + 1].to(dev), v_all[:, :, t:t + 1].to(dev))
        if cache.encoded_len == cache.length:
            enc_points.append(cache.length)
    torch.cuda.synchronize()
    assert enc_points == [364, 428]
    assert cache.length == 440 and cache.encoded_len == 428
    assert torch.equal(cache.keys().cpu(), k_all) and torch.equal(cache.values().cpu(), v_all)
    want, _ = orc.encode(k_all[:, :, :428].float().reshape(-1, D).numpy(), cb.numpy())
    got = cache.encoded_codes().reshape(-1, M).cpu().numpy()
    assert np.array_equal(got, want)


def test_decode_step_over_cache(dev, K, orc):
    """step_cached scores only encoded keys; the unencoded tail is attended
    through the local window; output matches the float64 keep-list attention."""
    from laprune_amd.cache import DecodeKVCache
    from laprune_amd.retrieval import RetrievalConfig, SparseDecoder
    g = _gen(170)
    B, Hq, Hkv, D, M, Kc = 1, 32, 8, 128, 32, 256
    T0, steps = 1000, 30
    cb = torch.randn(M, Kc, D, generator=g) * 0.02
    cache = DecodeKVCache(cb.to(dev), B, Hkv, D, capacity=T0 + steps, group_size=64)
    kk = torch.randn(B, Hkv, T0 + steps, D, generator=g).bfloat16()
    vv = torch.randn(B, Hkv, T0 + steps, D, generator=g).bfloat16()
    cache.append(kk[:, :, :T0].to(dev), vv[:, :, :T0].to(dev), prefill=True)
    cfg = RetrievalConfig(topk=64, select="group")
    dec = SparseDecoder(cb.to(dev), B, Hq, Hkv, D, T0 + steps, cfg)
    for t in range(T0, T0 + steps):
        cache.append(kk[:, :, t:t + 1].to(dev), vv[:, :, t:t + 1].to(dev))
        q = torch.randn(B, Hq, 1, D, generator=g).bfloat16()
        out = dec.step_cached(q.to(dev), cache)
        torch.cuda.synchronize()
        sel = dec.selected().cpu().numpy()
        assert sel.max() < cache.encoded_len and sel.shape[-1] == 64
        p = dec.plan(cache.encoded_len, cache.length)
        assert p["cand_end"] <= cache.encoded_len
        keep = lambda b, h: np.concatenate([sel[b, h // 4], np.arange(p["sink"]),
                                            np.arange(p["tail_start"], p["tail_start"] + p["tail_count"])])
        want = orc.attn_decode_f64(q[:, :, 0].double().numpy(), kk[:, :, :t + 1].double().numpy(),
                                   vv[:, :, :t + 1].double().numpy(), keep)
        assert _rel(out[:, :, 0].double().cpu().numpy(), want) < 1e-2


# ------------------------------------------------- decode RoPE + cache append

@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_rope_append_matches_hf(dev, dt):
    """lap_rope_append against HF apply_rotary_pos_emb and an index write:
    bit-identical rotated q, cache rows written at each sequence's position,
    nothing else touched, and a position at the capacity bound skipped."""
    from transformers.models.llama.modeling_llama import (LlamaRotaryEmbedding,
                                                          apply_rotary_pos_emb)
    from laprune_amd import _native as N
    from laprune_amd.llama import llama31_8b_config
    g = _gen(123)
    B, Hq, Hkv, D, cap = 4, 32, 8, 128, 96
    rot = LlamaRotaryEmbedding(llama31_8b_config(num_layers=1)).to(dev)
    h = (torch.randn(B, 1, (Hq + 2 * Hkv) * D, generator=g) * 3).to(dt).to(dev)
    q, k, v = h.split([Hq * D, Hkv * D, Hkv * D], dim=-1)   # strided views, like projections
    pos = torch.tensor([[5], [95], [0], [96]], dtype=torch.long, device=dev)  # 96: past capacity
    cos, sin = rot(h, torch.tensor([[5], [95], [0], [96]], device=dev))
    cos, sin = cos.to(dt), sin.to(dt)
    ck = torch.randn(B, Hkv, cap, D, generator=g).to(dt).to(dev)
    cv = torch.randn(B, Hkv, cap, D, generator=g).to(dt).to(dev)
    ck0, cv0 = ck.clone(), cv.clone()
    q_out = torch.empty(B, Hq, D, dtype=dt, device=dev)
    N.call("lap_rope_append", N.ptr(q), q.stride(0), D, N.ptr(k), k.stride(0), D, N.ptr(v),
           v.stride(0), D, N.ptr(cos), N.ptr(sin), cos.stride(0), N.dtype_code(dt), B, Hq, Hkv,
           D, N.ptr(pos), N.ptr(ck), ck.stride(0), ck.stride(1), ck.stride(2), N.ptr(cv),
           cv.stride(0), cv.stride(1), cv.stride(2), cap, N.ptr(q_out), N.stream_of(q_out))
    torch.cuda.synchronize()
    qh = q.view(B, 1, Hq, D).transpose(1, 2)
    kh = k.view(B, 1, Hkv, D).transpose(1, 2)
    qr, kr = apply_rotary_pos_emb(qh, kh, cos, sin)
    u16 = lambda t: t.contiguous().view(torch.int16).cpu()  # noqa: E731
    assert torch.equal(u16(q_out), u16(qr[:, :, 0]))
    want_k, want_v = ck0.clone(), cv0.clone()
    for b, t in enumerate(pos[:, 0].tolist()):
        if t < cap:
            want_k[b, :, t] = kr[b, :, 0]
            want_v[b, :, t] = v.view(B, Hkv, D)[b]
    assert torch.equal(u16(ck), u16(want_k))
    assert torch.equal(u16(cv), u16(want_v))
