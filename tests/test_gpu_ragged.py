"""Ragged batches (one length per sequence) and the per-head step, on the GPU.

Every sequence of a ragged call must get exactly what a call with its own
length would give: indices bit-exact against the oracle's top-k over that
sequence's scores and window, attention within 1e-2 of float64 over that
sequence's keep set.  Plans are built from the oracle's window and budget
arithmetic (oracle/orc.py) and handed to the C ABI as device arrays.
"""
import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SINK, LOCAL = 4, 64


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _np_u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-6))


def _keep_parts(t_total):
    """(sink, tail_start, tail_count) from the oracle's keep list."""
    kl = _orc().keep_list(np.zeros(0, np.int64), t_total, SINK, LOCAL)
    sink = int(np.sum(kl < SINK)) if kl.size else 0
    tail = kl[sink:]
    return sink, (int(tail[0]) if tail.size else t_total), int(tail.size)


def _orc():
    from oracle import orc
    return orc


def _plan(orc, tc, tt, topk):
    cs, ce = orc.candidate_window(tc, tt, SINK, LOCAL)
    n = ce - cs
    k = (min(topk, n) if topk is not None else orc.budget_k(n)) if tc > 0 else 0
    sink, ts, tn = _keep_parts(tt)
    return dict(t_codes=tc, t_total=tt, cand_start=cs, cand_end=ce, k=k, sink=sink,
                tail_start=ts, tail_count=tn)


def _plans_dev(plans, dev):
    from laprune_amd.retrieval import PLAN_FIELDS
    return torch.tensor([[p[f] for f in PLAN_FIELDS] for p in plans], dtype=torch.int32,
                        device=dev)


@pytest.mark.parametrize("topk,key_dt,per_head,lengths", [
    (2048, torch.float16, False, "short"),
    (None, torch.bfloat16, False, "short"),
    (2048, torch.float16, True, "short"),    # one top-k per query head (row kernel)
    (None, torch.bfloat16, True, "long"),    # ... rows past 32768 columns (chunked levels)
])
def test_retrieve_topk_ragged(dev, orc, topk, key_dt, per_head, lengths):
    """Per-sequence windows and budgets; short rows pad with -1; a sequence
    with no codes selects nothing."""
    from laprune_amd import _native as N
    from laprune_amd.aq_kernels import aq_lut_build
    g = _gen(300 + (topk or 0) + 7 * per_head)
    Hkv, Hq, cap = 8, 32, 64
    if lengths == "short":
        t_codes = [5000, 1300, 9000, 0]
        t_total = [5000, 1337, 9010, 40]
    else:
        t_codes = [40000, 33000, 0]
        t_total = [40030, 33000, 12]
    B, T = len(t_codes), max(t_codes)
    rows = Hq if per_head else Hkv
    q = torch.randn(B * Hq, 128, generator=g).bfloat16()
    cb = torch.randn(32, 256, 128, generator=g) * 0.02
    buf = torch.randint(0, 256, (B, Hkv, T + cap, 32), generator=g, dtype=torch.uint8)
    codes = buf.to(dev)[:, :, :T]
    lut = aq_lut_build(q.to(dev), cb.to(dev), G=4, layout="gmkg")
    plans = [_plan(orc, tc, tt, topk) for tc, tt in zip(t_codes, t_total)]
    k_cols = max(p["k"] for p in plans)
    out = torch.full((B, rows, k_cols), -7, dtype=torch.int32, device=dev)
    ws = torch.empty(N.size_query("lap_retrieve_workspace_size", B * rows, T), dtype=torch.uint8,
                     device=dev)
    kmode = N.KEY_BF16 if key_dt == torch.bfloat16 else N.KEY_F16
    if per_head:
        kmode |= N.SELECT_PER_HEAD
    pd = _plans_dev(plans, dev)
    N.call("lap_retrieve_topk_ragged", N.ptr(lut), N.ptr(codes), codes.stride(0), codes.stride(1),
           codes.stride(2), B, Hkv, T, N.ptr(pd), k_cols, kmode, None, N.ptr(out), N.I32,
           N.ptr(ws), ws.numel(), N.stream_of(out))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    lut_hmk = orc.lut_build(q.float().numpy(), cb.numpy())
    for b, p in enumerate(plans):
        kb = p["k"]
        assert np.all(got[b, :, kb:] == -1), b
        if kb == 0:
            continue
        s = orc.score_grouped(lut_hmk[b * Hq:(b + 1) * Hq], buf[b, :, :p["t_codes"]].numpy(), 4)
        want = orc.topk(s, kb, 1 if per_head else 4, p["cand_start"], p["cand_end"],
                        key_bf16=key_dt == torch.bfloat16)
        assert np.array_equal(got[b, :, :kb].astype(np.int64), want), b


def test_topk_select_ragged_per_head(dev, orc):
    """Per-head selection over fp16 scores with many ties, one plan per
    sequence of four rows."""
    from laprune_amd import _native as N
    g = _gen(310)
    B, Hq, T = 3, 4, 3000
    s = (torch.randn(B * Hq, T, generator=g) * 3).round().half() / 4
    plans = [_plan(orc, 3000, 3000, 700), _plan(orc, 900, 950, 700), _plan(orc, 70, 70, 700)]
    k_cols = max(p["k"] for p in plans)
    out = torch.full((B * Hq, k_cols), -7, dtype=torch.int64, device=dev)
    ws = torch.empty(N.size_query("lap_topk_workspace_size", B * Hq, T), dtype=torch.uint8,
                     device=dev)
    sd = s.to(dev)
    pd = _plans_dev(plans, dev)
    N.call("lap_topk_select_ragged", N.ptr(sd), T, B * Hq, 1, Hq, T, N.ptr(pd), k_cols,
           N.KEY_F16, N.ptr(out), N.I64, N.ptr(ws), ws.numel(), N.stream_of(out))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    bits = _np_u16(s)
    for r in range(B * Hq):
        p = plans[r // Hq]
        kb = p["k"]
        want = orc.topk(bits[r:r + 1], kb, 1, p["cand_start"], p["cand_end"])
        assert np.array_equal(got[r, :kb], want[0]), r
        assert np.all(got[r, kb:] == -1), r


@pytest.mark.parametrize("per_head", [False, True])
def test_sparse_attn_ragged(dev, orc, per_head):
    """Each sequence attends over its own indices (padded with -1), sinks and
    tail, bounded by its own length."""
    from laprune_amd import _native as N
    g = _gen(320 + per_head)
    B, Hq, Hkv, D = 3, 32, 8, 128
    t_total = [3000, 1500, 50]
    T = max(t_total) + 16
    q = torch.randn(B, Hq, 1, D, generator=g).bfloat16()
    kk = torch.randn(B, Hkv, T, D, generator=g).bfloat16()
    vv = torch.randn(B, Hkv, T, D, generator=g).bfloat16()
    plans = [_plan(orc, tt, tt, None) for tt in t_total]
    k_cols = max(p["k"] for p in plans)
    H_idx = Hq if per_head else Hkv
    idx = torch.full((B, H_idx, k_cols), -1, dtype=torch.int32)
    for b, p in enumerate(plans):
        for r in range(H_idx):
            pick = torch.randperm(p["cand_end"] - p["cand_start"], generator=g)[:p["k"]]
            idx[b, r, :p["k"]] = torch.sort(pick + p["cand_start"]).values.to(torch.int32)
    pd = _plans_dev(plans, dev)
    max_sink = max(p["sink"] for p in plans)
    max_tail = max(p["tail_count"] for p in plans)
    out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=dev)
    ws = torch.zeros(N.size_query("lap_attn_decode_workspace_size", B, Hq, D,
                                  k_cols + max_sink + max_tail), dtype=torch.uint8, device=dev)
    qd, kd, vd, idd = q.to(dev), kk.to(dev), vv.to(dev), idx.to(dev)
    N.call("lap_sparse_attn_decode_ragged", N.ptr(qd), qd.stride(0), qd.stride(1), N.ptr(kd),
           N.ptr(vd), N.BF16, B, Hq, Hkv, T, D, kd.stride(0), kd.stride(1), kd.stride(2),
           vd.stride(0), vd.stride(1), vd.stride(2), N.ptr(idd), N.I32, H_idx, k_cols, N.ptr(pd),
           max_sink, max_tail, 1.0 / math.sqrt(D), N.ptr(out), N.ptr(ws), ws.numel(),
           N.stream_of(out))
    torch.cuda.synchronize()
    G = Hq // Hkv

    def keep(b, h):
        row = idx[b, h if per_head else h // G].numpy()
        return orc.keep_list(row[row >= 0], t_total[b], SINK, LOCAL)

    want = orc.attn_decode_f64(q[:, :, 0].double().numpy(), kk.double().numpy(),
                               vv.double().numpy(), keep)
    assert _rel(out.double().cpu().numpy(), want) < 1e-2


def test_dense_decoder_ragged(dev, orc):
    """The dense comparator with one length per sequence."""
    from laprune_amd.retrieval import DenseDecoder
    g = _gen(330)
    B, Hq, Hkv, D = 3, 32, 8, 128
    lengths = [4000, 17, 2500]
    T = max(lengths)
    q = torch.randn(B, Hq, 1, D, generator=g).bfloat16()
    kk = torch.randn(B, Hkv, T, D, generator=g).bfloat16()
    vv = torch.randn(B, Hkv, T, D, generator=g).bfloat16()
    dd = DenseDecoder(B, Hq, Hkv, D, T, dev)
    out = dd.step(q.to(dev), kk.to(dev), vv.to(dev), lengths=lengths)
    torch.cuda.synchronize()
    want = orc.attn_decode_f64(q[:, :, 0].double().numpy(), kk.double().numpy(),
                               vv.double().numpy(), lambda b, h: np.arange(lengths[b]))
    assert _rel(out[:, :, 0].double().cpu().numpy(), want) < 1e-2


@pytest.mark.parametrize("select", ["group", "head"])
def test_sparse_decoder_ragged_matches_each_sequence_alone(dev, orc, select):
    """A ragged step selects, per sequence, exactly what a batch-1 step over
    that sequence selects; its output matches float64 over that keep set."""
    from laprune_amd.retrieval import RetrievalConfig, SparseDecoder
    g = _gen(340 + len(select))
    Hq, Hkv, D = 32, 8, 128
    t_total = [6000, 2100, 4100]
    t_codes = [5952, 2048, 4096]
    B, T = len(t_total), max(t_total)
    cb = (torch.randn(32, 256, D, generator=g) * 0.02).to(dev)
    codes = torch.randint(0, 256, (B, Hkv, T, 32), generator=g, dtype=torch.uint8).to(dev)
    kk = torch.randn(B, Hkv, T, D, generator=g).bfloat16().to(dev)
    vv = torch.randn(B, Hkv, T, D, generator=g).bfloat16().to(dev)
    q = torch.randn(B, Hq, 1, D, generator=g).bfloat16().to(dev)
    cfg = RetrievalConfig(topk=512 if select == "group" else None, select=select)
    dec = SparseDecoder(cb, B, Hq, Hkv, D, T, cfg)
    out = dec.step(q, codes, kk, vv, t_codes=t_codes, t_total=t_total).clone()
    sel = dec.selected().cpu().numpy()
    one = SparseDecoder(cb, 1, Hq, Hkv, D, T, cfg)
    G = Hq // Hkv
    for b in range(B):
        one.step(q[b:b + 1], codes[b:b + 1], kk[b:b + 1], vv[b:b + 1], t_codes=t_codes[b],
                 t_total=t_total[b])
        alone = one.selected().cpu().numpy()[0]
        kb = alone.shape[-1]
        assert np.array_equal(sel[b, :, :kb], alone), b
        assert np.all(sel[b, :, kb:] == -1), b

        def keep(bb, h, b=b):
            row = sel[b, h if select == "head" else h // G]
            return orc.keep_list(row[row >= 0], t_total[b], SINK, LOCAL)

        want = orc.attn_decode_f64(q[b:b + 1, :, 0].double().cpu().numpy(),
                                   kk[b:b + 1].double().cpu().numpy(),
                                   vv[b:b + 1].double().cpu().numpy(), keep)
        assert _rel(out[b:b + 1, :, 0].double().cpu().numpy(), want) < 1e-2, b


def test_sparse_decoder_head_mode_selection(dev, orc):
    """Per-head selection with batch 2 and fewer codes than the decoder's
    capacity: indices bit-exact against the oracle per query head."""
    from laprune_amd.retrieval import RetrievalConfig, SparseDecoder
    g = _gen(350)
    B, Hq, Hkv, D = 2, 32, 8, 128
    T_max, tc, tt = 8192, 5000, 5030
    cb = torch.randn(32, 256, D, generator=g) * 0.02
    codes = torch.randint(0, 256, (B, Hkv, T_max, 32), generator=g, dtype=torch.uint8)
    kk = torch.randn(B, Hkv, T_max, D, generator=g).bfloat16().to(dev)
    vv = torch.randn(B, Hkv, T_max, D, generator=g).bfloat16().to(dev)
    q = torch.randn(B, Hq, 1, D, generator=g).bfloat16()
    dec = SparseDecoder(cb.to(dev), B, Hq, Hkv, D, T_max, RetrievalConfig(select="head"))
    dec.step(q.to(dev), codes.to(dev), kk, vv, t_codes=tc, t_total=tt)
    torch.cuda.synchronize()
    sel = dec.selected().cpu().numpy()
    p = _plan(orc, tc, tt, None)
    assert sel.shape == (B, Hq, p["k"])
    lut = orc.lut_build(q[:, :, 0].reshape(B * Hq, D).float().numpy(), cb.numpy())
    for b in range(B):
        s = orc.score_grouped(lut[b * Hq:(b + 1) * Hq], codes[b, :, :tc].numpy(), 4)
        want = orc.topk(s, p["k"], 1, p["cand_start"], p["cand_end"])
        assert np.array_equal(sel[b].astype(np.int64), want), b


def test_ragged_cache_flushes_per_sequence(dev, orc):
    """Sequences prefilled to different lengths, then grown one token at a
    time: each flushes its own 64-token buffer, keys land at each sequence's
    end, and codes are exact."""
    from laprune_amd.cache import DecodeKVCache, flush_range
    g = _gen(360)
    B, H, D, M = 3, 2, 128, 32
    pre = [300, 100, 250]
    steps = 90
    cb = torch.randn(M, 256, D, generator=g) * 0.02
    cache = DecodeKVCache(cb.to(dev), B, H, D, capacity=128, group_size=64)
    ks = [(torch.randn(1, H, pre[b] + steps, D, generator=g) * 1.5).bfloat16() for b in range(B)]
    vs = [torch.randn(1, H, pre[b] + steps, D, generator=g).bfloat16() for b in range(B)]
    for b in range(B):
        cache.append_row(b, ks[b][:, :, :pre[b]].to(dev), vs[b][:, :, :pre[b]].to(dev))
    assert cache.lengths == pre and cache.encoded_lens == pre and cache.ragged
    enc = list(pre)
    for i in range(steps):
        kn = torch.cat([ks[b][:, :, pre[b] + i:pre[b] + i + 1] for b in range(B)]).to(dev)
        vn = torch.cat([vs[b][:, :, pre[b] + i:pre[b] + i + 1] for b in range(B)]).to(dev)
        cache.append(kn, vn)
        for b in range(B):
            rng = flush_range(pre[b] + i + 1, enc[b], 64, False)
            if rng is not None:
                enc[b] = rng[1]
        assert cache.encoded_lens == enc
    torch.cuda.synchronize()
    assert cache.lengths == [p + steps for p in pre]
    for b in range(B):
        n, e = cache.lengths[b], cache.encoded_lens[b]
        assert torch.equal(cache.k[b, :, :n].cpu(), ks[b][0])
        assert torch.equal(cache.v[b, :, :n].cpu(), vs[b][0])
        want, _ = orc.encode(ks[b][0, :, :e].float().reshape(-1, D).numpy(), cb.numpy())
        got = cache.codes[b, :, :e].reshape(-1, M).cpu().numpy()
        assert np.array_equal(got, want), b


def test_encode_keys_ranges_per_sequence(dev, orc):
    """Per-sequence device ranges: codes inside each range are exact, every
    other code byte is untouched (an empty range and a partial one)."""
    from laprune_amd import _native as N
    from laprune_amd.aq_kernels import aq_encode_prepare
    g = torch.Generator().manual_seed(370)
    B, H, T, D, M = 3, 2, 300, 128, 32
    keys = (torch.randn(B, H, T, D, generator=g) * 1.3).bfloat16()
    cb = torch.randn(M, 256, D, generator=g) * 0.02
    # the last range runs past the buffers' capacity T + 16 and is clipped there
    ranges = torch.tensor([[10, 74], [0, 0], [100, 137]], dtype=torch.int32)
    ranges_clip = torch.tensor([[10, 74], [0, 0], [290, 350]], dtype=torch.int32)
    kd, cbd = keys.to(dev), cb.to(dev)
    prep = aq_encode_prepare(cbd)
    codes = torch.full((B, H, T + 16, M), 0xAB, dtype=torch.uint8, device=dev)
    rd = ranges.to(dev)
    N.call("lap_encode_keys_ranges", N.ptr(kd), N.BF16, kd.stride(0), kd.stride(1), kd.stride(2),
           B, H, N.ptr(rd), 64, T, D, N.ptr(cbd), M, 256, N.ptr(prep), prep.numel(),
           N.ptr(codes), codes.stride(0), codes.stride(1), codes.stride(2), N.stream_of(codes))
    torch.cuda.synchronize()
    got = codes.cpu().numpy()
    # clipping: keys hold T tokens, so [290, 350) encodes 290..299 only
    codes2 = torch.full_like(codes, 0xAB)
    rc = ranges_clip.to(dev)
    N.call("lap_encode_keys_ranges", N.ptr(kd), N.BF16, kd.stride(0), kd.stride(1), kd.stride(2),
           B, H, N.ptr(rc), 64, T, D, N.ptr(cbd), M, 256, N.ptr(prep), prep.numel(),
           N.ptr(codes2), codes2.stride(0), codes2.stride(1), codes2.stride(2),
           N.stream_of(codes2))
    torch.cuda.synchronize()
    got2 = codes2.cpu().numpy()
    want2, _ = orc.encode(keys[2, 0, 290:300].float().numpy(), cb.numpy())
    assert np.array_equal(got2[2, 0, 290:300], want2)
    assert np.all(got2[2, :, 300:] == 0xAB) and np.all(got2[2, :, :290] == 0xAB)
    for b in range(B):
        t0, t1 = (int(x) for x in ranges[b])
        for h in range(H):
            if t1 > t0:
                want, _ = orc.encode(keys[b, h, t0:t1].float().numpy(), cb.numpy())
                assert np.array_equal(got[b, h, t0:t1], want), (b, h)
            outside = np.concatenate([got[b, h, :t0], got[b, h, t1:]])
            assert np.all(outside == 0xAB), (b, h)


def test_empty_keep_set_attends_newest_token(dev):
    """No candidates (nothing encoded yet), no sink and no local window: the
    reference keeps token T_total - 1 (aq_evaluation.py:233-234), so every
    head's output is that token's V row.  Uniform, ragged and device-plan
    steps."""
    from laprune_amd.retrieval import PLAN_FIELDS, RetrievalConfig, SparseDecoder
    g = _gen(380)
    B, Hq, Hkv, D, T = 2, 32, 8, 128, 96
    cb = (torch.randn(32, 256, D, generator=g) * 0.02).to(dev)
    codes = torch.zeros(B, Hkv, T, 32, dtype=torch.uint8, device=dev)
    kk = torch.randn(B, Hkv, T, D, generator=g).bfloat16().to(dev)
    vv = torch.randn(B, Hkv, T, D, generator=g).bfloat16().to(dev)
    q = torch.randn(B, Hq, 1, D, generator=g).bfloat16().to(dev)
    dec = SparseDecoder(cb, B, Hq, Hkv, D, T, RetrievalConfig(sink_size=0, local_window=0))

    def newest(lengths):
        rows = torch.stack([vv[b, :, n - 1] for b, n in enumerate(lengths)])  # [B, Hkv, D]
        return rows.repeat_interleave(Hq // Hkv, dim=1)

    out = dec.step(q, codes[:, :, :0], kk[:, :, :80], vv[:, :, :80], t_codes=0, t_total=80)
    assert torch.equal(out[:, :, 0], newest([80, 80]))
    lens = [50, 70]
    out = dec.step(q, codes, kk, vv, t_codes=[0, 0], t_total=lens)
    assert torch.equal(out[:, :, 0], newest(lens))
    plans = torch.tensor([[p[f] for f in PLAN_FIELDS] for p in dec.row_plans([0, 0], lens)],
                         dtype=torch.int32, device=dev)
    out = dec.step_dev(q, codes, kk, vv, plans)
    assert torch.equal(out[:, :, 0], newest(lens))
