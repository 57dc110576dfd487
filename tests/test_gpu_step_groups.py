"""The decode step (lap_decode_step through SparseDecoder) for G = Hq / Hkv
other than 4 (1, 2, 3, 6, 7 and 8 query heads per KV head), which the
reference's decode path
serves too: its scores come from the GQA gather kernel for any G
(aq_kv.py:684-699 -> aq_kernels/aq_lut_gqa.cu:350-422) before the same
window, budget and torch.topk (aq_evaluation.py:160-205).

Head dim 256 (with G = 4, the fused scorer's chain) is covered here too.
These shapes take the kernel chain: the per-head [B * Hq][32][256] table,
lap_lut_score_gqa of every head, lap_topk_select (_ragged) over the group
max (group selection) or each head's row, then the split-K sparse
attention.  Indices are checked bit for bit against the oracle's top-k of
the oracle's scores and the attention within 1e-2 of float64 softmax over
the keep set (:210-251), uniform and ragged, eager and from a replayed
graph.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SINK, LOCAL, Hkv = 4, 64, 4


def _rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-6))


def _inputs(seed, B, Hq, T, D, dev, dt=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    cb = torch.randn(32, 256, D, generator=g) * 0.02
    codes = torch.randint(0, 256, (B, Hkv, T, 32), generator=g, dtype=torch.uint8)
    q = torch.randn(B, Hq, 1, D, generator=g).to(dt)
    kk = torch.randn(B, Hkv, T, D, generator=g).to(dt).to(dev)
    vv = torch.randn(B, Hkv, T, D, generator=g).to(dt).to(dev)
    return cb, codes, kk, vv, q


def _want_idx(orc, cb, codes_b, q_b, plan, G, per_head, key_bf16=True):
    lut = orc.lut_build(q_b.float().numpy(), cb.numpy())
    s = orc.score_grouped(lut, codes_b[:, :plan["t_codes"]].numpy(), G)
    return orc.topk(s, plan["k"], 1 if per_head else G, plan["cand_start"], plan["cand_end"],
                    key_bf16=key_bf16)


def _check_attn(orc, out, q, kk, vv, want_b, b, t_total, G, per_head):
    def keep(bb, h):
        return orc.keep_list(want_b[h if per_head else h // G], t_total, SINK, LOCAL)

    ref = orc.attn_decode_f64(q[b:b + 1, :, 0].double().numpy(),
                              kk[b:b + 1, :, :t_total].double().cpu().numpy(),
                              vv[b:b + 1, :, :t_total].double().cpu().numpy(), keep)
    assert _rel(out[b:b + 1, :, 0].double().cpu().numpy(), ref) < 1e-2, b


def _decoder(cb, dev, B, Hq, D, T, topk, select, dt=torch.bfloat16, key_dt=torch.bfloat16):
    from laprune_amd.retrieval import RetrievalConfig, SparseDecoder
    cfg = RetrievalConfig(topk=topk, sink_size=SINK, local_window=LOCAL, select=select,
                          score_dtype=key_dt)
    return SparseDecoder(cb.to(dev), B, Hq, Hkv, D, T, cfg, dtype=dt)


@pytest.mark.parametrize("G,D,B,T,topk,select", [
    (1, 128, 1, 8192, None, "group"),   # MHA, reference budget (k = 163)
    (1, 128, 1, 8192, 256, "head"),
    (2, 128, 2, 6000, 300, "group"),
    (2, 64, 1, 4096, None, "head"),
    (8, 128, 1, 8192, 512, "group"),    # Llama-3-70B-like grouping
    (8, 128, 2, 5000, None, "head"),
    (4, 256, 1, 4096, 200, "group"),    # head_dim 256: the chain with the fused scorer
    (2, 256, 1, 4096, None, "head"),
    (7, 128, 2, 6000, 300, "group"),    # Qwen2.5-7B-like grouping (28 q / 4 KV heads)
    (3, 128, 1, 5000, None, "head"),
    (6, 64, 1, 4096, 256, "group"),
])
def test_step_other_groups(dev, orc, G, D, B, T, topk, select):
    per_head = select == "head"
    Hq = Hkv * G
    print(f"group size {G}: D={D} B={B} T={T} topk={topk} {select}", flush=True)
    cb, codes, kk, vv, q = _inputs(900 + 10 * G + B + per_head, B, Hq, T, D, dev)
    dec = _decoder(cb, dev, B, Hq, D, T, topk, select)
    tc = T - T % 64
    out = dec.step(q.to(dev), codes.to(dev), kk, vv, t_codes=tc, t_total=T).clone()
    sel = dec.selected().cpu().numpy()
    assert sel.shape[1] == (Hq if per_head else Hkv)
    p = dict(t_codes=tc, **dec.plan(tc, T))
    for b in range(B):
        want = _want_idx(orc, cb, codes[b], q[b, :, 0], p, G, per_head)
        assert np.array_equal(sel[b].astype(np.int64), want), b
        _check_attn(orc, out, q, kk, vv, want, b, T, G, per_head)


@pytest.mark.parametrize("G,select", [(8, "group"), (2, "head"), (7, "group")])
def test_step_other_groups_ragged_graph(dev, orc, G, select):
    """B = 3 ragged lengths through device plans, eager and replayed from a
    captured graph (twice, with the decoder's eager steps between)."""
    from laprune_amd.retrieval import PLAN_FIELDS
    B, T, D = 3, 9000, 128
    Hq, per_head = Hkv * G, select == "head"
    print(f"group size {G}: ragged B={B} {select}", flush=True)
    cb, codes, kk, vv, q = _inputs(950 + G, B, Hq, T, D, dev)
    dec = _decoder(cb, dev, B, Hq, D, T, 400, select)
    qd, cd = q.to(dev), codes.to(dev)
    t_total = [9000, 5003, 7777]
    t_codes = [t - t % 64 for t in t_total]
    plans = dec.row_plans(t_codes, t_total)
    pdev = torch.tensor([[p[f] for f in PLAN_FIELDS] for p in plans], dtype=torch.int32).to(dev)

    def check(out):
        idx = dec.idx.cpu().numpy()
        for b, p in enumerate(plans):
            want = _want_idx(orc, cb, codes[b], q[b, :, 0], p, G, per_head)
            assert np.array_equal(idx[b, :, :p["k"]].astype(np.int64), want), b
            assert np.all(idx[b, :, p["k"]:dec.k_cols] == -1), b
            _check_attn(orc, out, q, kk, vv, want, b, t_total[b], G, per_head)

    check(dec.step(qd, cd, kk, vv, t_codes=t_codes, t_total=t_total).clone())
    check(dec.step_dev(qd, cd, kk, vv, pdev).clone())
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        dec.step_dev(qd, cd, kk, vv, pdev)
    torch.cuda.current_stream(dev).wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out_g = dec.step_dev(qd, cd, kk, vv, pdev)
    for _ in range(2):
        g.replay()
        torch.cuda.synchronize()
        check(out_g.clone())
        dec.step(qd, cd, kk, vv, t_codes=t_codes, t_total=t_total)
        torch.cuda.synchronize()


@pytest.mark.parametrize("G,select", [(8, "group"), (3, "head")])
def test_step_other_groups_fp16(dev, orc, G, select):
    """fp16 queries, K/V and output with fp16 selection keys."""
    per_head, Hq, B, T, D = select == "head", Hkv * G, 2, 5000, 128
    print(f"group size {G}: fp16 {select}", flush=True)
    cb, codes, kk, vv, q = _inputs(980 + G, B, Hq, T, D, dev, torch.float16)
    dec = _decoder(cb, dev, B, Hq, D, T, 333, select, torch.float16, torch.float16)
    tc = T - T % 64
    out = dec.step(q.to(dev), codes.to(dev), kk, vv, t_codes=tc, t_total=T).clone()
    sel = dec.selected().cpu().numpy()
    p = dict(t_codes=tc, **dec.plan(tc, T))
    for b in range(B):
        want = _want_idx(orc, cb, codes[b], q[b, :, 0], p, G, per_head, key_bf16=False)
        assert np.array_equal(sel[b].astype(np.int64), want), b
        _check_attn(orc, out, q, kk, vv, want, b, T, G, per_head)


def test_step_group_size_refused(dev):
    """More than 8 query heads per KV head exceed the attention kernel's
    16-lane head tile as laid out: the decoder refuses them up front."""
    from laprune_amd.retrieval import SparseDecoder
    cb = torch.zeros(32, 256, 128, device=dev)
    with pytest.raises(RuntimeError, match="G = 1 to 8"):
        SparseDecoder(cb, 1, 48, 4, 128, 1024)
