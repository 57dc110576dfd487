"""The one-launch decode step (lap_decode_step) on the GPU, with group
selection (top-k of the group max) and with the reference's per-head
selection (each query head's own top-k, aq_evaluation.py:185-205).

Every case checks the selected indices bit for bit against the oracle's
top-k of the oracle's scores,
the attention output within 1e-2 of float64 softmax over the keep set
(:210-251), and that the step's health counters stay zero (no workgroup ran
off its row's XCD, no barrier gave up).  Shapes cover the C2 size (131072
columns, 32 workgroups per KV row), rows served by one workgroup (no split
merge), chunks of one to eight tokens per thread, two rows per XCD (B = 2),
fp16 and bf16, all-equal scores (ties: lowest columns win), keep-everything
budgets, ragged device plans and graph replays with rewritten plans; B = 16
at 32768 columns takes two workgroups per row and 16 tokens per thread.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SINK, LOCAL = 4, 64
Hq, Hkv, D = 32, 8, 128


def _rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-6))


def _inputs(seed, B, T, dt, zero_codes=False, dev=None):
    g = torch.Generator().manual_seed(seed)
    cb = torch.randn(32, 256, D, generator=g) * 0.02
    if zero_codes:
        codes = torch.zeros(B, Hkv, T, 32, dtype=torch.uint8)
    else:
        codes = torch.randint(0, 256, (B, Hkv, T, 32), generator=g, dtype=torch.uint8)
    q = torch.randn(B, Hq, 1, D, generator=g).to(dt)
    gd = torch.Generator(device=dev).manual_seed(seed + 1)
    kk = torch.randn((B, Hkv, T, D), generator=gd, device=dev).to(dt)
    vv = torch.randn((B, Hkv, T, D), generator=gd, device=dev).to(dt)
    return cb, codes, kk, vv, q


def _want_idx(orc, cb, codes_b, q_b, plan, key_bf16, per_head=False):
    lut = orc.lut_build(q_b.float().numpy(), cb.numpy())
    s = orc.score_grouped(lut, codes_b[:, :plan["t_codes"]].numpy(), 4)
    return orc.topk(s, plan["k"], 1 if per_head else 4, plan["cand_start"], plan["cand_end"],
                    key_bf16=key_bf16)


def _check_attn(orc, out, q, kk, vv, want_b, b, t_total, per_head=False):
    def keep(bb, h):
        return orc.keep_list(want_b[h if per_head else h // 4], t_total, SINK, LOCAL)

    ref = orc.attn_decode_f64(q[b:b + 1, :, 0].double().numpy(),
                              kk[b:b + 1, :, :t_total].double().cpu().numpy(),
                              vv[b:b + 1, :, :t_total].double().cpu().numpy(), keep)
    got = out[b:b + 1, :, 0].double().cpu().numpy()
    assert _rel(got, ref) < 1e-2, b


def _decoder(cb, dev, B, T, dt, key_dt, topk=None, mask_out=0.98, select="group"):
    from laprune_amd.retrieval import RetrievalConfig, SparseDecoder
    cfg = RetrievalConfig(topk=topk, mask_out=mask_out, sink_size=SINK, local_window=LOCAL,
                          select=select, score_dtype=key_dt)
    return SparseDecoder(cb.to(dev), B, Hq, Hkv, D, T, cfg, dtype=dt)


@pytest.mark.parametrize("B,T,tc,dt,key_dt,topk,zero,select", [
    (1, 131072, 131072, torch.bfloat16, torch.bfloat16, 2048, False, "group"),  # C2: 32 x 4096
    (1, 131072, 131008, torch.bfloat16, torch.bfloat16, None, False, "group"),  # budget 2621
    (1, 131072, 131072, torch.float16, torch.float16, 2048, True, "group"),     # all ties
    (1, 40003, 39936, torch.bfloat16, torch.float16, 700, False, "group"),  # partial last chunk
    (1, 300, 256, torch.bfloat16, torch.bfloat16, 16, False, "group"),      # one workgroup per row
    (1, 8192, 8192, torch.float16, torch.bfloat16, None, False, "group"),   # C1 size: 8 x 1024
    (2, 131072, 131072, torch.bfloat16, torch.bfloat16, 2048, False, "group"),  # 2 rows per XCD
    (16, 32768, 32768, torch.bfloat16, torch.bfloat16, 1024, False, "group"),  # 16 tokens/thread
    # per-head selection (the reference's rule)
    (1, 131072, 131008, torch.bfloat16, torch.bfloat16, None, False, "head"),  # k = 2621
    (1, 131072, 131072, torch.bfloat16, torch.bfloat16, 2048, False, "head"),
    (1, 131072, 131072, torch.float16, torch.float16, 2048, True, "head"),     # all ties
    (1, 40003, 39936, torch.bfloat16, torch.float16, 700, False, "head"),
    (1, 300, 256, torch.bfloat16, torch.bfloat16, 16, False, "head"),
    (1, 8192, 8192, torch.float16, torch.bfloat16, None, False, "head"),       # C1: k = 163
    (2, 131072, 131072, torch.bfloat16, torch.bfloat16, 2048, False, "head"),
])
def test_step_uniform(dev, orc, B, T, tc, dt, key_dt, topk, zero, select):
    per_head = select == "head"
    cb, codes, kk, vv, q = _inputs(700 + T % 997 + B + 3 * per_head, B, T, dt, zero, dev)
    dec = _decoder(cb, dev, B, T, dt, key_dt, topk, select=select)
    out = dec.step(q.to(dev), codes.to(dev)[:, :, :tc], kk, vv, t_codes=tc, t_total=T).clone()
    sel = dec.selected().cpu().numpy()
    assert sel.shape[1] == (Hq if per_head else Hkv)
    p = dict(t_codes=tc, **dec.plan(tc, T))
    for b in range(B):
        want = _want_idx(orc, cb, codes[b], q[b, :, 0], p, key_dt == torch.bfloat16, per_head)
        assert np.array_equal(sel[b].astype(np.int64), want), b
        _check_attn(orc, out, q, kk, vv, want, b, T, per_head)
    assert dec.fused_status() == (0, 0)


@pytest.mark.parametrize("select", ["group", "head"])
def test_step_keep_everything(dev, orc, select):
    """mask_out = 0: every candidate is selected, so the step is dense
    attention over the whole cache (a 131007-entry selection per row)."""
    T = 131072
    cb, codes, kk, vv, q = _inputs(720, 1, T, torch.bfloat16, dev=dev)
    dec = _decoder(cb, dev, 1, T, torch.bfloat16, torch.bfloat16, None, mask_out=0.0,
                   select=select)
    tc = T - 1
    out = dec.step(q.to(dev), codes.to(dev)[:, :, :tc], kk, vv, t_codes=tc, t_total=T).clone()
    p = dec.plan(tc, T)
    sel = dec.selected().cpu().numpy()
    want = np.tile(np.arange(p["cand_start"], p["cand_end"]), (Hq if select == "head" else Hkv, 1))
    assert np.array_equal(sel[0].astype(np.int64), want)
    ref = orc.attn_decode_f64(q[:, :, 0].double().numpy(), kk.double().cpu().numpy(),
                              vv.double().cpu().numpy(), lambda b, h: np.arange(T))
    assert _rel(out[:, :, 0].double().cpu().numpy(), ref) < 1e-2
    assert dec.fused_status() == (0, 0)


@pytest.mark.parametrize("select", ["group", "head"])
def test_step_ragged_plans_and_graph(dev, orc, select):
    """B = 2 ragged lengths through device plans (fixed launch arguments),
    eager and replayed from a captured graph, then replayed again after the
    host rewrites the plans."""
    from laprune_amd.retrieval import PLAN_FIELDS
    B, T = 2, 65536
    per_head = select == "head"
    cb, codes, kk, vv, q = _inputs(730 + per_head, B, T, torch.bfloat16, dev=dev)
    dec = _decoder(cb, dev, B, T, torch.bfloat16, torch.bfloat16, 1024, select=select)
    qd, cd = q.to(dev), codes.to(dev)

    def run_plans(t_total):
        t_codes = [t - t % 64 for t in t_total]
        plans = dec.row_plans(t_codes, t_total)
        return plans, torch.tensor([[p[f] for f in PLAN_FIELDS] for p in plans],
                                   dtype=torch.int32)

    def check(plans, t_total, out):
        idx = dec.idx.cpu().numpy()
        for b, p in enumerate(plans):
            want = _want_idx(orc, cb, codes[b], q[b, :, 0], p, True, per_head)
            assert np.array_equal(idx[b, :, :p["k"]].astype(np.int64), want), b
            assert np.all(idx[b, :, p["k"]:dec.k_cols] == -1), b
            _check_attn(orc, out, q, kk, vv, want, b, t_total[b], per_head)

    t1 = [65536, 40001]
    plans1, pd1 = run_plans(t1)
    pdev = pd1.to(dev)
    out = dec.step_dev(qd, cd, kk, vv, pdev).clone()
    check(plans1, t1, out)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        dec.step_dev(qd, cd, kk, vv, pdev)
    torch.cuda.current_stream(dev).wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out_g = dec.step_dev(qd, cd, kk, vv, pdev)
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        check(plans1, t1, out_g.clone())
        dec.step(qd, cd, kk, vv, t_codes=[t - t % 64 for t in t1], t_total=t1)  # eager between
        torch.cuda.synchronize()
    t2 = [33000, 65000]
    plans2, pd2 = run_plans(t2)
    pdev.copy_(pd2)
    g.replay()
    torch.cuda.synchronize()
    check(plans2, t2, out_g.clone())
    assert dec.fused_status() == (0, 0)
