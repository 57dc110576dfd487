"""The reference's Python boundary: AQLayerCodebookManager (laprune/llm/aq_kv.py)
and do_sdpa_attn (laprune/attention.py), mirrored in laprune_amd.aq_kv and
laprune_amd.attention.

CPU tests: argument rules and errors as the reference raises them, the
codebook directory round trip, and the tail-causal mask against its
definition.  GPU tests: scores bit-exact (fp16 bits) against the oracle's
LUT + grouped / per-head sums, codes bit-exact against the oracle's greedy
encode, and single-query attention through the native decode kernel within
1e-2 of float64.
"""
import math

import numpy as np
import pytest
import torch

from laprune_amd.aq_kv import AQLayerCodebookManager, AQLayerConfig
from laprune_amd.attention import _tail_causal_mask, do_sdpa_attn


def _mgr(device, M=32, K=256, d=128, hpg=8, num_heads=8, layers=(0, 3)):
    return AQLayerCodebookManager({L: AQLayerConfig(M=M, K=K, d=d, heads_per_group=hpg,
                                                    num_heads=num_heads) for L in layers},
                                  device=device)


# ----------------------------------------------------------------- CPU

def test_do_sdpa_attn_requires_post_rope():
    q = torch.zeros(1, 4, 1, 8)
    with pytest.raises(ValueError, match="post-RoPE"):
        do_sdpa_attn(q, q, q)


def test_do_sdpa_attn_rejects_bad_gqa():
    q = torch.zeros(1, 6, 1, 8)
    k = torch.zeros(1, 4, 5, 8)
    with pytest.raises(ValueError, match="invalid GQA"):
        do_sdpa_attn(q, k, k, already_rope=True)


def test_tail_causal_mask_definition():
    """Query i of nq at the end of nk keys sees keys 0 .. nk - nq + i."""
    nq, nk = 3, 7
    m = _tail_causal_mask(nq, nk, torch.float16, "cpu")[0, 0].float()
    for i in range(nq):
        for j in range(nk):
            visible = j <= nk - nq + i
            assert (m[i, j] == 0) == visible, (i, j)
            if not visible:
                assert m[i, j] == torch.finfo(torch.float16).min
    with pytest.raises(ValueError):
        _tail_causal_mask(8, 7, torch.float16, "cpu")


def test_do_sdpa_attn_cpu_shapes_and_tail_mask():
    """Multi-query prefill over a longer cache equals per-query attention
    over the visible keys (float32 on the CPU, checked in float64)."""
    g = torch.Generator().manual_seed(7)
    B, Hq, Hkv, nq, nk, D = 1, 4, 2, 3, 6, 8
    q = torch.randn(B, Hq, nq, D, generator=g)
    k = torch.randn(B, Hkv, nk, D, generator=g)
    v = torch.randn(B, Hkv, nk, D, generator=g)
    out = do_sdpa_attn(q, k, v, already_rope=True).double()
    assert out.shape == (B, nq, Hq * D)
    q, k, v = q.double(), k.double(), v.double()
    for h in range(Hq):
        kv = h // (Hq // Hkv)
        for i in range(nq):
            vis = nk - nq + i + 1
            s = (q[0, h, i] @ k[0, kv, :vis].T) / math.sqrt(D)
            want = torch.softmax(s, -1) @ v[0, kv, :vis]
            got = out[0, i, h * D:(h + 1) * D]
            assert torch.allclose(got, want, atol=1e-5)


def test_manager_argument_errors():
    m = _mgr("cpu")
    m.set_codebooks(0, 0, torch.zeros(32, 256, 128))
    with pytest.raises(ValueError, match="Invalid GQA"):
        m.approx_inner_product_multihead_gqa(0, torch.zeros(6, 128),
                                             torch.zeros(2, 5, 32, dtype=torch.uint8), 4)
    with pytest.raises(ValueError, match="must be 32"):
        m.approx_inner_product_multihead_gqa(0, torch.zeros(8, 128),
                                             torch.zeros(2, 5, 32, dtype=torch.uint8), 4,
                                             scoring_m=16)
    with pytest.raises(NotImplementedError):
        m.encode_keys_batch(0, 0, torch.zeros(3, 128), icm_iters=2)
    with pytest.raises(ValueError):
        m.set_codebooks(0, 1, torch.zeros(32, 256, 64))
    with pytest.raises(KeyError):
        m.codebooks(3, 0)
    with pytest.raises(NotImplementedError):
        m.fit_layer(0, torch.zeros(3, 128))


def test_manager_load_save_round_trip(tmp_path):
    g = torch.Generator().manual_seed(3)
    src = _mgr("cpu", M=4, K=16, d=8, hpg=4, num_heads=8)
    cbs = {(0, 0): torch.randn(4, 16, 8, generator=g), (0, 1): torch.randn(4, 16, 8, generator=g),
           (3, 0): torch.randn(4, 16, 8, generator=g)}
    for (L, G), cb in cbs.items():
        src.set_codebooks(L, G, cb)
    src.save(str(tmp_path))
    # files the configured grouping cannot use (group 2 of 8 heads / 4 per
    # group), layers not configured and unparsable names are skipped
    torch.save({"M": 4, "K": 16, "d": 8, "codebooks": torch.zeros(4, 16, 8)},
               tmp_path / "layer_0_group_2.pt")
    torch.save({"M": 4, "K": 16, "d": 8, "codebooks": torch.zeros(4, 16, 8)},
               tmp_path / "layer_9_group_0.pt")
    (tmp_path / "notes.txt").write_text("x")
    dst = _mgr("cpu", M=32, K=256, d=128, hpg=4, num_heads=8)
    dst.load(str(tmp_path))
    for key, cb in cbs.items():
        assert torch.equal(dst.codebooks(*key), cb)
    with pytest.raises(KeyError):
        dst.codebooks(0, 2)
    # the file's shape replaces the configured one, grouping is kept
    assert (dst.layer_cfgs[0].M, dst.layer_cfgs[0].K, dst.layer_cfgs[0].d) == (4, 16, 8)
    assert dst.layer_cfgs[0].heads_per_group == 4
    with pytest.raises(FileNotFoundError):
        dst.load(str(tmp_path / "missing"))


# ----------------------------------------------------------------- GPU

@pytest.mark.gpu
@pytest.mark.parametrize("B,G,qdt", [(1, 4, torch.float16), (2, 4, torch.bfloat16),
                                     (1, 2, torch.float32)])
def test_manager_gqa_scores_bit_exact(dev, orc, B, G, qdt):
    g = torch.Generator().manual_seed(500 + B * 10 + G)
    Hkv, T, D = 8, 3000, 128
    cb = torch.randn(32, 256, D, generator=g) * 0.02
    q = torch.randn(B * Hkv * G, D, generator=g).to(qdt)
    codes = torch.randint(0, 256, (B * Hkv, T, 32), generator=g, dtype=torch.uint8)
    m = _mgr(dev)
    m.set_codebooks(0, 0, cb)
    got = m.approx_inner_product_multihead_gqa(0, q.to(dev), codes.to(dev), G)
    assert got.dtype == torch.float16 and got.shape == (B * Hkv * G, T)
    lut = orc.lut_build(q.float().numpy(), cb.numpy())
    want = orc.score_grouped(lut, codes.numpy(), G)
    assert np.array_equal(got.cpu().view(torch.int16).numpy().view(np.uint16), want)


@pytest.mark.gpu
def test_manager_multihead_scores_bit_exact(dev, orc):
    g = torch.Generator().manual_seed(510)
    Q, T, D = 6, 1000, 128
    cb = torch.randn(32, 256, D, generator=g) * 0.02
    q = torch.randn(Q, D, generator=g).half()
    codes = torch.randint(0, 256, (Q, T, 32), generator=g, dtype=torch.uint8)
    m = _mgr(dev)
    m.set_codebooks(0, 0, cb)
    got = m.approx_inner_product_multihead(0, q.to(dev), codes.to(dev))
    lut = orc.lut_build(q.float().numpy(), cb.numpy()).reshape(Q, 32 * 256)
    want = orc.score_mha(lut, codes.numpy(), False)
    assert np.array_equal(got.cpu().view(torch.int16).numpy().view(np.uint16), want)


@pytest.mark.gpu
def test_manager_encode_bit_exact(dev, orc):
    g = torch.Generator().manual_seed(520)
    D = 128
    m = _mgr(dev, hpg=4, num_heads=8)
    cbs = [torch.randn(32, 256, D, generator=g) * 0.02 for _ in range(2)]
    for G, cb in enumerate(cbs):
        m.set_codebooks(3, G, cb)
    x = torch.randn(300, D, generator=g) * torch.empty(D).uniform_(0.5, 4.0, generator=g)
    for head in (1, 6):  # groups 0 and 1
        got = m.encode_keys(3, head, x.to(dev).bfloat16(), icm_iters=0)
        want, _ = orc.encode(x.bfloat16().float().numpy(), cbs[head // 4].numpy())
        assert np.array_equal(got.cpu().numpy(), want), head
    got = m.encode_keys_batch(3, 0, x.to(dev), icm_iters=0)
    assert np.array_equal(got.cpu().numpy(), orc.encode(x.numpy(), cbs[0].numpy())[0])


@pytest.mark.gpu
@pytest.mark.parametrize("dt,Hq,Hkv,T", [(torch.bfloat16, 32, 8, 5000),
                                         (torch.float16, 8, 8, 777)])
def test_do_sdpa_attn_decode_native(dev, orc, dt, Hq, Hkv, T):
    """One query, no mask: the native flash-decode kernel (bit-identical to
    aq_kernels.dense_attn_decode), within 1e-2 of float64 attention."""
    from laprune_amd.aq_kernels import _impl
    g = torch.Generator().manual_seed(530 + Hq)
    B, D = 2, 128
    q = torch.randn(B, Hq, 1, D, generator=g).to(dt)
    k = torch.randn(B, Hkv, T, D, generator=g).to(dt)
    v = torch.randn(B, Hkv, T, D, generator=g).to(dt)
    proj = torch.nn.Linear(Hq * D, 64, bias=False).to(dev, dt)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    out = do_sdpa_attn(qd, kd, vd, already_rope=True)
    assert out.shape == (B, 1, Hq * D)
    direct = _impl.dense_attn_decode(qd, kd, vd)
    assert torch.equal(out, direct.transpose(1, 2).flatten(2))
    want = orc.attn_decode_f64(q[:, :, 0].double().numpy(), k.double().numpy(),
                               v.double().numpy(), lambda b, h: np.arange(T))
    got = out.view(B, Hq, D).double().cpu().numpy()
    assert float(np.abs(got - want).max() / np.abs(want).max()) < 1e-2
    projected = do_sdpa_attn(qd, kd, vd, out_proj=proj, already_rope=True)
    assert torch.equal(projected, proj(out))
