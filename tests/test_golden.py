"""Committed golden fixtures (tests/golden/retrieval_small.npz, written by
tests/golden/make_golden.py from the oracle): the oracle still reproduces them
(CPU) and the gfx950 kernels reproduce them bit for bit (GPU)."""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import orc

GOLD = Path(__file__).resolve().parent / "golden" / "retrieval_small.npz"


@pytest.fixture(scope="module")
def gold():
    return dict(np.load(GOLD, allow_pickle=False))


def _bf16(bits):
    return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16)


def test_oracle_reproduces_golden(gold):
    q = _bf16(gold["q_bf16"]).float().numpy()
    cb = _bf16(gold["cb_bf16"]).float().numpy()
    lut = orc.lut_build(q, cb)
    assert np.array_equal(lut, gold["lut"])
    sc = orc.score_grouped(lut, gold["codes"], 4)
    assert np.array_equal(sc, gold["scores"])
    cs, ce, k = gold["cand"].tolist()
    assert np.array_equal(orc.topk(sc, k, 1, cs, ce), gold["idx_head"])
    assert np.array_equal(orc.topk(sc, 64, 4, cs, ce, key_bf16=True), gold["idx_group"])
    codes, rn = orc.encode(gold["x"], gold["enc_cb"])
    assert np.array_equal(codes, gold["enc_codes"]) and np.array_equal(rn, gold["enc_rnorm"])


@pytest.mark.gpu
def test_gpu_reproduces_golden(dev, gold):
    from laprune_amd import aq_kernels as K
    q = _bf16(gold["q_bf16"]).to(dev)
    cb = _bf16(gold["cb_bf16"]).float().to(dev)
    lut = K.aq_lut_build(q, cb)
    codes = torch.from_numpy(gold["codes"]).to(dev)
    sc = K.aq_lut_gather_grouped(lut, codes, 4)
    cs, ce, k = gold["cand"].tolist()
    ih = K.aq_topk(sc, k, 1, cs, ce)
    ig = K.aq_topk(sc, 64, 4, cs, ce, key_dtype=torch.bfloat16)
    ec, er = K.aq_encode_greedy(torch.from_numpy(gold["x"]).to(dev),
                                torch.from_numpy(gold["enc_cb"]).to(dev))
    torch.cuda.synchronize()
    u16 = lambda t: t.cpu().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    assert np.array_equal(u16(lut), gold["lut"])
    assert np.array_equal(u16(sc), gold["scores"])
    assert np.array_equal(ih.cpu().numpy(), gold["idx_head"])
    assert np.array_equal(ig.cpu().numpy(), gold["idx_group"])
    assert np.array_equal(ec.cpu().numpy(), gold["enc_codes"])
    assert np.array_equal(er.cpu().numpy().view(np.uint32), gold["enc_rnorm"].view(np.uint32))
    # the fused retrieve from the interleaved table: per head and per group
    lut_il = K.aq_lut_build(q, cb, G=4, layout="gmkg")
    c4 = codes.unsqueeze(0)
    fh = K.aq_retrieve_topk(lut_il, c4, k, cs, ce, per_head=True)
    fg = K.aq_retrieve_topk(lut_il, c4, 64, cs, ce, key_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert np.array_equal(fh[0].cpu().numpy().astype(np.int64), gold["idx_head"])
    assert np.array_equal(fg[0].cpu().numpy().astype(np.int64), gold["idx_group"])
