"""Host-side selection arithmetic of laprune_amd.retrieval against the oracle's
restatement of aq_evaluation.py:185-237 and closed forms."""
import os

import numpy as np
import pytest
import torch

from laprune_amd import retrieval as R
from oracle import orc


@pytest.mark.parametrize("t", [0, 1, 3, 50, 64, 65, 68, 1000, 8192, 131072])
@pytest.mark.parametrize("sink,local", [(4, 64), (0, 64), (4, 0), (0, 0), (128, 16)])
def test_window_budget_keep(t, sink, local):
    assert R.candidate_window(t, t, sink, local) == orc.candidate_window(t, t, sink, local)
    cs, ce = R.candidate_window(t, t, sink, local)
    n = ce - cs
    assert R.budget_k(n, 0.98, 20) == orc.budget_k(n)
    sb, start, tail = R.keep_plan(0, t, sink, local)
    keep = orc.keep_list(np.zeros(0, np.int64), t, sink, local)
    assert keep.tolist() == list(range(sb)) + list(range(start, start + tail))


def test_empty_keep_set_keeps_newest_token():
    """No candidate selected, no sink and no local window: the reference
    keeps token T_total - 1 (aq_evaluation.py:233-234); selecting something
    or having either window disables the fallback."""
    for t in (1, 2, 100, 131072):
        assert R.keep_plan(0, t, 0, 0) == (0, t - 1, 1)
        assert orc.keep_list(np.zeros(0, np.int64), t, 0, 0).tolist() == [t - 1]
        assert R.keep_plan(5, t, 0, 0) == (0, t, 0)
        assert orc.keep_list(np.array([0]), t, 0, 0).tolist() == [0]
    assert R.keep_plan(0, 0, 0, 0) == (0, 0, 0)
    assert R.keep_plan(0, 100, 4, 0) == (4, 100, 0)
    assert R.keep_plan(0, 100, 0, 8) == (0, 92, 8)


def _tiny_attention(bias: bool):
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaAttention
    cfg = LlamaConfig(hidden_size=64, num_attention_heads=4, num_key_value_heads=2, head_dim=16,
                      attention_bias=bias)
    torch.manual_seed(3)
    attn = LlamaAttention(cfg, layer_idx=0)
    with torch.no_grad():
        for p in attn.parameters():
            p.normal_()
    return attn


@pytest.mark.parametrize("bias", [False, True])
def test_fused_qkv_projection(bias):
    """The fused [q; k; v] GEMV equals the three module projections, with and
    without biases, and is fused again when the parameters are replaced
    (model.to(dtype) after wrapping)."""
    from laprune_amd.llama import LAPruneLlama
    attn = _tiny_attention(bias)
    h = torch.randn(2, 3, 64)
    want = [attn.q_proj(h), attn.k_proj(h), attn.v_proj(h)]
    LAPruneLlama._fuse_qkv(attn)
    w, b, sizes = attn._lap_qkv
    assert sizes == [64, 32, 32] and (b is not None) == bias
    got = LAPruneLlama._project(attn, h)
    for g_, w_ in zip(got, want):
        torch.testing.assert_close(g_, w_, rtol=0, atol=1e-5)
    assert LAPruneLlama._fused_current(attn)
    attn.to(torch.float64)  # replaces every parameter
    assert not LAPruneLlama._fused_current(attn)
    h64 = h.double()
    got = LAPruneLlama._project(attn, h64)
    assert attn._lap_qkv[0].dtype == torch.float64 and LAPruneLlama._fused_current(attn)
    for g_, w_ in zip(got, want):
        torch.testing.assert_close(g_.float(), w_, rtol=0, atol=1e-4)


def test_fused_qkv_mixed_bias_falls_back():
    from laprune_amd.llama import LAPruneLlama
    attn = _tiny_attention(True)
    attn.k_proj.bias = None
    h = torch.randn(1, 2, 64)
    want = [attn.q_proj(h), attn.k_proj(h), attn.v_proj(h)]
    LAPruneLlama._fuse_qkv(attn)
    assert attn._lap_qkv is None
    for g_, w_ in zip(LAPruneLlama._project(attn, h), want):
        assert torch.equal(g_, w_)


def test_keep_parts_are_disjoint_from_candidates():
    for t in (100, 1000, 131072):
        cs, ce = R.candidate_window(t, t, 4, 64)
        sb, start, tail = R.keep_segments(t, 4, 64)
        assert sb <= cs and ce <= start and start + tail == t


def test_unencoded_tail_stays_in_local_window():
    """aq_decode_group_size=64 leaves <= 63 keys unencoded; with local_window=64 they
    are never candidates (aq_evaluation.py:189-192, :370-374)."""
    for total in range(4096, 4096 + 64):
        encoded = total - ((total - 4096) % 64)
        cs, ce = R.candidate_window(encoded, total, 0, 64)
        assert ce <= encoded and ce == min(encoded, total - 64)


def test_config_validation():
    with pytest.raises(ValueError):
        R.RetrievalConfig(select="other")
    c = R.RetrievalConfig()
    assert (c.mask_out, c.min_remain, c.sink_size, c.local_window) == (0.98, 20, 4, 64)


def test_decoder_requires_native_or_gpu():
    cb = torch.zeros(32, 256, 128)
    with pytest.raises(RuntimeError):
        R.SparseDecoder(cb, 1, 32, 8, 128, 1024)


# ------------------------------------------------- decode caches (host policy)
from laprune_amd import cache as KC


def test_flush_range_policy():
    """Encode when >= group_size keys are pending in decode; always in prefill
    (aq_evaluation.py:369-382, :430-447)."""
    assert KC.flush_range(100, 0, 64, prefill=True) == (0, 100)
    assert KC.flush_range(100, 64, 64, prefill=False) is None      # 36 pending
    assert KC.flush_range(128, 64, 64, prefill=False) == (64, 128)  # 64 pending
    assert KC.flush_range(64, 64, 64, prefill=False) is None        # nothing pending
    assert KC.flush_range(65, 64, 1, prefill=False) == (64, 65)     # group 1: every token
    assert KC.flush_range(70, 64, 64, prefill=True) == (64, 70)


def test_flush_sequence_matches_reference_rule():
    """Prefill 300 keys, then decode one at a time: encodes happen exactly when
    the pending tail reaches 64, and the tail never exceeds 63 keys after a step."""
    length, enc = 300, 0
    rng = KC.flush_range(length, enc, 64, prefill=True)
    enc = rng[1]
    flushes = []
    for _ in range(200):
        length += 1
        rng = KC.flush_range(length, enc, 64, prefill=False)
        if rng is not None:
            assert rng == (enc, length) and length - enc == 64
            flushes.append(length)
            enc = length
        assert 0 <= length - enc <= 63
    assert flushes == [364, 428, 492]


def test_grown_capacity():
    assert KC.grown_capacity(16, 17) == 32
    assert KC.grown_capacity(16, 100) == 100
    assert KC.grown_capacity(1024, 1025) == 2048


def test_per_row_lengths_argument():
    from laprune_amd.retrieval import _per_row
    assert _per_row(None, 3, "x") is None
    assert _per_row(7, 3, "x") == [7, 7, 7]
    assert _per_row((1, 2, 3), 3, "x") == [1, 2, 3]
    with pytest.raises(RuntimeError, match="one length per sequence"):
        _per_row([1, 2], 3, "x")


def test_plan_fields_match_the_c_struct():
    """PLAN_FIELDS is the field order of lap_row_plan in include/laprune_hip.h."""
    import re
    from pathlib import Path
    from laprune_amd.retrieval import PLAN_FIELDS
    text = (Path(__file__).resolve().parent.parent / "include" / "laprune_hip.h").read_text()
    body = re.search(r"typedef struct lap_row_plan \{(.*?)\} lap_row_plan;", text, re.S).group(1)
    fields = re.findall(r"(\w+)\s*[,;]", body)
    assert tuple(fields) == PLAN_FIELDS


# ------------------------------------------------------------ codebook files

def test_codebook_file_round_trip(tmp_path):
    from laprune_amd import codebooks as CB
    g = torch.Generator().manual_seed(11)
    cb = torch.randn(4, 16, 8, generator=g)
    CB.save_file(str(tmp_path / "layer_3_group_0.pt"), cb, metadata={"target": "key_post_rope"})
    got = CB.load_file(str(tmp_path / "layer_3_group_0.pt"))
    assert (got.layer, got.group, got.M, got.K, got.d) == (3, 0, 4, 16, 8)
    assert torch.equal(got.codebooks, cb) and got.extras["metadata"]["target"] == "key_post_rope"


def test_codebook_dir_rules(tmp_path):
    """Unparsable names are ignored; groups the head grouping cannot use are
    skipped (the reference's rule); a layer filter applies."""
    from laprune_amd import codebooks as CB
    cb = torch.zeros(2, 4, 8)
    for name in ("layer_0_group_0.pt", "layer_0_group_1.pt", "layer_1_group_0.pt",
                 "layer_x_group_0.pt", "notes.txt"):
        CB.save_file(str(tmp_path / name), cb) if name.endswith(".pt") else \
            (tmp_path / name).write_text("x")
    assert sorted(CB.load_dir(str(tmp_path))) == [(0, 0), (0, 1), (1, 0)]
    # 8 KV heads in one group of 8 -> only group 0 is usable
    assert sorted(CB.load_dir(str(tmp_path), num_heads=8, heads_per_group=8)) == [(0, 0), (1, 0)]
    assert sorted(CB.load_dir(str(tmp_path), layers=[1])) == [(1, 0)]
    with pytest.raises(FileNotFoundError):
        CB.load_dir(str(tmp_path / "missing"))


def test_codebook_file_checks(tmp_path):
    from laprune_amd import codebooks as CB
    torch.save({"M": 2, "K": 4, "d": 8, "codebooks": torch.zeros(2, 4, 9)}, tmp_path / "a.pt")
    with pytest.raises(RuntimeError, match="do not match"):
        CB.load_file(str(tmp_path / "a.pt"))
    torch.save({"M": 2, "K": 300, "d": 8, "codebooks": torch.zeros(2, 300, 8)}, tmp_path / "b.pt")
    with pytest.raises(RuntimeError, match="uint8"):
        CB.load_file(str(tmp_path / "b.pt"))
    torch.save({"M": 2, "d": 8, "codebooks": torch.zeros(2, 4, 8)}, tmp_path / "c.pt")
    with pytest.raises(RuntimeError, match="missing 'K'"):
        CB.load_file(str(tmp_path / "c.pt"))


SHIPPED = "/root/reference/codebooks/llama31-8b-instruct"


@pytest.mark.skipif(not os.path.isdir(SHIPPED), reason="reference codebooks not present")
def test_shipped_codebooks_load():
    """The reference's Llama-3.1 files (read only where they exist, never
    copied): 32 layers of [32, 256, 128] float32; layer 0 has std 0.426 and
    absmax 8.82, and its stage norms decay (residual-ordered stages)."""
    from laprune_amd import codebooks as CB
    books = CB.load_dir(SHIPPED, num_heads=8, heads_per_group=8)
    assert len(books) == 32 and all(g == 0 for _, g in books)
    b0 = books[(0, 0)]
    assert (b0.M, b0.K, b0.d) == (32, 256, 128)
    assert abs(b0.codebooks.std().item() - 0.426) < 5e-3
    assert abs(b0.codebooks.abs().max().item() - 8.82) < 1e-2
    stage_norm = b0.codebooks.norm(dim=2).mean(dim=1)
    assert stage_norm[0] > 4 * stage_norm[-1]


def test_step_health_raises_on_nonzero_counters():
    """The one-launch step's two health counters (rows split over XCDs,
    barrier time-outs) turn into StepHealthError naming both counts; zeros
    pass quietly."""
    R.check_step_health(0, 0, "x")
    with pytest.raises(R.StepHealthError, match="2 KV row"):
        R.check_step_health(2, 0, "x")
    with pytest.raises(R.StepHealthError, match="5 row barrier"):
        R.check_step_health(0, 5, "x")
    assert issubclass(R.StepHealthError, RuntimeError)


def test_llama_health_check_names_layers():
    """LAPruneLlama.check_health gathers every LAPrune layer's status words
    (hand-set here in host workspaces) and names the unhealthy layers."""
    import types
    from laprune_amd.llama import LAPruneLlama

    class FakeDec:
        status_words = R.SparseDecoder.status_words

        def __init__(self, split, tmo):
            self.ws = torch.zeros(64, dtype=torch.uint8)
            self.ws[:8].view(torch.int32).copy_(torch.tensor([split, tmo], dtype=torch.int32))

    def st(dec):
        return types.SimpleNamespace(sparse=dec)

    fake = types.SimpleNamespace(states=[st(None), st(FakeDec(0, 0)), st(FakeDec(1, 0)),
                                         st(FakeDec(0, 2))], _since_check=7)
    with pytest.raises(R.StepHealthError) as e:
        LAPruneLlama.check_health(fake)
    msg = str(e.value)
    assert "layers [2, 3]" in msg and "1 KV row" in msg and "2 row barrier" in msg
    assert fake._since_check == 0
    fake.states = [st(None), st(FakeDec(0, 0))]
    LAPruneLlama.check_health(fake)  # healthy: no error
