"""Host-side selection arithmetic of laprune_amd.retrieval against the oracle's
restatement of aq_evaluation.py:185-237 and closed forms."""
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
    sb, start, tail = R.keep_segments(t, sink, local)
    keep = orc.keep_list(np.zeros(0, np.int64), t, sink, local)
    assert keep.tolist() == list(range(sb)) + list(range(start, start + tail))


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
