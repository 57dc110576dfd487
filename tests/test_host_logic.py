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
