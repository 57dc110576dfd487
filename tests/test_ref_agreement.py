"""Agreement of the build's arithmetic contract with the reference's own fp32
path at the configs' sizes (CPU only).

The GPU kernels are bit-exact to the oracle (the explicit-order contract:
fp16 table, sequential fp32 sums, fp16 scores, lowest-index ties).  The
reference's CPU path (oracle/ref_path.py restating laprune/llm/aq_kv.py:
614-628, aq_evaluation.py:166, 185-201 and quantizer.py:346-355) scores in
fp32 and breaks ties its own way, so the two selections can differ.  These
tests bound every difference instead of counting an allowance:

* selection (C1 per-head k = 163 and group top-2048 at T = 8192; C2
  per-head k = 2621 at T = 131072; bf16 keys, the model-dtype cast of
  aq_evaluation.py:166): every index in the symmetric difference of the two
  top-k sets has an fp32 score within the error band of the k-th fp32 score.
  The band is what the contract can move a score by: the fp16 rounding of
  the 32 table entries and of the sum, plus one bf16 step on each side of
  the rank key (keys that round to one bf16 value tie, and the two paths
  break ties differently).
* encode (C3: 512 post-RoPE keys): at every stage, with the reference's own
  residual (teacher forcing on its codes), the oracle's argmin equals the
  reference's unless the two candidates' float64 distances differ by less
  than the fp32 error of the two distance formulas.

The counts found are printed (pytest -s) and recorded in the design notes.
"""
import numpy as np
import pytest
import torch

from oracle import orc, ref_path

from _synth import c3_keys, gaussian_codebooks

Hq, Hkv, D, M, K = 32, 8, 128, 32, 256
SINK, LOCAL = 4, 64


def _c_inputs(seed, T):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(Hq, D, generator=g).bfloat16().float()
    cb = gaussian_codebooks(seed + 1)
    codes = torch.randint(0, 256, (Hkv, T, M), generator=g, dtype=torch.uint8)
    return q, cb, codes


def _bf16_ulp(x):
    x = np.maximum(np.abs(x), np.float32(2.0 ** -126))
    return np.exp2(np.floor(np.log2(x)) - 7)


def _ours(q, cb, codes):
    lut = orc.lut_build(q.numpy(), cb.numpy())  # fp16 bits [Hq, M, K]
    heads = orc.score_grouped(lut, codes.numpy(), 4)  # fp16 bits [Hq, T]
    lut_abs = float(np.abs(orc.h_vals(lut.reshape(-1))).max())
    return heads, lut_abs


def _check_band(ref_rows, mine_sets, k, lut_abs):
    """ref_rows [R, n] fp32 scores over the candidate window; mine_sets: sets
    of window-relative indices.  Returns (differing, bf16 ties)."""
    differing = ties = 0
    for r, mine in enumerate(mine_sets):
        s = ref_rows[r].astype(np.float64)
        ref_key = torch.from_numpy(ref_rows[r]).bfloat16().float().numpy()
        order = np.argsort(-ref_key, kind="stable")
        theirs = set(order[:k].tolist())
        kth = float(s[order[k - 1]])
        e_tab = M * lut_abs * 2.0 ** -11 + abs(kth) * 2.0 ** -11 + abs(kth) * 2.0 ** -20
        band = 2 * e_tab + 2 * float(_bf16_ulp(np.float32(kth)))
        kth_key = ref_key[order[k - 1]]
        for t in mine ^ theirs:
            assert abs(s[t] - kth) <= band, (r, t, s[t], kth, band)
            ties += int(ref_key[t] == kth_key)
        differing += len(mine ^ theirs)
    return differing, ties


@pytest.mark.parametrize("name,T,k,seed", [("C1", 8192, None, 11), ("C2", 131072, None, 12)])
def test_per_head_selection_vs_reference_fp32(name, T, k, seed):
    q, cb, codes = _c_inputs(seed, T)
    ref = ref_path.scores_fp32(q, cb, codes, 4).numpy()  # [Hq, T] fp32
    cs, ce = orc.candidate_window(T, T, SINK, LOCAL)
    kk = orc.budget_k(ce - cs) if k is None else k
    assert kk == {8192: 163, 131072: 2621}[T]
    heads, lut_abs = _ours(q, cb, codes)
    sel = orc.topk(heads, kk, 1, cs, ce, key_bf16=True)  # [Hq, k] absolute
    mine = [set((row - cs).tolist()) for row in sel]
    differing, ties = _check_band(ref[:, cs:ce], mine, kk, lut_abs)
    print(f"{name} per-head k={kk}: {differing} of {Hq * kk} indices differ "
          f"({ties} at the k-th bf16 key)")


def test_group_selection_vs_reference_fp32_c1():
    """Group top-2048 at C1: the group key is the max over the KV group's
    four heads, ranked in bf16 on both sides."""
    T, kk = 8192, 2048
    q, cb, codes = _c_inputs(13, T)
    ref = ref_path.scores_fp32(q, cb, codes, 4).numpy().reshape(Hkv, 4, T).max(axis=1)
    cs, ce = orc.candidate_window(T, T, SINK, LOCAL)
    heads, lut_abs = _ours(q, cb, codes)
    sel = orc.topk(heads, kk, 4, cs, ce, key_bf16=True)  # [Hkv, k]
    mine = [set((row - cs).tolist()) for row in sel]
    differing, ties = _check_band(ref[:, cs:ce], mine, kk, lut_abs)
    print(f"C1 group top-{kk}: {differing} of {Hkv * kk} indices differ "
          f"({ties} at the k-th bf16 key)")


def _teacher_forced_encode_check(x: torch.Tensor, cb: torch.Tensor, cb_ours=None):
    """(stage codes that differ, rows identical free-running); asserts every
    difference is a float64 near-tie.  cb_ours: the codebooks the oracle is
    handed (a planted mistake in the negative control), default cb."""
    ref = ref_path.encode_fp32(x, cb).numpy()
    cbo = (cb if cb_ours is None else cb_ours).numpy()
    ours_full, _ = orc.encode(x.numpy(), cbo)
    n, Mc = ref.shape
    cbn = cb.numpy()
    cb64 = cbn.astype(np.float64)
    r = x.numpy().copy()
    mismatches = 0
    # fp32 error of one distance (|r|^2 + |c|^2 - 2 r.c, or dot16 of r - c):
    # at most 2 * gamma_D * (|r| + |c|)^2 with gamma_D = D u / (1 - D u)
    u = 2.0 ** -24
    Dx = x.shape[1]
    gamma = Dx * u / (1 - Dx * u)
    for m in range(Mc):
        mine, _ = orc.encode(r, cbo[m:m + 1])
        mine = mine[:, 0].astype(np.int64)
        cmax = float(np.linalg.norm(cb64[m], axis=1).max())
        for i in np.nonzero(mine != ref[:, m])[0]:
            r64 = r[i].astype(np.float64)
            d_ref = float(((r64 - cb64[m, ref[i, m]]) ** 2).sum())
            d_mine = float(((r64 - cb64[m, mine[i]]) ** 2).sum())
            tol = 2 * 2 * gamma * (float(np.linalg.norm(r64)) + cmax) ** 2
            assert abs(d_ref - d_mine) <= tol, (i, m, d_ref, d_mine, tol)
            mismatches += 1
        r = (r - cbn[m][ref[:, m]]).astype(np.float32)
    rows_equal = int((ours_full.astype(np.int64) == ref).all(axis=1).sum())
    return mismatches, n * Mc, rows_equal, n


def test_encode_vs_reference_fp32_c3_teacher_forced():
    x = c3_keys(20)  # [512, 128] fp32: C3's post-RoPE keys
    diff, total, same, n = _teacher_forced_encode_check(x, gaussian_codebooks(21))
    print(f"C3 encode: {diff} of {total} teacher-forced stage codes differ (all float64 "
          f"near-ties); {same} of {n} free-running rows identical")


def test_encode_vs_reference_fp32_unrotated_keys():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(256, D, generator=g) * (torch.rand(D, generator=g) * 3.5 + 0.5)
    diff, total, same, n = _teacher_forced_encode_check(x, gaussian_codebooks(22))
    print(f"unrotated keys encode: {diff} of {total} stage codes differ; {same} of {n} rows "
          f"identical")


def test_band_check_catches_an_index_slip():
    """Negative control: scoring each key with its neighbour's codes (an
    off-by-one token index) puts selections far outside the band."""
    T = 8192
    q, cb, codes = _c_inputs(11, T)
    ref = ref_path.scores_fp32(q, cb, codes, 4).numpy()
    cs, ce = orc.candidate_window(T, T, SINK, LOCAL)
    kk = orc.budget_k(ce - cs)
    heads, lut_abs = _ours(q, cb, torch.roll(codes, 1, dims=1))
    sel = orc.topk(heads, kk, 1, cs, ce, key_bf16=True)
    mine = [set((row - cs).tolist()) for row in sel]
    with pytest.raises(AssertionError):
        _check_band(ref[:, cs:ce], mine, kk, lut_abs)


def test_teacher_forced_check_catches_a_row_slip():
    """Negative control: the oracle handed codebooks whose rows are rolled by
    one (an off-by-one entry index) picks codes that are no near-ties."""
    x = c3_keys(20)[:64]
    cb = gaussian_codebooks(21)
    with pytest.raises(AssertionError):
        _teacher_forced_encode_check(x, cb, torch.roll(cb, 1, dims=1))
