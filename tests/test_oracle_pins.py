"""Pins of the CPU oracle (oracle/aq_oracle.c) against independent truths.

The reference ships no tests or golden vectors (its kernels are CUDA and
cannot be built here), so each oracle function is pinned by mathematics:
exact rational arithmetic, float64 closed forms, independent numpy
restatements and constructed inputs with known answers.  A plausible slip
(wrong rounding, dropped term, transposed index, wrong tie rule) fails one
of these.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import orc, ref_path

RNG = np.random.default_rng(1234)


# ----------------------------------------------------------- exact helpers

def _round_f32(fr: Fraction) -> np.float32:
    """Correct RNE rounding of an exact rational to float32 (normal range)."""
    if fr == 0:
        return np.float32(0.0)
    cand = np.float32(float(fr))  # float64 rounding then float32: may double-round
    # fix-up: pick the float32 neighbour nearest to fr (ties to even)
    best = None
    for c in (np.nextafter(cand, np.float32(-np.inf)), cand, np.nextafter(cand, np.float32(np.inf))):
        err = abs(Fraction(float(c)) - fr)
        key = (err, int(np.array(c, dtype=np.float32).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return np.float32(best[1])


def _fma_exact(a, b, c) -> np.float32:
    return _round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def _add_exact(a, b) -> np.float32:
    return _round_f32(Fraction(float(a)) + Fraction(float(b)))


# ------------------------------------------------------------ conversions

def test_h2f_all_patterns():
    L = orc.lib()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([L.orc_h2f(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f2h_roundtrip_and_numpy():
    L = orc.lib()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = bits.view(np.float16).astype(np.float32)
    ok = ~np.isnan(vals)
    back = np.array([L.orc_f2h(float(v)) for v in vals[ok]], dtype=np.uint16)
    assert np.array_equal(back, bits[ok])
    # random floats over the whole fp16 range, subnormals and exact ties
    x = np.concatenate([
        RNG.standard_normal(60000).astype(np.float32) * 10.0 ** RNG.uniform(-9, 5, 60000).astype(np.float32),
        (vals[ok][:20000].astype(np.float64) + np.float64(2.0) ** -25).astype(np.float32),
        np.array([65504, 65519.99, 65520, 65536, 2 ** -24, 2 ** -25, 3 * 2 ** -26, -0.0], np.float32),
    ])
    got = np.array([L.orc_f2h(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(got, x.astype(np.float16).view(np.uint16))


def test_bf16_rounding_matches_torch():
    x = (RNG.standard_normal(100000) * 10.0 ** RNG.uniform(-30, 30, 100000)).astype(np.float32)
    want = torch.from_numpy(x).bfloat16().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.f2bf_bits(x), want)
    L = orc.lib()
    got = np.array([L.orc_f2bf(float(v)) for v in x[:5000]], dtype=np.uint16)
    assert np.array_equal(got, want[:5000])


# --------------------------------------------------------------- A1 LUT

def test_lut_exact_rational_chain():
    q = RNG.standard_normal((3, 16)).astype(np.float32)
    cb = (RNG.standard_normal((2, 5, 16)) * 0.3).astype(np.float32)
    got = orc.lut_build(q, cb)
    for h in range(3):
        for m in range(2):
            for k in range(5):
                acc = np.float32(0)
                for d in range(16):
                    acc = _fma_exact(q[h, d], cb[m, k, d], acc)
                assert got[h, m, k] == np.float16(acc).view(np.uint16)


def test_lut_order_is_pinned_by_cancellation():
    """[2^24, 1, -2^24] summed in d order gives 0 ((2^24 + 1) rounds to even),
    in reverse order gives 1: the chain direction is observable."""
    q = np.zeros((1, 16), np.float32)
    q[0, :3] = 1.0
    cb = np.zeros((1, 2, 16), np.float32)
    cb[0, 0, :3] = [2.0 ** 24, 1.0, -(2.0 ** 24)]
    cb[0, 1, :3] = [-(2.0 ** 24), 1.0, 2.0 ** 24]
    got = orc.h_vals(orc.lut_build(q, cb).reshape(-1))
    assert got.tolist() == [0.0, 1.0]


def test_lut_float64_bound():
    q = RNG.standard_normal((8, 128)).astype(np.float32)
    cb = (RNG.standard_normal((4, 64, 128)) * 0.02).astype(np.float32)
    got = orc.h_vals(orc.lut_build(q, cb))
    exact = np.einsum("hd,mkd->hmk", q.astype(np.float64), cb.astype(np.float64))
    absum = np.einsum("hd,mkd->hmk", np.abs(q).astype(np.float64), np.abs(cb).astype(np.float64))
    bound = 128 * 2.0 ** -24 * absum * 1.01 + np.abs(exact) * 2.0 ** -11 + 2.0 ** -25
    assert np.all(np.abs(got - exact) <= bound)


def test_lut_one_hot_codebook_and_linearity():
    D, M, K = 32, 2, 16
    cb = np.zeros((M, K, D), np.float32)
    for m in range(M):
        for k in range(K):
            cb[m, k, (m * K + k) % D] = 1.0
    q = RNG.standard_normal((4, D)).astype(np.float32)
    got = orc.lut_build(q, cb)
    for m in range(M):
        for k in range(K):
            assert np.array_equal(got[:, m, k], q[:, (m * K + k) % D].astype(np.float16).view(np.uint16))
    cb2 = (RNG.standard_normal((M, K, D)) * 0.1).astype(np.float32)
    a = orc.h_vals(orc.lut_build(q, cb2))
    b = orc.h_vals(orc.lut_build(2 * q, cb2))
    normal = np.abs(a) > 2 ** -13
    assert np.array_equal(2 * a[normal], b[normal])


# ------------------------------------------------------------ A2 scorers

def _np_sequential_scores(lut_bits, codes, G):
    lut = orc.h_vals(lut_bits.reshape(-1)).reshape(lut_bits.shape)
    H, M, K = lut.shape
    Hkv, T, _ = codes.shape
    out = np.empty((H, T), np.uint16)
    for h in range(H):
        acc = np.zeros(T, np.float32)
        for m in range(M):
            acc = acc + lut[h, m, codes[h // G, :, m].astype(np.int64)]
        out[h] = acc.astype(np.float16).view(np.uint16)
    return out


def test_score_grouped_vs_numpy_sequential():
    lut = (RNG.standard_normal((8, 32, 256)) * 0.3).astype(np.float16).view(np.uint16)
    buf = RNG.integers(0, 256, (2, 600, 32), dtype=np.uint8)
    view = buf[:, :500, :]
    assert np.array_equal(orc.score_grouped(lut, view, 4), _np_sequential_scores(lut, view, 4))


def test_score_special_cases():
    H, M, K = 4, 32, 256
    lut_v = (RNG.standard_normal((H, M, K)) * 0.3).astype(np.float16)
    lut = lut_v.view(np.uint16)
    zeros = np.zeros((1, 7, M), np.uint8)
    got = orc.h_vals(orc.score_grouped(lut, zeros, 4).reshape(-1)).reshape(H, 7)
    for h in range(H):
        acc = np.float32(0)
        for m in range(M):
            acc = np.float32(acc + np.float32(lut_v[h, m, 0]))
        assert np.all(got[h] == np.float16(acc))
    # one-hot LUT counts how many codebooks chose entry 5
    onehot = np.zeros((4, M, K), np.float16)
    onehot[:, :, 5] = 1
    codes = RNG.integers(0, 8, (1, 300, M), dtype=np.uint8)
    cnt = orc.h_vals(orc.score_grouped(onehot.view(np.uint16), codes, 4).reshape(-1)).reshape(4, 300)
    assert np.array_equal(cnt[0], (codes[0] == 5).sum(axis=1).astype(np.float32))


def test_group_invariance_grouped_gqa_mha():
    lut = (RNG.standard_normal((8, 32, 256)) * 0.3).astype(np.float16).view(np.uint16)
    codes = RNG.integers(0, 256, (2, 333, 32), dtype=np.uint8)
    a = orc.score_grouped(lut, codes, 4)
    b = orc.score_gqa(lut, codes, 4, 0, 32)
    expanded = np.repeat(codes, 4, axis=0)  # reference fallback, aq_kv.py:696-699
    c = orc.score_mha(lut.reshape(8, -1), expanded, f32=False)
    assert np.array_equal(a, b) and np.array_equal(a, c)


def test_score_gqa_indices_and_mrange():
    lut = (RNG.standard_normal((4, 32, 256)) * 0.3).astype(np.float16).view(np.uint16)
    codes = RNG.integers(0, 256, (1, 100, 32), dtype=np.uint8)
    idx = np.array([[5, -1, 100, 99, 0]] * 4, np.int64)
    dense = orc.score_gqa(lut, codes, 4, 8, 20)
    sp = orc.score_gqa(lut, codes, 4, 8, 20, idx)
    assert np.all(sp[:, 1] == 0) and np.all(sp[:, 2] == 0)
    assert np.array_equal(sp[:, [0, 3, 4]], dense[:, [5, 99, 0]])
    sub = _np_sequential_scores(lut[:, 8:20, :].copy(), codes[:, :, 8:20].copy(), 4)
    assert np.array_equal(dense, sub)


def test_score_mha_clamp_and_signed_codes():
    Q, n, M, K = 2, 50, 4, 100
    lut = RNG.standard_normal((Q, M * K)).astype(np.float32)
    codes = RNG.integers(-300, 600, (Q, n, M)).astype(np.int64)
    got = orc.score_mha(lut, codes, f32=True)
    for q in range(Q):
        for j in range(n):
            acc = np.float32(0)
            for m in range(M):
                c = min(int(codes[q, j, m]) & 0xFF, K - 1)
                acc = np.float32(acc + lut[q, m * K + c])
            assert got[q, j] == acc


# ------------------------------------------------------- reconstruction

def test_reconstruct_vs_numpy_sequential_and_clamp():
    """Elementwise fp32 sum over m ascending from 0 (aq_kv.py:454-456),
    restated with numpy float32 adds; codes read by their low 8 bits and
    clamped to K - 1."""
    M, K, D, n = 6, 40, 12, 70
    cb = RNG.standard_normal((M, K, D)).astype(np.float32)
    codes = RNG.integers(-300, 600, (n, M)).astype(np.int64)
    got = orc.reconstruct(cb, codes)
    want = np.zeros((n, D), dtype=np.float32)
    for m in range(M):
        c = np.minimum(codes[:, m] & 0xFF, K - 1)
        want = (want + cb[m, c]).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_reconstruct_order_is_pinned():
    """1 + 2^-24 + 2^-24 in fp32 depends on the order: ascending m gives
    (1 + 2^-24) + 2^-24 = 1 (each add ties to even), the reverse order gives
    1 + 2^-23.  The oracle must give the ascending-m value."""
    M, K, D = 3, 2, 4
    cb = np.zeros((M, K, D), dtype=np.float32)
    cb[0, 1] = 1.0
    cb[1, 1] = 2.0 ** -24
    cb[2, 1] = 2.0 ** -24
    codes = np.ones((1, M), dtype=np.uint8)
    got = orc.reconstruct(cb, codes)
    assert np.all(got == np.float32(1.0))
    rev = np.float32(np.float32(np.float32(2.0 ** -24) + np.float32(2.0 ** -24)) + np.float32(1.0))
    assert rev == np.float32(1.0 + 2.0 ** -23)  # the order matters for this input


def test_reconstruct_one_hot_and_float64_bound():
    """Codebook m holding 2^m on coordinate m at entry 1 (zero elsewhere) spells
    the code pattern exactly; random codebooks stay within the fp32 bound of
    the float64 sum."""
    M, K, D = 8, 4, 8
    cb = np.zeros((M, K, D), dtype=np.float32)
    for m in range(M):
        cb[m, 1, m] = 2.0 ** m
    codes = RNG.integers(0, K, (200, M)).astype(np.uint8)
    got = orc.reconstruct(cb, codes)
    want = (codes == 1).astype(np.float32) * (2.0 ** np.arange(M, dtype=np.float32))[None, :]
    assert np.array_equal(got, want)
    cb = RNG.standard_normal((32, 256, 16)).astype(np.float32)
    codes = RNG.integers(0, 256, (300, 32)).astype(np.uint8)
    got = orc.reconstruct(cb, codes).astype(np.float64)
    rows = cb[np.arange(32)[None, :], codes]  # [n, M, D]
    exact = rows.astype(np.float64).sum(axis=1)
    bound = 32 * 2.0 ** -24 * np.abs(rows).astype(np.float64).sum(axis=1)
    assert np.all(np.abs(got - exact) <= bound)


def test_aq_direct_f32_exact_and_f16_restatement():
    q = RNG.standard_normal((2, 8)).astype(np.float32)
    cb = (RNG.standard_normal((3, 6, 8)) * 0.5).astype(np.float32)
    codes = RNG.integers(0, 9, (2, 5, 3)).astype(np.int64)  # 6..8 are skipped (>= K)
    got = orc.aq_direct(q, cb, codes, f16=False)
    for a in range(2):
        for j in range(5):
            acc = np.float32(0)
            for m in range(3):
                c = int(codes[a, j, m])
                if c >= 6:
                    continue
                for i in range(8):
                    acc = _fma_exact(q[a, i], cb[m, c, i], acc)
            assert got[a, j] == acc
    qh = q.astype(np.float16)
    cbh = cb.astype(np.float16)
    got16 = orc.aq_direct(qh.view(np.uint16), cbh.view(np.uint16), codes, f16=True)
    for a in range(2):
        for j in range(5):
            acc = np.float32(0)
            for m in range(3):
                c = int(codes[a, j, m])
                if c >= 6:
                    continue
                p = (qh[a] * cbh[m, c]).astype(np.float16).astype(np.float32)
                for i in range(0, 8, 2):
                    acc = np.float32(acc + np.float32(p[i] + p[i + 1]))
            assert got16[a, j] == np.float16(acc).view(np.uint16)


# --------------------------------------------------------------- A3 top-k

def test_budget_closed_forms():
    assert orc.budget_k(131008) == 2621
    assert orc.budget_k(8128) == 163
    assert orc.budget_k(16384 - 64) == 327
    assert orc.budget_k(32768 - 64) == 655
    assert orc.budget_k(10) == 10 and orc.budget_k(0) == 0 and orc.budget_k(25) == 20
    assert orc.candidate_window(131072, 131072, 0, 64) == (0, 131008)
    assert orc.candidate_window(131072, 131072, 4, 64) == (4, 131008)
    assert orc.candidate_window(50, 50, 4, 64) == (4, 4)


@pytest.mark.parametrize("group,bf", [(1, False), (4, False), (4, True)])
def test_topk_vs_lexsort(group, bf):
    s = ((RNG.standard_normal((3 * group, 5000)) * 4).round() / 4).astype(np.float16).view(np.uint16)
    for k, cs, ce in [(100, 0, 5000), (2048, 7, 4900), (5000, 0, 5000), (1, 3, 4)]:
        a = orc.topk(s, k, group, cs, ce, key_bf16=bf)
        b = orc.topk_numpy(s, k, group, cs, ce, key_bf16=bf)
        assert np.array_equal(a, b)
        assert a.shape[1] == min(k, ce - cs)


def test_topk_special_cases():
    s = np.zeros((2, 1000), np.float16)
    s[1] = -0.0
    out = orc.topk(s.view(np.uint16), 10, cand_start=5, cand_end=900)
    assert np.array_equal(out, np.tile(np.arange(5, 15), (2, 1)))
    ramp = np.arange(1000, dtype=np.float16)[None, :]
    assert np.array_equal(orc.topk(ramp.view(np.uint16), 3), [[997, 998, 999]])
    neg = -ramp
    assert np.array_equal(orc.topk(neg.view(np.uint16), 3), [[0, 1, 2]])


def test_topk_tie_aware_vs_reference_fp32_path():
    """Our contract (fp16 LUT, sequential fp32, fp16 score) vs the reference's
    fp32 path (fp32 LUT, torch sum, top-k): selections differ only where the
    fp32 scores are within the fp16-LUT error of the k-th fp32 score."""
    g = torch.Generator().manual_seed(5)
    Hq, Hkv, T, D, k = 8, 2, 4096, 128, 163
    q = torch.randn(Hq, D, generator=g).bfloat16().float()
    cb = torch.randn(32, 256, D, generator=g) * 0.02
    codes = torch.randint(0, 256, (Hkv, T, 32), generator=g, dtype=torch.uint8)
    ref = ref_path.scores_fp32(q, cb, codes, 4).numpy()
    lut = orc.lut_build(q.numpy(), cb.numpy())
    ours = orc.score_grouped(lut, codes.numpy(), 4)
    sel = orc.topk(ours, k)
    lut_abs = np.abs(orc.h_vals(lut.reshape(-1))).max()
    eps = 32 * (lut_abs * 2.0 ** -11) + np.abs(ref).max() * 2.0 ** -10 + 1e-6
    differing = 0
    for h in range(Hq):
        kth = np.sort(ref[h])[::-1][k - 1]
        mine = set(sel[h].tolist())
        theirs = set(np.argsort(-ref[h], kind="stable")[:k].tolist())
        for t in mine ^ theirs:
            assert abs(ref[h, t] - kth) <= 2 * eps
        differing += len(mine ^ theirs)


# -------------------------------------------------------------- A6 encode

def _dot16_exact(a, b):
    D = a.shape[0]
    L = D // 16
    s = []
    for j in range(16):
        acc = np.float32(0)
        for t in range(L):
            acc = _fma_exact(a[j * L + t], b[j * L + t], acc)
        s.append(acc)
    for w in (8, 4, 2, 1):
        for j in range(w):
            s[j] = _add_exact(s[j], s[j + w])
    return s[0]


def test_dot16_exact_rational():
    for D in (16, 64, 128):
        for _ in range(20):
            a = RNG.standard_normal(D).astype(np.float32)
            b = (RNG.standard_normal(D) * 10.0 ** RNG.uniform(-3, 3, D)).astype(np.float32)
            assert orc.dot16(a, b) == _dot16_exact(a, b)


def test_dot16_fold_pairing_is_pinned():
    """Chain sums s_j = (2^24, 1, -2^24, 0, ...) in block order: the contract's
    pairing (s0+s8, s1+s9, ...) then (s0+s4, ...) keeps the 1; pairing chains
    in a different order loses it to rounding (2^24 + 1 -> 2^24)."""
    D = 16
    a = np.ones(D, np.float32)
    b = np.zeros(D, np.float32)
    b[0], b[8], b[4] = 2.0 ** 24, -(2.0 ** 24), 1.0
    # contract: w=8: s0 = 2^24 + (-2^24) = 0, s4 = 1; w=4: s0 = 0 + 1 = 1
    assert orc.dot16(a, b) == np.float32(1.0)
    assert _dot16_exact(a, b) == np.float32(1.0)
    b2 = np.zeros(D, np.float32)
    b2[0], b2[1], b2[9] = 2.0 ** 24, 1.0, -(2.0 ** 24)
    # contract: w=8: s1 = 1 + (-2^24) = -16777215; w=1 (after s0 stays 2^24): 2^24 - 16777215 = 1
    assert orc.dot16(a, b2) == _dot16_exact(a, b2) == np.float32(1.0)


def test_encode_block_orthogonal_recovery():
    """Stage m lives on dims [4m, 4m+4): stages decouple, so x = sum_m C_m[c_m]
    is recovered exactly with a zero residual."""
    M, K, D = 32, 16, 128
    cb = np.zeros((M, K, D), np.float32)
    for m in range(M):
        cb[m, :, 4 * m:4 * m + 4] = RNG.standard_normal((K, 4)).astype(np.float32)
    truth = RNG.integers(0, K, (20, M))
    x = np.zeros((20, D), np.float32)
    for i in range(20):
        for m in range(M):
            x[i] += cb[m, truth[i, m]]
    codes, rn = orc.encode(x, cb)
    assert np.array_equal(codes, truth.astype(np.uint8))
    assert np.all(rn == 0)


def test_encode_teacher_forced_float64_argmin():
    """Every stage's code is the float64 argmin of ||r - C_m[k]||^2 computed
    from the oracle's own residual, except documented near-ties."""
    M, K, D, N = 32, 256, 128, 24
    cb = (RNG.standard_normal((M, K, D)) * 0.02).astype(np.float32)
    x = (RNG.standard_normal((N, D)) * RNG.uniform(0.5, 4, D)).astype(np.float32)
    codes, rn, tr = orc.encode(x, cb, trace=True)
    near_ties = 0
    for i in range(N):
        r = x[i].copy()
        for m in range(M):
            d64 = ((r.astype(np.float64)[None, :] - cb[m].astype(np.float64)) ** 2).sum(1)
            best = int(np.argmin(d64))
            c = int(codes[i, m])
            scale = (np.linalg.norm(r.astype(np.float64)) + np.linalg.norm(cb[m], axis=1).max()) ** 2
            tol = scale * 2.0 ** -20
            if c != best:
                assert d64[c] - d64[best] <= tol, (i, m, c, best)
                near_ties += 1
            # the fp32 distances the oracle ranked are close to the float64 ones
            assert np.allclose(tr[i, m].astype(np.float64), d64, atol=tol)
            r = (r - cb[m, c]).astype(np.float32)
        assert np.float32(np.sqrt(np.float32(orc.dot16(r, r)))) == rn[i]
    assert near_ties <= 2


def test_encode_tie_takes_lowest_index():
    """Duplicated codebook rows give exactly equal distances: the first wins
    (torch.argmin's rule at laprune/quantizer.py:354)."""
    M, K, D = 3, 8, 32
    cb = (RNG.standard_normal((M, K, D)) * 0.1).astype(np.float32)
    cb[:, 5] = cb[:, 2]
    x = np.stack([cb[0, 2] + cb[1, 2] + cb[2, 2], cb[0, 5] * 1.0001])
    codes, _ = orc.encode(x, cb)
    assert codes[0].tolist() == [2, 2, 2]
    assert codes[1, 0] == 2


def test_encode_zero_input_first_stage():
    M, K, D = 4, 32, 64
    cb = (RNG.standard_normal((M, K, D)) * 0.1).astype(np.float32)
    codes, _ = orc.encode(np.zeros((1, D), np.float32), cb)
    norms = np.array([orc.dot16(cb[0, k], cb[0, k]) for k in range(K)])
    assert codes[0, 0] == int(np.argmin(norms))


# ------------------------------------------------------- A4/A5 attention

def test_attention_oracle_vs_torch_sdpa_and_single_key():
    g = torch.Generator().manual_seed(3)
    B, Hq, Hkv, T, D = 1, 8, 2, 300, 64
    q = torch.randn(B, Hq, D, generator=g, dtype=torch.float64)
    K = torch.randn(B, Hkv, T, D, generator=g, dtype=torch.float64)
    V = torch.randn(B, Hkv, T, D, generator=g, dtype=torch.float64)
    want = torch.nn.functional.scaled_dot_product_attention(
        q[:, :, None], K.repeat_interleave(4, 1), V.repeat_interleave(4, 1))[:, :, 0]
    got = orc.attn_decode_f64(q.numpy(), K.numpy(), V.numpy(), lambda b, h: np.arange(T))
    assert np.allclose(got, want.numpy(), atol=1e-12)
    one = orc.attn_decode_f64(q.numpy(), K.numpy(), V.numpy(), lambda b, h: np.array([17]))
    assert np.allclose(one[0, 5], V[0, 1, 17].numpy(), atol=1e-15)


@pytest.mark.parametrize("T,sink,local", [(1000, 4, 64), (50, 4, 64), (64, 4, 64), (66, 4, 64),
                                          (1000, 0, 64), (1000, 4, 0), (3, 4, 64)])
def test_keep_list_restatement(T, sink, local):
    topk = np.array([10, 20], np.int64)
    keep = orc.keep_list(topk, T, sink, local)
    # reference semantics, aq_evaluation.py:211-237
    sb = min(sink, T) if sink > 0 else 0
    start = max(T - local, 0) if local > 0 else T
    sb_eff = 0 if start <= 0 else sb
    if start > 0 and start < sb_eff:
        start = sb_eff
    want = list(topk) + list(range(sb_eff)) + (list(range(start, T)) if local > 0 and start < T else [])
    assert keep.tolist() == want
