"""The encode's coarse shortlist at C3, restated on the CPU (test only).

The GPU encode (csrc/encode.hip) prunes each stage's 256 candidates with
bf16 MFMA distances G_k = (rn + cn_k) - 2 bf16(r).bf16(C_k) and a proven
error bound eps_k; entry k survives unless G_k - eps_k > min_j (G_j + eps_j),
and only survivors get the exact fp32 recheck.  Along the oracle's own
encode trajectory this test recomputes the shortlist in float64 with the
kernel's eps formula, checks that the exact argmin (the oracle's code)
always survives, and reports survivors per row and stage for N(0, 0.02)
codebooks and for residual-ordered ones of trained magnitude.
"""
import numpy as np
import pytest

from oracle import orc

from _synth import c3_keys, gaussian_codebooks, residual_codebooks


def _bf16(a):
    b = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000  # round to nearest even
    return b.view(np.float32).astype(np.float64)


def _shortlist_sizes(x, cb):
    codes, _ = orc.encode(x, cb)
    r = x.astype(np.float32).copy()
    n, M = codes.shape
    sizes = np.zeros((n, M), np.int64)
    cn = (cb.astype(np.float64) ** 2).sum(-1)  # [M, K]
    for m in range(M):
        rn = (r.astype(np.float64) ** 2).sum(-1)[:, None]
        dm = _bf16(r) @ _bf16(cb[m]).T
        A = rn + cn[m][None, :]
        G = A - 2 * dm
        eps = (1.0078125 * 2.0 ** -6 * np.sqrt(rn) * np.sqrt(cn[m])[None, :]
               + 2.0 ** -21 * (np.abs(A) + 2 * np.abs(dm))
               + 2.0 ** -116 * (1 + np.sqrt(rn) + np.sqrt(cn[m])[None, :]))
        U = (G + eps).min(axis=1, keepdims=True)
        keep = ~(G - eps > U)
        assert keep[np.arange(n), codes[:, m]].all(), m  # the exact argmin survives
        sizes[:, m] = keep.sum(1)
        r = (r - cb[m][codes[:, m]]).astype(np.float32)
    return sizes


@pytest.mark.parametrize("kind", ["gaussian", "residual"])
def test_encode_shortlist_c3(kind):
    x = c3_keys(60).numpy()
    cb = (gaussian_codebooks(61) if kind == "gaussian" else residual_codebooks(61)).numpy()
    s = _shortlist_sizes(x, cb)
    assert s.min() >= 1
    first, last = s[:, 0].mean(), s[:, -1].mean()
    print(f"{kind}: survivors per row and stage mean {s.mean():.2f}, p99 "
          f"{np.percentile(s, 99):.0f}, max {s.max()}; stage 0 {first:.2f}, stage 31 {last:.2f}")
