"""Exact integer GEMM partials and the fp64 epilogue of the quantized linear.

Reference anchors
-----------------
* `experiments/qwen21-kernel/kernels/g64_bench6.py:50-68` (`ref`): the GEMM reference sums per
  K-group products af[:, g] @ bf[:, g].T and applies the group's scales, then the row scales and
  the bias: out = sum_g (A_g B_g^T) * scale_g ; out * sa[:, None] * sb[None, :] + bias.
* `g64_gemm6.cu:3-12`: policy 0 = full-K int32 accumulator with the row scales in the epilogue
  (the shipped ConvRot W4A4 and the W8A8 `int8_tensorwise` path); weight-group policies scale
  each group's int32 partial.

For the configs' W4A8 scheme (uint4 asymmetric, group G = 64, fp16 scale s, uint4 zero z):
    P[g, m, n] = sum_{k in g} qa[m, k] * (qw[n, k] - z[n, g])           (exact integer)
    y[m, n]    = sa[m] * sum_g s[n, g] * P[g, m, n] + bias[n]             (fp64, then bf16)
For W4A4 with int4 symmetric per-group weights, z = 0. For per-row weight scales there is one
group spanning K and the weight scale is per row n.

Exactness: |qa| <= 127, |qw - z| <= 15, so |P| <= 64 * 127 * 15 < 2^17 per group and the full-K
int8 x int8 sum is < K * 127^2 < 2^31 for K <= 133 000. The partials are computed with float64
BLAS: every product and every partial sum is an integer of magnitude < 2^53, so the float64
result is exact and independent of summation order. `partials_int64` is the brute-force int64
form used to cross-check it on small shapes.

Pinning: tests/test_oracle_gemm.py checks float64 == int64 brute force, closed forms
(all-ones inputs, one-hot inputs that select a single weight, zero-point-only weights),
linearity, and the epilogue against a direct fp64 dequantized matmul.
"""
from __future__ import annotations

import numpy as np


def partials(qa: np.ndarray, wq: np.ndarray, group: int) -> np.ndarray:
    """P[g, m, n] = sum_{k in g} qa[m, k] * wq[n, k], exact, as int64 [K/group, M, N].

    qa: integer [M, K]; wq: integer [N, K] (already zero-point adjusted, q - z).
    """
    qa = np.asarray(qa)
    wq = np.asarray(wq)
    m, k = qa.shape
    n, k2 = wq.shape
    if k != k2 or k % group:
        raise ValueError("shape mismatch")
    g = k // group
    a = qa.astype(np.float64).reshape(m, g, group).transpose(1, 0, 2)   # [g, M, G]
    b = wq.astype(np.float64).reshape(n, g, group).transpose(1, 2, 0)   # [g, G, N]
    p = np.matmul(a, b)
    return p.astype(np.int64)


def partials_int64(qa: np.ndarray, wq: np.ndarray, group: int) -> np.ndarray:
    """Brute-force int64 restatement of `partials` (small shapes only)."""
    qa = np.asarray(qa).astype(np.int64)
    wq = np.asarray(wq).astype(np.int64)
    m, k = qa.shape
    n = wq.shape[0]
    g = k // group
    out = np.zeros((g, m, n), dtype=np.int64)
    for gi in range(g):
        sl = slice(gi * group, (gi + 1) * group)
        out[gi] = np.einsum("mk,nk->mn", qa[:, sl], wq[:, sl])
    return out


def zero_adjusted(q: np.ndarray, z: np.ndarray, group: int) -> np.ndarray:
    """(q - z[n, k // group]) as int16 [N, K]."""
    n, k = q.shape
    return (q.astype(np.int16).reshape(n, k // group, group) - z.astype(np.int16)[..., None]).reshape(n, k)


def epilogue_group(p: np.ndarray, sa: np.ndarray, sw: np.ndarray, bias=None) -> np.ndarray:
    """y[m, n] = sa[m] * sum_g sw[n, g] * P[g, m, n] + bias[n], float64 (g64_bench6.py:50-68)."""
    acc = np.einsum("gmn,ng->mn", p.astype(np.float64), np.asarray(sw, dtype=np.float64))
    y = acc * np.asarray(sa, dtype=np.float64)[:, None]
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)[None, :]
    return y


def epilogue_row(p_full: np.ndarray, sa: np.ndarray, sw: np.ndarray, bias=None) -> np.ndarray:
    """Policy 0 (g64_gemm6.cu:5): y = P * sa[m] * sw[n] + bias[n], P the full-K int32 sum."""
    y = p_full.astype(np.float64) * np.asarray(sa, np.float64)[:, None] * np.asarray(sw, np.float64).reshape(1, -1)
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)[None, :]
    return y


def rel_l2(ref: np.ndarray, got: np.ndarray) -> float:
    ref = np.asarray(ref, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))
