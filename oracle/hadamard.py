"""Hadamard block rotation: closed form and the pinned-order fp32 FWHT.

Reference anchors
-----------------
* `experiments/qwen21-kernel/kernels/g64_quant.cu:1-8` and `:87`: the rotation is the regular
  Hadamard of block 256 built as kron^4(H4) normalised, i.e. H_256 = (H4/2)^(x4), where H4/2 has
  rows [1/2, 1/2, 1/2, -1/2], [1/2, 1/2, -1/2, 1/2], [1/2, -1/2, 1/2, 1/2], [-1/2, 1/2, 1/2, 1/2].
* `g64_quant.cu:68-86`: the fp32 radix-4 FWHT. Stages run with strides 1, 4, 16, 64. In each
  stage, the butterfly with index bf reads x_i = b[base + i*st], base = (bf % st) + (bf / st)*4*st,
  computes hs = 0.5f * (x0 + x1 + x2 + x3) (C evaluates the sum left to right) and writes
  y_i = hs - x_{3-i}.
* `experiments/qwen21-kernel/node/__init__.py:69-71,92` and `g64_quant_test.py:63-64`: the same
  rotation written as x.reshape(M, K/b, b) @ H_b (an fp32 matmul whose summation order is not
  fixed).

Pinning
-------
* `hadamard(b)`: closed form; checked for symmetry, H.H = I, entries +-1/sqrt(b), the H4/2 rows
  above, and the Kronecker recursion (tests/test_oracle_hadamard.py).
* `fwht_pinned`: one-hot inputs give the columns of H_b exactly in fp32; agrees with the fp64
  matmul form to within fp32 rounding; the operation order is the reference kernel's, so the
  result is unique. For b = 16 and 64 the same power-of-4 construction is a builder assumption
  (comfy-kitchen's `_build_hadamard(16/64)` is absent from the reference tree).
"""
from __future__ import annotations

import numpy as np

F32 = np.float32
BLOCKS = (16, 64, 256)


def h4_half() -> np.ndarray:
    """H4/2 = J/2 - P4 (P4 the anti-identity), g64_quant.cu:7 ("y_i = (x0+x1+x2+x3)/2 - x_{3-i}")."""
    return 0.5 * np.ones((4, 4)) - np.fliplr(np.eye(4))


def hadamard(b: int) -> np.ndarray:
    """Closed-form H_b = (H4/2)^{(x) log4 b} in float64 (g64_quant.cu:87)."""
    if b not in BLOCKS and not (b >= 4 and (b & (b - 1)) == 0 and (b.bit_length() - 1) % 2 == 0):
        raise ValueError(f"Hadamard block must be a power of 4, got {b}")
    h = np.ones((1, 1))
    while h.shape[0] < b:
        h = np.kron(h4_half(), h)
    return h


def fwht_pinned(x: np.ndarray, block: int) -> np.ndarray:
    """Rotate each row of x (float32 [M, K]) by H_block in blocks along K, in the pinned order.

    Follows g64_quant.cu:68-86 exactly: for st in (1, 4, 16, 64)[:log4(block)], every butterfly
    computes h = 0.5f * (((x0 + x1) + x2) + x3) in float32 and writes y_i = h - x_{3-i}.
    """
    x = np.asarray(x, dtype=F32)
    if x.ndim != 2:
        raise ValueError("x must be 2-D")
    m, k = x.shape
    if block not in BLOCKS:
        raise ValueError(f"block must be one of {BLOCKS}")
    if k % block:
        raise ValueError(f"K={k} must be a multiple of the Hadamard block {block}")
    y = x.reshape(m, k // block, block).copy()
    st = 1
    half = F32(0.5)
    while st < block:
        # element index within the block e = (bf // st) * 4 * st + i * st + (bf % st)
        v = y.reshape(m, k // block, block // (4 * st), 4, st)
        x0, x1, x2, x3 = v[:, :, :, 0, :], v[:, :, :, 1, :], v[:, :, :, 2, :], v[:, :, :, 3, :]
        h = half * (((x0 + x1) + x2) + x3)
        out = np.stack([h - x3, h - x2, h - x1, h - x0], axis=3)
        y = out.reshape(m, k // block, block)
        st *= 4
    return y.reshape(m, k).astype(F32, copy=False)


def rotate_matmul64(x: np.ndarray, block: int) -> np.ndarray:
    """The matmul form x.reshape(M, K/b, b) @ H_b in float64 (node/__init__.py:92,
    g64_quant_test.py:63-64). Used only as an independent cross-check of `fwht_pinned`."""
    x = np.asarray(x, dtype=np.float64)
    m, k = x.shape
    return (x.reshape(m, k // block, block) @ hadamard(block)).reshape(m, k)
