"""End-to-end oracle of the quantized linears (rotate -> quantize -> integer GEMM -> epilogue).

Each function returns every intermediate the GPU path must match: the activation codes and
scales (bit-exact), the per-group int32 partials (bit-exact) and the fp64 output the bf16 result
is compared against (relative L2 <= 1e-2).

Reference anchors: online W4A8 linear `tools/quant_mixed.py:315-317` / `tools/svdquant_probe.py:
99-102` (rotation + int8 per-token activations + int GEMM + scales + bias), online ConvRot W4A4
`patches/comfy_kitchen_swiglu_w4a4_fused.patch:41-67` (quantize_int4_rowwise_convrot64 then
int4_linear with row x row scales), `int8_linear` `tools/verify_w4a4.py:342-370`, and the weight
rotation W_rot = W.reshape(N, K/b, b) @ H_b of `experiments/qwen21-kernel/node/__init__.py:92`
(restated with the pinned FWHT order so that weight codes are reproducible).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import gemm, quant
from .hadamard import fwht_pinned


@dataclass
class LinearResult:
    qa: np.ndarray          # activation codes int8 [M, K]
    sa: np.ndarray          # per-token scale float32 [M]
    partials: np.ndarray    # int64 [G, M, N] (one group spanning K for per-row weights)
    y: np.ndarray           # float64 [M, N]


def rotate_weight(w: np.ndarray, block: int) -> np.ndarray:
    """W_rot = W @ H_b per block along K (node/__init__.py:92), pinned FWHT order."""
    return fwht_pinned(np.asarray(w, dtype=np.float32), block)


def w4a8_asym_linear(x, q, s16, z, bias, block: int = 256, group: int = 64) -> LinearResult:
    """Configs' W4A8: x float32 [M, K] (bf16 values); q uint8 codes [N, K]; s16 float16 [N, K/G];
    z uint8 [N, K/G]; bias float or None. Weights were quantized from the rotated weight."""
    qa, sa = quant.rotquant(x, block, 8)
    wq = gemm.zero_adjusted(q, z, group)
    p = gemm.partials(qa, wq, group)
    y = gemm.epilogue_group(p, sa, s16.astype(np.float64), bias)
    return LinearResult(qa, sa, p, y)


def w4a4_group_linear(x, q, s16, bias, block: int = 64, group: int = 64) -> LinearResult:
    """Configs' W4A4: int4 per-token activations after H_block, int4 symmetric g64 fp16 weights."""
    qa, sa = quant.rotquant(x, block, 4)
    p = gemm.partials(qa, q, group)
    y = gemm.epilogue_group(p, sa, s16.astype(np.float64), bias)
    return LinearResult(qa, sa, p, y)


def w4a4_row_linear(x, q, s_row, bias, block: int = 256, act_bits: int = 4) -> LinearResult:
    """Shipped ConvRot W4A4 (per-row F32 weight scale); act_bits 8 = linear_dtype "int8"."""
    qa, sa = quant.rotquant(x, block, act_bits)
    k = qa.shape[1]
    p = gemm.partials(qa, q, k)
    y = gemm.epilogue_row(p[0], sa, s_row, bias)
    return LinearResult(qa, sa, p, y)


def w8a8_linear(x, q, s_row, bias, block=None) -> LinearResult:
    """int8_tensorwise: per-row int8 weights, int8 per-token activations, optional rotation."""
    xf = np.asarray(x, dtype=np.float32)
    qa, sa = quant.rotquant(xf, block, 8) if block else quant.quant_per_token(xf, 127)
    k = qa.shape[1]
    p = gemm.partials(qa, q, k)
    y = gemm.epilogue_row(p[0], sa, np.asarray(s_row).reshape(-1), bias)
    return LinearResult(qa, sa, p, y)
