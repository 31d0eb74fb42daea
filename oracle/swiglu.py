"""SwiGLU prologue of the activation quantizer, restated in numpy float32.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Reference: `tools/ck_swiglu/swiglu_quant.cu:23-97`. The input h [M, 2K] holds gate | up; each
element of the activation is `a = g / (1 + exp(-g)) * u` computed in fp32 and rounded once to the
input dtype (bf16), straight from h (:56-66, "silu(g) * u in fp32, one rounding below"); the
rounded activation then goes through the same rotation and per-token quantization as an ordinary
input. The dispatch (`patches/comfyui_swiglu_triton_env.patch:65-97`,
`patches/comfy_kitchen_swiglu_w4a4_fused.patch:17-33`) passes the whole `[gate | up]` row, K a
multiple of 256 and at most 16384.

The reference evaluates exp with CUDA's hardware approximation `__expf`, whose bits are not
published. This build takes silu correctly rounded to fp32 instead, the exact function the
reference approximates:

    silu32(g) = RN_fp32(g / (1 + exp(-g)))            (exact real arithmetic, one rounding)
    swiglu_bf16(g, u) = RN_bf16(RN_fp32(silu32(g) * u))

Here silu32 is evaluated in float64 and rounded to fp32. For the bf16 and fp16 gate values this
path sees, that equals the correctly rounded value; tests/test_oracle_swiglu.py checks every finite
bf16 and fp16 pattern against exact decimal arithmetic. Closed forms it reproduces for bf16 gates:
|g| < 2^-25 gives g / 2, g >= 128 gives g and g <= -128 gives -0.

fp16 inputs round the product to fp16 instead (the reference's from_float<InType>,
swiglu_quant.cu:63-70, dispatched for kHalf at :128-132):

    swiglu_f16(g, u) = RN_fp16(RN_fp32(silu32(g) * u))

Outside comfy-kitchen's fused domain (convrot_w4a4_linear with linear_dtype="int8", a convrot
group other than 256, `patches/comfy_kitchen_swiglu_w4a4_fused.patch:25-31`) the activation is
applied eagerly first (:60-64) as `silu(gate).mul_(up)` in the input's type
(`patches/comfyui_swiglu_triton_env.patch:16-20`): torch rounds silu's fp32 value to the input
type, then the product (exact in fp32: two 8- or 11-bit significands) again:

    swiglu_bf16_eager(g, u) = RN_bf16(RN_bf16(silu32(g)) * u)
    swiglu_f16_eager(g, u)  = RN_fp16(RN_fp16(silu32(g)) * u)

(torch evaluates silu in fp32 with its own exp, which can differ from silu32 in the last fp32 bit;
that changes the first rounding only where silu32 lies within one fp32 ulp of a bf16 / fp16
rounding boundary.)

Pinning (tests/test_oracle_swiglu.py): exhaustive comparison with Python's decimal module at
60 digits over every finite bf16 gate (rounded to the nearest fp32 with ties to even), the
closed-form regions, silu's identities (silu(g) - silu(-g) = g, sign and monotonicity on
g > -1.27), the bf16 rounding of the product against a float64 product, and the composition
with the rotation and quantizer.
"""
from __future__ import annotations

import numpy as np

from .quant import bf16_bits_to_f32, f32_to_bf16_bits, rotquant

F32 = np.float32


def silu32(g: np.ndarray) -> np.ndarray:
    """silu(g) = g / (1 + exp(-g)) correctly rounded to fp32, for g holding bf16 values."""
    g64 = np.asarray(g, dtype=F32).astype(np.float64)
    with np.errstate(over="ignore"):
        return (g64 / (1.0 + np.exp(-g64))).astype(F32)


def swiglu_bf16(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """bf16-rounded silu(g) * u (swiglu_quant.cu:64 with silu correctly rounded), returned as
    float32 holding bf16 values."""
    prod = (silu32(g) * np.asarray(u, dtype=F32)).astype(F32)
    return bf16_bits_to_f32(f32_to_bf16_bits(prod))


def swiglu_f16(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """fp16-rounded silu(g) * u for fp16 inputs, returned as float32 holding fp16 values."""
    prod = (silu32(g) * np.asarray(u, dtype=F32)).astype(F32)
    with np.errstate(over="ignore"):
        return prod.astype(np.float16).astype(F32)


def swiglu_bf16_eager(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """silu(gate).mul_(up) in bf16: silu rounded to bf16, then the product rounded to bf16."""
    s = bf16_bits_to_f32(f32_to_bf16_bits(silu32(g)))
    prod = (s * np.asarray(u, dtype=F32)).astype(F32)
    return bf16_bits_to_f32(f32_to_bf16_bits(prod))


def swiglu_f16_eager(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """silu(gate).mul_(up) in fp16: silu rounded to fp16, then the product rounded to fp16."""
    with np.errstate(over="ignore"):
        s = silu32(g).astype(np.float16).astype(F32)
        prod = (s * np.asarray(u, dtype=F32)).astype(F32)
        return prod.astype(np.float16).astype(F32)


def swiglu_rotquant(h: np.ndarray, block: int, bits: int, dtype: str = "bf16",
                    eager: bool = False) -> tuple[np.ndarray, np.ndarray]:
    """SwiGLU quantizer: h float32 (bf16 or fp16 values, per `dtype`) [M, 2K] = gate | up ->
    rotquant of the activation [M, K] rounded to that type, once (the fused quantizer,
    swiglu_quant.cu:23-97) or, with eager, twice (silu(gate).mul_(up)), then the per-token int8 /
    int4 quantizer of this path. Returns (q int8 codes [M, K], s float32 [M])."""
    h = np.asarray(h, dtype=F32)
    if h.shape[1] % 2:
        raise ValueError("h must hold gate | up halves")
    k = h.shape[1] // 2
    if dtype == "f16":
        act = swiglu_f16_eager if eager else swiglu_f16
    else:
        act = swiglu_bf16_eager if eager else swiglu_bf16
    return rotquant(act(h[:, :k], h[:, k:]), block, bits)
