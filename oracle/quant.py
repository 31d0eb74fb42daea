"""Quantizers and int4 packing, restated in numpy float32 / integer arithmetic.

Activation side (online)
------------------------
`quant_per_token(xr, limit)` follows `tools/activation_balance.py:65-71` (`quantize_rowwise` with
group_size None): s = (absmax / limit).clamp(min=1e-10); q = (x / s).round().clamp(-limit, limit),
with limit = 127 (int8, W4A8) or 7 (int4, W4A4). The same arithmetic appears in
`tools/gptq_w4a4.py:112-114` (`q4_token`) and `tools/weight_balance.py:117-127`. Division is IEEE
fp32 x / s (not x * (1/s)); rounding is half-to-even (torch.round).

`rotquant(x, block, bits)` = `fwht_pinned` then `quant_per_token`: the online activation path of
the W4A8/W4A4 linear (`g64_quant.cu:27-108` with a per-token instead of per-group scale).

Weight side (offline)
---------------------
* `quant_weight_u4_asym(w, G)`: the configs' uint4 asymmetric per-group scheme. Builder-defined
  spec following the in-repo affine forms `custom_nodes/comfy-lowbit-loader/formats.py:131-149`
  (per-group lo/hi, step = (hi - lo)/levels, code = round((x - lo)/step).clamp) and the integer
  zero-point form W = (q - z) * s of `patches/comfyui_awq_w4a16_format.patch:80`. The range is
  widened to contain 0 (lo <= 0 <= hi) so that z fits in [0, 15]:
      s = fp16((hi - lo) / 15); z = clamp(rne(-lo / s), 0, 15); q = clamp(rne(w / s) + z, 0, 15);
  an all-zero group stores s = 0, z = 0, q = 0.
* `quant_weight_i4_sym_group(w, G)`: int4 symmetric per group with fp16 scale,
  `tools/svdquant_probe.py:105-115` form: s = fp16(absmax / 7); q = clamp(rne(w / s), -7, 7);
  an all-zero group stores s = 0, q = 0.
* `quant_weight_i4_rowwise(w)`: the shipped ConvRot W4A4 weight (per-row F32 scale), RTN check of
  `tools/gptq_w4a4.py:197-203`: s = absmax.clamp(min=1e-10) / 7; q = (w / s).round().clamp(-7, 7).
* `quant_weight_i8_rowwise(w)`: `int8_tensorwise` per-row int8 (`tools/_formats.py:128-167`),
  s = absmax.clamp(min=1e-10) / 127, q = (w / s).round().clamp(-127, 127), scale shape [N, 1].

Packing
-------
`pack_i4` / `unpack_i4`: byte j of a row holds k = 2j in bits 0-3 and k = 2j + 1 in bits 4-7;
signed nibbles v >= 8 decode as v - 16 (`experiments/qwen21-kernel/node/__init__.py:82-86`,
`g64_bench6.py:44-47`, `g64_quant_test.py:48-52`). `pack_u4` / `unpack_u4` are the unsigned
LSB-first form of `custom_nodes/comfy-lowbit-loader/kernel.py:75-81`.

Pinning
-------
tests/test_oracle_quant.py: hand-computed known answers (zero row, saturation, exact ties,
constant / two-valued / zero-containing groups), torch.round half-even semantics, pack round
trips and hand-packed bytes, and the statistical round-trip errors quoted at README.md:448-452
(int8 per-token ~0.009, int4 ~0.17 rel-L2 on Gaussian rows after rotation).
"""
from __future__ import annotations

import numpy as np

from .hadamard import fwht_pinned

F32 = np.float32
EPS_SCALE = F32(1e-10)


# --------------------------------------------------------------------------- bf16 helpers

def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(F32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.asarray(x, dtype=F32).view(np.uint32).astype(np.uint64)
    rounded = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return rounded.astype(np.uint16)


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    """float32 -> float16, IEEE round to nearest even (numpy's cast)."""
    return np.asarray(x, dtype=F32).astype(np.float16)


# --------------------------------------------------------------------------- activations

def quant_per_token(xr: np.ndarray, limit: int) -> tuple[np.ndarray, np.ndarray]:
    """Per-token symmetric quantizer, tools/activation_balance.py:65-71 (group_size None).

    Returns (q int8 [M, K], s float32 [M]).

    Non-finite values (a row whose activation overflowed, e.g. an fp16 SwiGLU product beyond 65504,
    spreads +-inf and NaN over its Hadamard block): the absmax is taken over the row's non-NaN
    magnitudes (an inf makes it inf, so s = inf), and a value whose quotient x / s is not finite
    (inf / inf, NaN) gets code 0; finite values of such a row quantize to 0 under s = inf. The
    reference computes that scale through finite_absmax_for_int4_scale<InType>
    (tools/ck_swiglu/swiglu_quant.cu:85), whose source is not in the reference tree: this rule is
    this path's own ("parity unpinned" for rows with non-finite values).
    """
    xr = np.asarray(xr, dtype=F32)
    with np.errstate(invalid="ignore", divide="ignore"):
        mag = np.abs(xr)
        mag = np.where(np.isnan(mag), F32(0), mag)
        amax = mag.max(axis=1) if xr.shape[1] else np.zeros(xr.shape[0], F32)
        s = np.maximum(amax / F32(limit), EPS_SCALE).astype(F32)
        t = np.rint(xr / s[:, None])
        q = np.where(np.isfinite(t), np.clip(t, -limit, limit), 0).astype(np.int8)
    return q, s


def rotquant(x: np.ndarray, block: int, bits: int) -> tuple[np.ndarray, np.ndarray]:
    """Online activation path: pinned FWHT by H_block, then per-token int8 (bits=8) or int4
    (bits=4) quantization. Input float32 (bf16 values) [M, K]; returns (q int8 codes [M, K],
    s float32 [M]). int4 codes are returned unpacked (values in [-7, 7]); see `pack_i4`."""
    if bits not in (4, 8):
        raise ValueError("bits must be 4 or 8")
    limit = 127 if bits == 8 else 7
    return quant_per_token(fwht_pinned(x, block), limit)


# --------------------------------------------------------------------------- packing

def pack_i4(q: np.ndarray) -> np.ndarray:
    """Signed int4 codes [R, K] -> int8 [R, K/2], low nibble = even k (node/__init__.py:82-86)."""
    q = np.asarray(q)
    if q.shape[-1] % 2:
        raise ValueError("K must be even to pack int4")
    lo = q[..., 0::2].astype(np.int16) & 0xF
    hi = q[..., 1::2].astype(np.int16) & 0xF
    return (lo | (hi << 4)).astype(np.uint8).view(np.int8)


def unpack_i4(p: np.ndarray) -> np.ndarray:
    """int8 [R, K/2] -> signed int4 codes [R, K] (g64_quant_test.py:48-52)."""
    u = np.asarray(p).view(np.uint8).astype(np.int16)
    lo, hi = u & 0xF, (u >> 4) & 0xF
    v = np.stack([lo, hi], axis=-1).reshape(*u.shape[:-1], u.shape[-1] * 2)
    return np.where(v >= 8, v - 16, v).astype(np.int8)


def pack_u4(q: np.ndarray) -> np.ndarray:
    """Unsigned 4-bit codes [R, K] in [0, 15] -> uint8 [R, ceil(K/2)], LSB-first along K
    (custom_nodes/comfy-lowbit-loader/kernel.py:75-81 with bits = 4)."""
    q = np.asarray(q).astype(np.int32)
    if q.min(initial=0) < 0 or q.max(initial=0) > 15:
        raise ValueError("u4 codes must lie in [0, 15]")
    if q.shape[-1] % 2:                       # odd length: the last byte's high nibble is 0
        q = np.concatenate([q, np.zeros((*q.shape[:-1], 1), np.int32)], axis=-1)
    return (q[..., 0::2] | (q[..., 1::2] << 4)).astype(np.uint8)


def unpack_u4(p: np.ndarray) -> np.ndarray:
    u = np.asarray(p, dtype=np.uint8)
    return np.stack([u & 0xF, u >> 4], axis=-1).reshape(*u.shape[:-1], u.shape[-1] * 2)


# --------------------------------------------------------------------------- weights

def quant_weight_u4_asym(w: np.ndarray, group: int = 64):
    """uint4 asymmetric per-group weights with fp16 scale and uint4 zero-point (configs' scheme).

    Returns (q uint8 codes [N, K] in [0,15], s float16 [N, K/G], z uint8 [N, K/G] in [0,15]).
    Dequantized weight: W = (q - z) * s.
    """
    w = np.asarray(w, dtype=F32)
    n, k = w.shape
    if k % group:
        raise ValueError(f"K={k} must be a multiple of the group size {group}")
    g = w.reshape(n, k // group, group)
    lo = np.minimum(g.min(axis=2), F32(0))
    hi = np.maximum(g.max(axis=2), F32(0))
    s16 = f32_to_f16((hi - lo) / F32(15))
    if not np.isfinite(s16).all():
        raise ValueError("group range overflows the fp16 scale")
    s = s16.astype(F32)
    zero = s == 0
    safe = np.where(zero, F32(1), s)
    z = np.clip(np.rint(-lo / safe), 0, 15)
    q = np.clip(np.rint(g / safe[..., None]) + z[..., None], 0, 15)
    q = np.where(zero[..., None], 0, q)
    z = np.where(zero, 0, z)
    return q.reshape(n, k).astype(np.uint8), s16, z.astype(np.uint8)


def dequant_u4_asym(q: np.ndarray, s: np.ndarray, z: np.ndarray) -> np.ndarray:
    """W = (q - z) * s in float64 (exact for 4-bit codes and fp16 scales)."""
    n, k = q.shape
    groups = s.shape[1]
    gq = q.reshape(n, groups, k // groups).astype(np.float64)
    return ((gq - z.astype(np.float64)[..., None]) * s.astype(np.float64)[..., None]).reshape(n, k)


def quant_weight_i4_sym_group(w: np.ndarray, group: int = 64):
    """int4 symmetric per-group weights with fp16 scale (configs' W4A4 scheme,
    tools/svdquant_probe.py:105-115 with the scale stored in fp16).

    Returns (q int8 codes [N, K] in [-7, 7], s float16 [N, K/G]).
    """
    w = np.asarray(w, dtype=F32)
    n, k = w.shape
    if k % group:
        raise ValueError(f"K={k} must be a multiple of the group size {group}")
    g = w.reshape(n, k // group, group)
    s16 = f32_to_f16(np.abs(g).max(axis=2) / F32(7))
    s = s16.astype(F32)
    safe = np.where(s == 0, F32(1), s)
    q = np.clip(np.rint(g / safe[..., None]), -7, 7)
    q = np.where((s == 0)[..., None], 0, q)
    return q.reshape(n, k).astype(np.int8), s16


def quant_weight_i4_rowwise(w: np.ndarray):
    """Shipped ConvRot W4A4 weight codes from an already rotated weight: per-row F32 scale,
    tools/gptq_w4a4.py:197-203. Returns (q int8 [N, K] in [-7, 7], s float32 [N])."""
    w = np.asarray(w, dtype=F32)
    s = (np.maximum(np.abs(w).max(axis=1), EPS_SCALE) / F32(7)).astype(F32)
    q = np.clip(np.rint(w / s[:, None]), -7, 7).astype(np.int8)
    return q, s


def quant_weight_i8_rowwise(w: np.ndarray):
    """int8_tensorwise per-row weight (tools/_formats.py:128-167): returns (q int8 [N, K],
    s float32 [N, 1])."""
    w = np.asarray(w, dtype=F32)
    s = (np.maximum(np.abs(w).max(axis=1), EPS_SCALE) / F32(127)).astype(F32)
    q = np.clip(np.rint(w / s[:, None]), -127, 127).astype(np.int8)
    return q, s[:, None]
