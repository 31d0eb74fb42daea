"""Load-time decode of comfy-kitchen's shipped `asym_w4a8_int8` weights to an int8 weight with a
per-row scale, restated in numpy.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Tensors per Linear (`tools/_formats.py:79-125`, `tools/quant_w4a8.py:8-13`, headers quoted at
`tools/verify_w4a4.py:205-212`):
    qdata      I8  [N, K/2]   4-bit codes, byte j holds k = 2j (bits 0-3) and k = 2j+1 (bits 4-7)
    s_rel      U8  [N, K/gs]  fp8 e4m3fn per-group scale stored as raw bytes
    s_channel  F32 [N]        per-row scale
    codebook   F32 [16]       Lloyd-Max levels (absent under --no-codebook)
comfy-kitchen finishes a decoded W4A8 weight as
`dequantize_int8_convrot_weight_dtype(int8_weight, s_channel, ...)`
(`patches/comfy_kitchen_w4a8_dequant_fused.patch:15-18`): the decoded int8 weight is paired with the
stored `s_channel` as its per-row scale, unchanged, so `level * s_rel` is already in int8 units:

    level[n, k] = codebook[code]            (code = unsigned nibble)      with a codebook
                = code as signed int4       (v >= 8 -> v - 16)            without
    t[n, k]     = fp32(level * fp8(s_rel[n, k / gs]))
    q8[n, k]    = clamp(rne(t[n, k]), -127, 127)      (0 where t is NaN)
    row_scale[n] = s_channel[n]

so q8 * row_scale is level * s_rel * s_channel to within half an int8 step (s_channel / 2) wherever
|t| <= 127.5. The pairing is the reference's; the rounding of t (half to even here) is not in the
reference tree (comfy-kitchen is absent), so that detail is "parity unpinned". The oracle is pinned
by the fp8 format definition (torch's float8_e4m3fn on all 256 bytes), hand-built rows with known
codes, ties and saturation, and the reconstruction bound (tests/test_oracle_codebook.py).
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


def fp8_e4m3fn_to_f32(b: np.ndarray) -> np.ndarray:
    """OCP fp8 e4m3fn (1 sign, 4 exponent bits with bias 7, 3 mantissa bits, no infinities,
    S.1111.111 = NaN) to float32, exactly."""
    b = np.asarray(b, dtype=np.uint8).astype(np.int32)
    sign = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = b & 0x7
    val = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * 2.0 ** (e - 7))
    val = np.where((e == 0xF) & (m == 0x7), np.nan, val)
    return (sign * val).astype(F32)


def unpack_codes(qdata: np.ndarray) -> np.ndarray:
    """I8/U8 [N, K/2] -> unsigned nibbles [N, K] (low nibble = even k)."""
    u = np.asarray(qdata).view(np.uint8)
    return np.stack([u & 0xF, u >> 4], axis=-1).reshape(u.shape[0], u.shape[1] * 2)


def levels(qdata: np.ndarray, codebook) -> np.ndarray:
    codes = unpack_codes(qdata)
    if codebook is None:
        return np.where(codes >= 8, codes.astype(np.int16) - 16, codes).astype(F32)
    return np.asarray(codebook, dtype=F32)[codes]


def decode_w4a8_codebook(qdata, s_rel_u8, s_channel, codebook, group_size: int):
    """Returns (q8 int8 [N, K], row_scale float32 [N]) per the module docstring."""
    lev = levels(qdata, codebook)
    n, k = lev.shape
    if k % group_size:
        raise ValueError("K must be a multiple of group_size")
    srel = fp8_e4m3fn_to_f32(s_rel_u8)
    if srel.shape != (n, k // group_size):
        raise ValueError("s_rel must be [N, K / group_size]")
    t = (lev * np.repeat(srel, group_size, axis=1)).astype(F32)
    with np.errstate(invalid="ignore"):
        q = np.clip(np.rint(t), -127, 127)
    q = np.where(np.isnan(t), 0, q).astype(np.int8)
    return q, np.asarray(s_channel, dtype=F32).reshape(-1).copy()


def dequant_rotated(qdata, s_rel_u8, s_channel, codebook, group_size: int) -> np.ndarray:
    """The weight the tensors describe, level * s_rel * s_channel, in float64 (rotated space)."""
    lev = levels(qdata, codebook).astype(np.float64)
    srel = fp8_e4m3fn_to_f32(s_rel_u8).astype(np.float64)
    return lev * np.repeat(srel, group_size, axis=1) * np.asarray(s_channel, np.float64)[:, None]
