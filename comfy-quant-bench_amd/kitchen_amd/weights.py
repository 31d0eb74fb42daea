"""Offline weight quantizers (the converter side of the path).

They run once per layer at conversion or load time and produce the packed tensors the GEMM entry
points consume. A weight on the GPU is quantized by the library's HIP kernel (mq_quantize_weight);
a weight in host memory by the same arithmetic in torch float32 on the CPU (for conversions on a
machine without the GPU). Rotation uses the fp32 radix-4 FWHT order of the online activation
kernel (experiments/qwen21-kernel/kernels/g64_quant.cu:68-86), and both implementations use IEEE
divisions, so codes and scales are identical bit for bit.

    quantize_w4a8_asym_weight     configs' W4A8: uint4 asymmetric per group, fp16 scale, uint4 zero
    quantize_w4a4_group_weight    configs' W4A4: int4 symmetric per group, fp16 scale
    quantize_convrot_w4a4_weight  shipped ConvRot W4A4: int4 per row, F32 scale [N]
                                  (comfy-kitchen signature, tools/_formats.py:72-76)
    quantize_int8_convrot_weight  int8_tensorwise: int8 per row, F32 scale [N, 1]
                                  (tools/_formats.py:128-167)
"""
from __future__ import annotations

import torch

HADAMARD_BLOCKS = (16, 64, 256)


def _div(a: torch.Tensor, d: float) -> torch.Tensor:
    """IEEE a / d. torch on a GPU turns `tensor / python_scalar` into a multiplication by the
    reciprocal, which rounds differently; dividing by a tensor keeps the true quotient."""
    return a / torch.full_like(a, d)


def fwht(x: torch.Tensor, block: int) -> torch.Tensor:
    """Rotate rows of x (float32 [R, K]) by H_block per block, pinned radix-4 order:
    h = 0.5 * (((x0 + x1) + x2) + x3), y_i = h - x_{3-i}, strides 1, 4, 16, 64."""
    if block not in HADAMARD_BLOCKS:
        raise ValueError(f"convrot_groupsize must be one of {HADAMARD_BLOCKS}, got {block}")
    r, k = x.shape
    if k % block:
        raise ValueError(f"K={k} is not a multiple of the convrot group size {block}")
    y = x.to(torch.float32).reshape(r, k // block, block)
    st = 1
    while st < block:
        v = y.reshape(r, k // block, block // (4 * st), 4, st)
        x0, x1, x2, x3 = v[:, :, :, 0], v[:, :, :, 1], v[:, :, :, 2], v[:, :, :, 3]
        h = 0.5 * (((x0 + x1) + x2) + x3)
        y = torch.stack([h - x3, h - x2, h - x1, h - x0], dim=3).reshape(r, k // block, block)
        st *= 4
    return y.reshape(r, k)


def pack_i4(q: torch.Tensor) -> torch.Tensor:
    """Signed int4 codes [R, K] -> int8 [R, K/2], low nibble = even k
    (experiments/qwen21-kernel/node/__init__.py:82-86)."""
    lo = q[:, 0::2].to(torch.int16) & 0xF
    hi = q[:, 1::2].to(torch.int16) & 0xF
    return (lo | (hi << 4)).to(torch.uint8).view(torch.int8).contiguous()


def pack_u4(q: torch.Tensor) -> torch.Tensor:
    """Unsigned 4-bit codes [R, K] -> uint8 [R, ceil(K/2)], LSB first
    (custom_nodes/comfy-lowbit-loader/kernel.py:75-81). An odd K is padded with a zero code."""
    if q.shape[1] % 2:
        q = torch.cat([q, q.new_zeros(q.shape[0], 1)], dim=1)
    lo = q[:, 0::2].to(torch.int16)
    hi = q[:, 1::2].to(torch.int16)
    return (lo | (hi << 4)).to(torch.uint8).contiguous()


def _hip_quantize(weight: torch.Tensor, convrot_groupsize: int | None, fmt: int):
    """mq_quantize_weight on a device-resident weight [N, K]: (q, scale[, zero]) as the torch
    quantizers below return them."""
    from . import _lib

    if weight.dim() != 2:
        raise ValueError("weight must be 2-D [N, K]")
    dts = {torch.bfloat16: _lib.DT_BF16, torch.float16: _lib.DT_F16, torch.float32: _lib.DT_F32}
    w = weight if weight.dtype in dts else weight.to(torch.float32)
    if w.stride(1) != 1:
        w = w.contiguous()
    n, k = w.shape
    cg = int(convrot_groupsize or 0)
    if cg and cg not in HADAMARD_BLOCKS:
        raise ValueError(f"convrot_groupsize must be one of {HADAMARD_BLOCKS}, got {cg}")
    dev = w.device
    group = fmt in (_lib.WFMT_U4_ASYM_G64, _lib.WFMT_I4_SYM_G64)
    qdt = torch.uint8 if fmt == _lib.WFMT_U4_ASYM_G64 else torch.int8
    q = torch.empty((n, k if fmt == _lib.WFMT_I8_ROW else k // 2), dtype=qdt, device=dev)
    s = torch.empty((n, k // 64) if group else (n,), dtype=torch.float16 if group else torch.float32, device=dev)
    z = torch.empty((n, (k // 64 + 1) // 2), dtype=torch.uint8, device=dev) if fmt == _lib.WFMT_U4_ASYM_G64 else None
    _lib.call("mq_quantize_weight", w.data_ptr(), dts[w.dtype], n, k, w.stride(0), cg, fmt, q.data_ptr(),
              q.stride(0), s.data_ptr(), s.stride(0) if group else 1, _lib.ptr(z), z.stride(0) if z is not None else 0,
              _lib.stream_of(w))
    if group and not torch.isfinite(s).all():
        raise ValueError("group range overflows the fp16 scale")
    return (q, s) if z is None else (q, s, z)


def _on_gpu(weight: torch.Tensor) -> bool:
    return weight.device.type == "cuda"


def _rotated(weight: torch.Tensor, convrot_groupsize: int | None) -> torch.Tensor:
    if weight.dim() != 2:
        raise ValueError("weight must be 2-D [N, K]")
    w = weight.to(torch.float32)
    return fwht(w, convrot_groupsize) if convrot_groupsize else w


def quantize_w4a8_asym_weight(weight: torch.Tensor, group_size: int = 64, convrot_groupsize: int = 256):
    """Configs' W4A8 weight: rotate by H_cg, then per group of `group_size` along K
    lo = min(min w, 0), hi = max(max w, 0), s = fp16((hi - lo) / 15), z = clamp(rne(-lo / s), 0, 15),
    q = clamp(rne(w / s) + z, 0, 15); an all-zero group stores s = z = q = 0.
    Returns (qdata uint8 [N, K/2], scales float16 [N, K/G], zeros uint8 [N, ceil(K/G/2)])."""
    if _on_gpu(weight) and group_size == 64:
        from . import _lib
        return _hip_quantize(weight, convrot_groupsize, _lib.WFMT_U4_ASYM_G64)
    w = _rotated(weight, convrot_groupsize)
    n, k = w.shape
    if k % group_size:
        raise ValueError(f"K={k} must be a multiple of the group size {group_size}")
    g = w.reshape(n, k // group_size, group_size)
    zero = torch.zeros((), dtype=torch.float32, device=w.device)
    lo = torch.minimum(g.amin(dim=2), zero)
    hi = torch.maximum(g.amax(dim=2), zero)
    s16 = _div(hi - lo, 15.0).to(torch.float16)
    if not torch.isfinite(s16).all():
        raise ValueError("group range overflows the fp16 scale")
    s = s16.to(torch.float32)
    is0 = s == 0
    safe = torch.where(is0, torch.ones_like(s), s)
    z = torch.clamp(torch.round(-lo / safe), 0, 15)
    q = torch.clamp(torch.round(g / safe[..., None]) + z[..., None], 0, 15)
    q = torch.where(is0[..., None], torch.zeros_like(q), q)
    z = torch.where(is0, torch.zeros_like(z), z)
    return pack_u4(q.reshape(n, k).to(torch.uint8)), s16.contiguous(), pack_u4(z.to(torch.uint8))


def quantize_w4a4_group_weight(weight: torch.Tensor, group_size: int = 64, convrot_groupsize: int = 64):
    """Configs' W4A4 weight: rotate by H_cg, int4 symmetric per group with fp16 scale
    (tools/svdquant_probe.py:105-115): s = fp16(absmax / 7), q = clamp(rne(w / s), -7, 7).
    Returns (qweight int8 [N, K/2] packed signed, wscales float16 [N, K/G])."""
    if _on_gpu(weight) and group_size == 64:
        from . import _lib
        return _hip_quantize(weight, convrot_groupsize, _lib.WFMT_I4_SYM_G64)
    w = _rotated(weight, convrot_groupsize)
    n, k = w.shape
    if k % group_size:
        raise ValueError(f"K={k} must be a multiple of the group size {group_size}")
    g = w.reshape(n, k // group_size, group_size)
    s16 = _div(g.abs().amax(dim=2), 7.0).to(torch.float16)
    s = s16.to(torch.float32)
    safe = torch.where(s == 0, torch.ones_like(s), s)
    q = torch.clamp(torch.round(g / safe[..., None]), -7, 7)
    q = torch.where((s == 0)[..., None], torch.zeros_like(q), q)
    return pack_i4(q.reshape(n, k).to(torch.int8)), s16.contiguous()


def quantize_convrot_w4a4_weight(weight: torch.Tensor, convrot_groupsize: int = 256, quant_group_size: int = 64,
                                 stochastic_rounding: int = 0):
    """Shipped ConvRot W4A4 weight (comfy-kitchen signature, tools/_formats.py:72-76): rotate by
    H_cg, then per-row s = absmax.clamp(min=1e-10) / 7, q = (w / s).round().clamp(-7, 7)
    (RTN check of tools/gptq_w4a4.py:197-203). Returns (qweight int8 [N, K/2], wscales f32 [N])."""
    if quant_group_size != 64:
        raise ValueError(f"int4 MMA kernel requires quant_group_size 64")
    if stochastic_rounding:
        raise NotImplementedError("stochastic rounding is not part of this path")
    if _on_gpu(weight):
        from . import _lib
        return _hip_quantize(weight, convrot_groupsize, _lib.WFMT_I4_ROW)
    w = _rotated(weight, convrot_groupsize)
    s = _div(torch.clamp(w.abs().amax(dim=1), min=1e-10), 7.0)
    q = torch.clamp(torch.round(w / s[:, None]), -7, 7).to(torch.int8)
    return pack_i4(q), s.contiguous()


def quantize_int8_convrot_weight(weight: torch.Tensor, group_size: int | None = 256):
    """int8_tensorwise weight (tools/_formats.py:128-167; group_size is the rotation block, None
    for --no-convrot): s = absmax.clamp(min=1e-10) / 127, q = (w / s).round().clamp(-127, 127).
    Returns (qdata int8 [N, K], scale f32 [N, 1])."""
    if _on_gpu(weight):
        from . import _lib
        q, s = _hip_quantize(weight, group_size, _lib.WFMT_I8_ROW)
        return q, s[:, None]
    w = _rotated(weight, group_size)
    s = _div(torch.clamp(w.abs().amax(dim=1), min=1e-10), 127.0)
    q = torch.clamp(torch.round(w / s[:, None]), -127, 127).to(torch.int8)
    return q.contiguous(), s[:, None].contiguous()
