"""ComfyUI registration of the two formats this repository writes (`kitchen_amd.convert`):
`w4a8_asym_g64` (uint4 asymmetric per group of 64, fp16 scale, packed uint4 zero-point) and
`w4a4_sym_g64` (int4 symmetric per group of 64, fp16 scale), both rotated by a Hadamard block
folded into the weight.

ComfyUI's loader finds a format through `comfy.quant_ops.QUANT_ALGOS[format]` (storage type,
parameter tensors, layout class name, `quantize_input`, and the `params_from_state_dict` reader
hook that `_load_quantized_module` calls, `patches/comfyui_awq_w4a16_format.patch:27-32,79-97`) and
the layout class registered under that name (`register_layout_class`). The layout classes here
follow the shape of `custom_nodes/comfy-lowbit-loader/layout.py:27-91`: a frozen `Params`
dataclass over comfy-kitchen's `BaseLayoutParams`, `quantize` / `dequantize`,
`get_plain_tensors`, `state_dict_tensors`. Their `linear` runs the quantized op of this package
(`ops.w4a8_int8_linear` / `ops.convrot_w4a4_linear`); `dequantize` rebuilds the float weight
(used by ComfyUI for LoRA merges and full-precision fallbacks).

How a linear reaches the kernels. ComfyUI's `quant_ops` imports comfy-kitchen's
`register_layout_op` (`patches/comfyui_awq_w4a16_format.patch:54`), the hook through which a
layout supplies its own handler for a torch op on a QuantizedTensor weight; a layout without one
is dequantized to a float weight and multiplied by a plain matmul. `register()` therefore
registers an `aten.linear.default` handler for each layout whenever `register_layout_op` is
present: `handler(func, args, kwargs)` takes (input, weight, bias) and runs the layout's
`linear` on the GPU (falling back to dequantize + `F.linear` for host tensors). The decorator's
exact signature is not in the reference tree (comfy-kitchen is absent); the form used is
`register_layout_op(torch_op, layout_cls)(handler)`. Without `register_layout_op` ComfyUI runs these
formats through `dequantize`.

comfy and comfy_kitchen are not imported at module load: `register()` imports them (or takes
stand-ins, as the CPU tests do) when a ComfyUI process calls it.
"""
from __future__ import annotations

import dataclasses
import logging

import torch

from . import ops, weights

W4A8_FORMAT, W4A8_LAYOUT = "w4a8_asym_g64", "KitchenAMDW4A8AsymG64Layout"
W4A4_FORMAT, W4A4_LAYOUT = "w4a4_sym_g64", "KitchenAMDW4A4SymG64Layout"
GROUP = 64


def _unpack_u4(p: torch.Tensor) -> torch.Tensor:
    """Packed uint4 [R, C] (low nibble first) -> codes uint8 [R, 2C]."""
    p = p.view(torch.uint8)
    return torch.stack([p & 0xF, p >> 4], dim=-1).reshape(p.shape[0], -1)


def _unpack_i4(p: torch.Tensor) -> torch.Tensor:
    """Packed signed int4 [R, C] (low nibble first) -> codes int8 [R, 2C]."""
    u = _unpack_u4(p).to(torch.int8)
    return torch.where(u >= 8, u - 16, u)


def _unrotate(w_rot: torch.Tensor, cg: int) -> torch.Tensor:
    """W from W_rot = W H_cg: H_cg is symmetric and orthogonal, its own inverse."""
    return weights.fwht(w_rot, cg) if cg else w_rot


def dequantize_w4a8(qdata, scale, zero, group_size: int, convrot_groupsize: int, dtype) -> torch.Tensor:
    n = qdata.shape[0]
    q = _unpack_u4(qdata).float()
    k = q.shape[1]
    g = k // group_size
    z = _unpack_u4(zero)[:, :g].float()
    w = (q.reshape(n, g, group_size) - z[..., None]) * scale.float()[..., None]
    return _unrotate(w.reshape(n, k), convrot_groupsize).to(dtype)


def dequantize_w4a4(qdata, scale, group_size: int, convrot_groupsize: int, dtype) -> torch.Tensor:
    n = qdata.shape[0]
    q = _unpack_i4(qdata).float()
    k = q.shape[1]
    w = q.reshape(n, k // group_size, group_size) * scale.float()[..., None]
    return _unrotate(w.reshape(n, k), convrot_groupsize).to(dtype)


def _cfg_int(layer_conf: dict, key: str, default: int) -> int:
    """A layer's integer setting, from the top level or its nested "params" (as the AWQ reader does,
    patches/comfyui_awq_w4a16_format.patch:85-88)."""
    params = layer_conf.get("params", {})
    if not isinstance(params, dict):
        params = {}
    return int(layer_conf.get(key, params.get(key, default)))


def w4a8_params_from_state_dict(layer_name, module, weight, pop_scale, layer_conf) -> dict:
    """Reader hook of w4a8_asym_g64: the layer's fp16 group scales and packed zero-points."""
    scale, zero = pop_scale("weight_scale"), pop_scale("weight_zero")
    if scale is None or zero is None:
        raise ValueError(f"{W4A8_FORMAT}: missing weight_scale / weight_zero for layer {layer_name}")
    return {"scale": scale, "zero": zero, "group_size": _cfg_int(layer_conf, "group_size", GROUP),
            "convrot_groupsize": _cfg_int(layer_conf, "convrot_groupsize", 256)}


def w4a4_params_from_state_dict(layer_name, module, weight, pop_scale, layer_conf) -> dict:
    """Reader hook of w4a4_sym_g64: the layer's fp16 group scales."""
    scale = pop_scale("weight_scale")
    if scale is None:
        raise ValueError(f"{W4A4_FORMAT}: missing weight_scale for layer {layer_name}")
    return {"scale": scale, "group_size": _cfg_int(layer_conf, "group_size", GROUP),
            "convrot_groupsize": _cfg_int(layer_conf, "convrot_groupsize", 64)}


QUANT_ALGO_ENTRIES = {
    W4A8_FORMAT: {"storage_t": torch.uint8, "parameters": {"weight_scale", "weight_zero"},
                  "comfy_tensor_layout": W4A8_LAYOUT, "quantize_input": False,
                  "params_from_state_dict": w4a8_params_from_state_dict},
    W4A4_FORMAT: {"storage_t": torch.int8, "parameters": {"weight_scale"},
                  "comfy_tensor_layout": W4A4_LAYOUT, "quantize_input": False,
                  "params_from_state_dict": w4a4_params_from_state_dict},
}


def make_layout_classes(quantized_layout, base_params) -> dict:
    """The two layout classes over comfy-kitchen's `QuantizedLayout` / `BaseLayoutParams`."""

    class W4A8AsymG64Layout(quantized_layout):
        """uint4 codes with a per-group affine map along K: W_rot = (q - z) * s, W = W_rot H."""

        MIN_SM_VERSION = None
        QUANTIZES_INPUT = False
        FORMAT = W4A8_FORMAT

        @dataclasses.dataclass(frozen=True)
        class Params(base_params):
            zero: torch.Tensor
            group_size: int = GROUP
            convrot_groupsize: int = 256

            def _tensor_fields(self):
                return ["scale", "zero"]

            def _validate_tensor_fields(self):
                return

        @classmethod
        def quantize(cls, tensor, group_size: int = GROUP, convrot_groupsize: int = 256, **kwargs):
            qd, s16, zp = weights.quantize_w4a8_asym_weight(tensor, group_size, convrot_groupsize)
            return qd, cls.Params(scale=s16, orig_dtype=tensor.dtype, orig_shape=tuple(tensor.shape), zero=zp,
                                  group_size=group_size, convrot_groupsize=convrot_groupsize)

        @classmethod
        def dequantize(cls, qdata, params):
            return dequantize_w4a8(qdata, params.scale, params.zero, params.group_size, params.convrot_groupsize,
                                   params.orig_dtype)

        @classmethod
        def get_plain_tensors(cls, qtensor):
            return qtensor._qdata, qtensor._params.scale, qtensor._params.zero

        @classmethod
        def state_dict_tensors(cls, qdata, params):
            return {"": qdata, "_scale": params.scale, "_zero": params.zero}

        @classmethod
        def linear(cls, x, qdata, params, bias=None):
            return ops.w4a8_int8_linear(x, qdata, params.scale, None, None, params.zero, bias, params.group_size,
                                        params.convrot_groupsize, x.dtype)

    class W4A4SymG64Layout(quantized_layout):
        """int4 codes with a per-group scale along K: W_rot = q * s, W = W_rot H."""

        MIN_SM_VERSION = None
        QUANTIZES_INPUT = False
        FORMAT = W4A4_FORMAT

        @dataclasses.dataclass(frozen=True)
        class Params(base_params):
            group_size: int = GROUP
            convrot_groupsize: int = 64

            def _tensor_fields(self):
                return ["scale"]

            def _validate_tensor_fields(self):
                return

        @classmethod
        def quantize(cls, tensor, group_size: int = GROUP, convrot_groupsize: int = 64, **kwargs):
            qw, s16 = weights.quantize_w4a4_group_weight(tensor, group_size, convrot_groupsize)
            return qw, cls.Params(scale=s16, orig_dtype=tensor.dtype, orig_shape=tuple(tensor.shape),
                                  group_size=group_size, convrot_groupsize=convrot_groupsize)

        @classmethod
        def dequantize(cls, qdata, params):
            return dequantize_w4a4(qdata, params.scale, params.group_size, params.convrot_groupsize,
                                   params.orig_dtype)

        @classmethod
        def get_plain_tensors(cls, qtensor):
            return qtensor._qdata, qtensor._params.scale

        @classmethod
        def state_dict_tensors(cls, qdata, params):
            return {"": qdata, "_scale": params.scale}

        @classmethod
        def linear(cls, x, qdata, params, bias=None):
            return ops.convrot_w4a4_linear(x, qdata, params.scale, bias, convrot_groupsize=params.convrot_groupsize,
                                           quant_group_size=params.group_size, linear_dtype="int4")

    return {W4A8_LAYOUT: W4A8AsymG64Layout, W4A4_LAYOUT: W4A4SymG64Layout}


def _use_kernels(x: torch.Tensor, qdata: torch.Tensor) -> bool:
    return x.is_cuda and qdata.is_cuda and x.dtype in ops.FLOAT_TYPES


def make_linear_handler(layout_cls):
    """The aten.linear.default handler of a layout: `handler(func, args, kwargs)` with args
    (input, QuantizedTensor weight[, bias]); the weight carries `_qdata` and `_params`."""

    def handler(func, args, kwargs):
        kwargs = kwargs or {}
        x, w = args[0], args[1]
        bias = args[2] if len(args) > 2 else kwargs.get("bias")
        qdata, params = w._qdata, w._params
        if _use_kernels(x, qdata):
            return layout_cls.linear(x, qdata, params, bias)
        wf = layout_cls.dequantize(qdata, params).to(device=x.device, dtype=x.dtype)
        return torch.nn.functional.linear(x, wf, None if bias is None else bias.to(x.dtype))

    handler.__name__ = f"{layout_cls.__name__}_linear"
    return handler


def register(quant_ops=None, kitchen_base=None) -> dict:
    """Register both layouts and QUANT_ALGOS entries with ComfyUI (idempotent). `quant_ops` is
    `comfy.quant_ops` and `kitchen_base` `comfy_kitchen.tensor.base`; both are imported when not
    given. Returns {layout name: class}."""
    if quant_ops is None:
        import comfy.quant_ops as quant_ops  # noqa: PLC0415 - only inside a ComfyUI process
    if kitchen_base is None:
        import comfy_kitchen.tensor.base as kitchen_base  # noqa: PLC0415
    existing = getattr(quant_ops, "_kitchen_amd_layouts", None)
    if existing is not None:
        return dict(existing)
    classes = make_layout_classes(kitchen_base.QuantizedLayout, kitchen_base.BaseLayoutParams)
    layout_op = getattr(quant_ops, "register_layout_op", None)
    for name, cls in classes.items():
        quant_ops.register_layout_class(name, cls)
        if layout_op is not None:
            layout_op(torch.ops.aten.linear.default, cls)(make_linear_handler(cls))
    for fmt, entry in QUANT_ALGO_ENTRIES.items():
        quant_ops.QUANT_ALGOS[fmt] = dict(entry)
    quant_ops._kitchen_amd_layouts = classes
    if layout_op is None:
        logging.warning("kitchen_amd: comfy.quant_ops has no register_layout_op; %s layers will be "
                        "dequantized and run through a plain matmul", ", ".join(QUANT_ALGO_ENTRIES))
    logging.info("kitchen_amd: registered %s with ComfyUI", ", ".join(QUANT_ALGO_ENTRIES))
    return dict(classes)
