"""The caller side of the boundary: opaque torch custom ops for torch.compile, the backend swap
for ComfyUI's `quant_ops.ck`, and a loader that turns a quantized checkpoint's layers into
callables.

* `register_custom_ops()` wraps the linears in `torch.library.custom_op(..., mutates_args=())`
  with fakes returning `x.new_empty((*x.shape[:-1], N))`, the fix `compile_support.py:75-117`
  applies to comfy-kitchen's `convrot_w4a4_linear` (Dynamo otherwise traces into the kernel call
  and fails on a FakeTensor data pointer). Namespace `kitchen_amd`; idempotent.
* `install_backend(ck)` sets the drop-in ops on a comfy-kitchen-like namespace (ComfyUI calls
  `quant_ops.ck.<op>(...)` with keyword arguments, `patches/comfyui_swiglu_triton_env.patch:88-95`).
* `install_compile_support(base)` gives comfy-kitchen's `QuantizedTensor` the other two
  torch.compile fixes of `compile_support.py`: a stable hash for PT2's cache (`:38-72`) and a
  `__tensor_unflatten__` that honours the outer size and stride torch.compile passes under dynamic
  shapes (`:120-165`).
* `layer_linear(tensors, config)` maps one layer's tensors and its `_quantization_metadata` entry
  (`tools/_formats.py:109-111`, `tools/verify_w4a4.py:205-212`) to the op the loader would call,
  with the loader's constants (`quant_group_size=64`, `linear_dtype="int4"`,
  `tools/_native_probe.py:81-100`); `load_quantized(path)` does it for every layer of a file.
"""
from __future__ import annotations

import dataclasses
import json
from pathlib import Path
from typing import Callable

import torch

from . import convert as _conv
from . import ops

LOADER_QUANT_GROUP_SIZE = 64
LOADER_LINEAR_DTYPE = "int4"

_registered: dict[str, Callable] = {}


def register_custom_ops() -> dict[str, Callable]:
    """Register the opaque ops once; returns {name: dispatching wrapper with the ops' signature}."""
    if _registered:
        return dict(_registered)

    @torch.library.custom_op("kitchen_amd::convrot_w4a4_linear", mutates_args=())
    def _convrot(x: torch.Tensor, qweight: torch.Tensor, wscales: torch.Tensor, bias: torch.Tensor | None,
                 convrot_groupsize: int, quant_group_size: int, linear_dtype: str,
                 input_act: str | None) -> torch.Tensor:
        return ops.convrot_w4a4_linear(x, qweight, wscales, bias, convrot_groupsize=convrot_groupsize,
                                       quant_group_size=quant_group_size, linear_dtype=linear_dtype,
                                       input_act=input_act)

    @_convrot.register_fake
    def _(x, qweight, wscales, bias, convrot_groupsize, quant_group_size, linear_dtype, input_act):
        return x.new_empty((*x.shape[:-1], qweight.shape[0]))

    @torch.library.custom_op("kitchen_amd::w4a8_int8_linear", mutates_args=())
    def _w4a8(x: torch.Tensor, qdata: torch.Tensor, s_rel: torch.Tensor, s_channel: torch.Tensor | None,
              codebook: torch.Tensor | None, correction: torch.Tensor | None, bias: torch.Tensor | None,
              group_size: int, convrot_groupsize: int, out_dtype: torch.dtype) -> torch.Tensor:
        return ops.w4a8_int8_linear(x, qdata, s_rel, s_channel, codebook, correction, bias, group_size,
                                    convrot_groupsize, out_dtype)

    @_w4a8.register_fake
    def _(x, qdata, s_rel, s_channel, codebook, correction, bias, group_size, convrot_groupsize, out_dtype):
        return x.new_empty((*x.shape[:-1], qdata.shape[0]), dtype=out_dtype)

    @torch.library.custom_op("kitchen_amd::int8_linear", mutates_args=())
    def _int8(x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor, bias: torch.Tensor | None,
              out_dtype: torch.dtype, convrot: bool, convrot_groupsize: int, input_act: str | None) -> torch.Tensor:
        return ops.int8_linear(x, weight, weight_scale, bias, out_dtype, convrot, convrot_groupsize, input_act)

    @_int8.register_fake
    def _(x, weight, weight_scale, bias, out_dtype, convrot, convrot_groupsize, input_act):
        n = weight_scale.numel() if ops.is_tile16(weight) else weight.shape[0]
        return x.new_empty((*x.shape[:-1], n), dtype=out_dtype)

    def convrot_w4a4_linear(x, qweight, wscales, bias=None, convrot_groupsize=256, quant_group_size=64,
                            linear_dtype="int4", input_act=None):
        return torch.ops.kitchen_amd.convrot_w4a4_linear(x, qweight, wscales, bias, int(convrot_groupsize),
                                                         int(quant_group_size), str(linear_dtype), input_act)

    def w4a8_int8_linear(x, qdata, s_rel, s_channel=None, codebook=None, correction=None, bias=None,
                         group_size=64, convrot_groupsize=256, out_dtype=torch.bfloat16):
        return torch.ops.kitchen_amd.w4a8_int8_linear(x, qdata, s_rel, s_channel, codebook, correction, bias,
                                                      int(group_size), int(convrot_groupsize), out_dtype)

    def int8_linear(x, weight, weight_scale, bias=None, out_dtype=torch.bfloat16, convrot=False,
                    convrot_groupsize=256, input_act=None):
        return torch.ops.kitchen_amd.int8_linear(x, weight, weight_scale, bias, out_dtype, bool(convrot),
                                                 int(convrot_groupsize), input_act)

    _registered.update(convrot_w4a4_linear=convrot_w4a4_linear, w4a8_int8_linear=w4a8_int8_linear,
                       int8_linear=int8_linear)
    return dict(_registered)


def install_compile_support(kitchen_base=None) -> dict:
    """Patch `comfy_kitchen.tensor.base.QuantizedTensor` (or the given module's) for torch.compile;
    idempotent. Returns {"stable_hash": patched now?, "dynamic_shapes": patched now?}."""
    if kitchen_base is None:
        import comfy_kitchen.tensor.base as kitchen_base  # noqa: PLC0415 - only inside a ComfyUI process
    qt = kitchen_base.QuantizedTensor
    done = {"stable_hash": False, "dynamic_shapes": False}

    if not hasattr(qt, "_stable_hash_for_caching"):
        def _stable_hash_for_caching(self) -> str:
            # everything that changes the traced graph: layout, storage and logical type and shape,
            # and the layout parameters that are not tensors
            p = self._params
            parts = [str(self._layout_cls), str(self._qdata.dtype), str(tuple(self._qdata.shape)),
                     str(p.orig_dtype), str(tuple(p.orig_shape))]
            parts += [f"{f.name}={getattr(p, f.name)!r}" for f in dataclasses.fields(p)
                      if f.name not in ("orig_dtype", "orig_shape")
                      and not isinstance(getattr(p, f.name), torch.Tensor)]
            return "|".join(parts)

        qt._stable_hash_for_caching = _stable_hash_for_caching
        done["stable_hash"] = True

    if not getattr(qt, "_kitchen_amd_dynamic_shapes", False):
        def __new__(cls, qdata, layout_cls, params, outer_stride=None):
            return torch.Tensor._make_wrapper_subclass(cls, params.orig_shape, strides=outer_stride,
                                                       device=qdata.device, dtype=params.orig_dtype,
                                                       requires_grad=False)

        def __init__(self, qdata, layout_cls, params, outer_stride=None):
            self._qdata = qdata
            self._layout_cls = layout_cls
            self._params = params

        def __tensor_unflatten__(inner_tensors, ctx, outer_size, outer_stride):
            fields = dict(ctx["non_tensor_fields"])
            fields.update({name: inner_tensors[attr] for name, attr in ctx["tensor_fields"].items()})
            params = ctx["params_class"](**fields)
            # torch.compile passes the (possibly symbolic) size and stride the rebuilt tensor must
            # report; other callers pass scalar placeholders meaning "keep the stored shape"
            if isinstance(outer_size, (tuple, list, torch.Size)):
                params = dataclasses.replace(params, orig_shape=tuple(outer_size))
                return qt(inner_tensors["_qdata"], ctx["layout_cls"], params, outer_stride=outer_stride)
            return qt(inner_tensors["_qdata"], ctx["layout_cls"], params)

        qt.__new__ = __new__
        qt.__init__ = __init__
        qt.__tensor_unflatten__ = staticmethod(__tensor_unflatten__)
        qt._kitchen_amd_dynamic_shapes = True
        done["dynamic_shapes"] = True
    return done


BACKEND_OPS = ("convrot_w4a4_linear", "w4a8_int8_linear", "int8_linear")
BACKEND_FUNCTIONS = ("quantize_int4_rowwise_convrot64", "swiglu_quantize_int4_rowwise_convrot64",
                     "quantize_convrot_w4a4_weight")


def install_backend(ck, compile_safe: bool = True) -> list[str]:
    """Point a comfy-kitchen-like namespace (`comfy.quant_ops.ck`) at this backend; the linears go
    through the opaque custom ops when compile_safe. Returns the names set."""
    from . import weights

    lin = register_custom_ops() if compile_safe else {n: getattr(ops, n) for n in BACKEND_OPS}
    names = []
    for name in BACKEND_OPS:
        setattr(ck, name, lin[name])
        names.append(name)
    for name in BACKEND_FUNCTIONS:
        setattr(ck, name, getattr(ops, name, None) or getattr(weights, name))
        names.append(name)
    return names


def _t(tensors: dict, key: str, required: bool = True):
    if key in tensors:
        return tensors[key]
    if required:
        raise KeyError(f"quantized layer is missing tensor {key!r}")
    return None


def layer_linear(tensors: dict, layer: str, config: dict, compile_safe: bool = False) -> Callable:
    """f(x, bias=None) for one quantized layer, dispatched the way the loader dispatches its format."""
    fmt = config.get("format")
    lin = register_custom_ops() if compile_safe else {n: getattr(ops, n) for n in BACKEND_OPS}
    cg = int(config.get("convrot_groupsize", 256))
    w = _t(tensors, f"{layer}.weight")
    scale = _t(tensors, f"{layer}.weight_scale", required=fmt != "asym_w4a8_int8")
    if fmt in ("convrot_w4a4", "w4a4_sym_g64"):
        dtype = config.get("linear_dtype", LOADER_LINEAR_DTYPE)
        return lambda x, bias=None, input_act=None: lin["convrot_w4a4_linear"](
            x, w, scale, bias, convrot_groupsize=cg, quant_group_size=LOADER_QUANT_GROUP_SIZE, linear_dtype=dtype,
            input_act=input_act)
    if fmt == "w4a8_asym_g64":
        zero = _t(tensors, f"{layer}.weight_zero")
        gs = int(config.get("group_size", 64))
        return lambda x, bias=None, out_dtype=torch.bfloat16: lin["w4a8_int8_linear"](
            x, w, scale, None, None, zero, bias, group_size=gs, convrot_groupsize=cg, out_dtype=out_dtype)
    if fmt == "asym_w4a8_int8":
        s_rel = _t(tensors, f"{layer}.weight_s_rel")
        s_ch = _t(tensors, f"{layer}.weight_s_channel")
        cb = _t(tensors, f"{layer}.weight_codebook", required=False)
        gs = int(config["group_size"])
        if not compile_safe and w.is_cuda:
            # decoded once here, at load: a forward runs only rotate + quantize and the int8 GEMM
            prepared = ops.PreparedW4A8(w, s_rel, s_ch, cb, gs, cg)
            return lambda x, bias=None, out_dtype=torch.bfloat16: prepared(x, bias, out_dtype)
        return lambda x, bias=None, out_dtype=torch.bfloat16: lin["w4a8_int8_linear"](
            x, w, s_rel, s_ch, cb, None, bias, group_size=gs, convrot_groupsize=cg, out_dtype=out_dtype)
    if fmt == "int8_tensorwise":
        # a missing "convrot" key means no rotation: quant_int8.py --no-convrot writes neither key
        # (tools/_formats.py:150-152) and the loader reads layer_conf.get("convrot", False)
        # (tools/verify_w4a4.py:313-315,338)
        convrot = bool(config.get("convrot", False))
        if w.is_cuda and w.dim() == 2 and w.shape[1] >= 192 and w.shape[1] % 64 == 0:
            w = ops.tile_int8_weight(w)   # prepared once at load: same results, whole-line weight loads
        return lambda x, bias=None, out_dtype=torch.bfloat16, input_act=None: lin["int8_linear"](
            x, w, scale, bias, out_dtype, convrot, cg if cg else 256, input_act)
    raise NotImplementedError(f"{layer}: format {fmt!r} is not on this path")


def load_quantized(path, device="cuda", compile_safe: bool = False) -> dict[str, Callable]:
    """{layer: f(x, bias=None)} for every layer listed in the file's _quantization_metadata."""
    path = Path(path)
    header, metadata, data_start = _conv.read_header(path)
    qm = json.loads(metadata.get("_quantization_metadata", "{}") or "{}")
    layers = qm.get("layers", {})
    out = {}
    for layer, config in layers.items():
        keys = [k for k in header if k == f"{layer}.weight" or k.startswith(f"{layer}.weight_")]
        tensors = {k: _conv.read_tensor(path, header[k], data_start).to(device) for k in keys}
        out[layer] = layer_linear(tensors, layer, config, compile_safe)
    return out
