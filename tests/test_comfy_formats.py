"""ComfyUI registration of the formats this repository writes, and the torch.compile fixes for
comfy-kitchen's QuantizedTensor, on the CPU with stand-in comfy / comfy_kitchen modules (the real
ones are not installed; the reference's own tests inject stand-ins the same way,
tools/test_formats_e2e.py:68-85)."""
import dataclasses
import types

import numpy as np
import pytest
import torch

from kitchen_amd import comfy_formats as CF
from kitchen_amd import comfy_glue as G
from kitchen_amd import convert as C
from kitchen_amd import ops, weights


@dataclasses.dataclass(frozen=True)
class FakeBaseParams:
    """The fields comfy-kitchen's BaseLayoutParams carries (custom_nodes/comfy-lowbit-loader/layout.py:33-41,
    tools/quant_te_residuos.py:99): scale, orig_dtype, orig_shape."""
    scale: torch.Tensor
    orig_dtype: torch.dtype
    orig_shape: tuple


class FakeQuantizedLayout:
    pass


def _fake_comfy(with_layout_op=True):
    registered = {}
    quant_ops = types.SimpleNamespace(QUANT_ALGOS={"int8_tensorwise": {}},
                                      register_layout_class=lambda name, cls: registered.__setitem__(name, cls),
                                      get_layout_class=lambda name: registered[name])
    if with_layout_op:
        quant_ops.LAYOUT_OPS = {}

        def register_layout_op(torch_op, layout_cls):
            def deco(handler):
                quant_ops.LAYOUT_OPS[(torch_op, layout_cls)] = handler
                return handler
            return deco

        quant_ops.register_layout_op = register_layout_op
    base = types.SimpleNamespace(QuantizedLayout=FakeQuantizedLayout, BaseLayoutParams=FakeBaseParams)
    return quant_ops, base, registered


class StandInQuantizedTensor(torch.Tensor):
    """A weight as ComfyUI holds it (QuantizedTensor: _qdata, _params, its layout class). F.linear on
    it looks up the layout's aten.linear.default handler in the layout-op registry, as a layout
    dispatch does, and dequantizes when the layout has none."""

    @staticmethod
    def __new__(cls, qdata, layout_cls, params, registry):
        return torch.Tensor._make_wrapper_subclass(cls, params.orig_shape, dtype=params.orig_dtype,
                                                   device=qdata.device)

    def __init__(self, qdata, layout_cls, params, registry):
        self._qdata, self._layout_cls, self._params, self._registry = qdata, layout_cls, params, registry

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        if func is torch.nn.functional.linear:
            w = args[1]
            handler = w._registry.get((torch.ops.aten.linear.default, w._layout_cls))
            if handler is not None:
                return handler(torch.ops.aten.linear.default, args, kwargs)
            wf = w._layout_cls.dequantize(w._qdata, w._params)
            return torch.nn.functional.linear(args[0], wf, *args[2:], **kwargs)
        with torch._C.DisableTorchFunctionSubclass():
            return func(*args, **kwargs)

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        raise NotImplementedError(f"stand-in weight: {func} is not modelled")


def test_register_adds_quant_algos_and_layouts():
    quant_ops, base, registered = _fake_comfy()
    classes = CF.register(quant_ops, base)
    assert set(registered) == {CF.W4A8_LAYOUT, CF.W4A4_LAYOUT} and registered == classes
    for fmt, layout, storage, params in ((CF.W4A8_FORMAT, CF.W4A8_LAYOUT, torch.uint8, {"weight_scale", "weight_zero"}),
                                         (CF.W4A4_FORMAT, CF.W4A4_LAYOUT, torch.int8, {"weight_scale"})):
        e = quant_ops.QUANT_ALGOS[fmt]
        assert e["comfy_tensor_layout"] == layout and e["storage_t"] == storage and e["parameters"] == params
        assert e["quantize_input"] is False and callable(e["params_from_state_dict"])
        assert issubclass(registered[layout], FakeQuantizedLayout)
    # idempotent: a second call registers nothing new
    assert CF.register(quant_ops, base) == classes
    assert "int8_tensorwise" in quant_ops.QUANT_ALGOS
    # each layout has its aten.linear handler in the layout-op registry
    assert set(quant_ops.LAYOUT_OPS) == {(torch.ops.aten.linear.default, classes[CF.W4A8_LAYOUT]),
                                         (torch.ops.aten.linear.default, classes[CF.W4A4_LAYOUT])}


def test_linear_dispatch_reaches_the_layout_handler(monkeypatch):
    """F.linear on a QuantizedTensor weight goes through the registered aten.linear handler: on the
    GPU to the layout's quantized op (recorded here), on the host to dequantize + F.linear."""
    quant_ops, base, _ = _fake_comfy()
    classes = CF.register(quant_ops, base)
    torch.manual_seed(0)
    w = torch.randn(32, 256)
    x = torch.randn(5, 256)
    b = torch.randn(32)
    for layout, q in ((CF.W4A8_LAYOUT, classes[CF.W4A8_LAYOUT].quantize(w)),
                      (CF.W4A4_LAYOUT, classes[CF.W4A4_LAYOUT].quantize(w))):
        cls = classes[layout]
        qdata, params = q
        wq = StandInQuantizedTensor(qdata, cls, params, quant_ops.LAYOUT_OPS)
        # host tensors: the handler dequantizes (what the kernels approximate within the int codes)
        y = torch.nn.functional.linear(x, wq, b)
        ref = x @ cls.dequantize(qdata, params).T + b
        assert torch.allclose(y, ref, atol=1e-4, rtol=1e-4)
        # device tensors: the handler calls the layout's quantized op with the weight's parameters
        calls = []
        monkeypatch.setattr(CF, "_use_kernels", lambda x_, q_: True)
        monkeypatch.setattr(ops, "w4a8_int8_linear", lambda *a, **k: calls.append(("w4a8", a, k)) or "w4a8")
        monkeypatch.setattr(ops, "convrot_w4a4_linear", lambda *a, **k: calls.append(("w4a4", a, k)) or "w4a4")
        out = torch.nn.functional.linear(x, wq, b)
        monkeypatch.undo()
        kind = "w4a8" if layout == CF.W4A8_LAYOUT else "w4a4"
        assert out == kind and len(calls) == 1 and calls[0][0] == kind
        a = calls[0][1]
        assert a[0] is x and a[1] is qdata and a[2] is params.scale
        if kind == "w4a8":
            assert a[5] is params.zero and a[6] is b and a[7] == 64 and a[8] == 256
        else:
            assert a[3] is b and calls[0][2]["convrot_groupsize"] == params.convrot_groupsize
    # without register_layout_op the layers still load; linear then dequantizes
    quant_ops2, base2, _ = _fake_comfy(with_layout_op=False)
    assert set(CF.register(quant_ops2, base2)) == {CF.W4A8_LAYOUT, CF.W4A4_LAYOUT}


def test_reader_hooks_follow_the_converter_output(tmp_path):
    # the tensors and per-layer config convert.py writes are what the readers pop and parse
    from safetensors.torch import save_file

    src, out = tmp_path / "m.safetensors", tmp_path / "q.safetensors"
    save_file({"a.weight": torch.randn(16, 256), "b.weight": torch.randn(32, 512)}, str(src))
    C.convert(src, out, C.make_format("w4a8_asym_g64"), "cpu")
    header, metadata, start = C.read_header(out)
    import json

    layers = json.loads(metadata["_quantization_metadata"])["layers"]
    conf = layers["b"]
    tensors = {k: C.read_tensor(out, header[k], start) for k in header if k.startswith("b.")}
    popped = []

    def pop_scale(name):
        popped.append(name)
        return tensors.pop(f"b.{name}", None)

    p = CF.w4a8_params_from_state_dict("b", None, tensors["b.weight"], pop_scale, conf)
    assert popped == ["weight_scale", "weight_zero"]
    assert p["scale"].dtype == torch.float16 and p["scale"].shape == (32, 8)
    assert p["zero"].shape == (32, 4) and p["group_size"] == 64 and p["convrot_groupsize"] == 256
    # nested "params" are honoured like the AWQ reader does; missing tensors are an error
    p = CF.w4a4_params_from_state_dict("x", None, None, lambda n: torch.zeros(2, 2),
                                       {"format": "w4a4_sym_g64", "params": {"convrot_groupsize": 16}})
    assert p["convrot_groupsize"] == 16 and p["group_size"] == 64
    with pytest.raises(ValueError, match="weight_zero"):
        CF.w4a8_params_from_state_dict("b", None, None, lambda n: None if n == "weight_zero" else 1, {})


@pytest.mark.parametrize("fmt", ["w4a8", "w4a4"])
def test_layout_quantize_dequantize_round_trip(fmt):
    quant_ops, base, _ = _fake_comfy()
    classes = CF.register(quant_ops, base)
    layout = classes[CF.W4A8_LAYOUT if fmt == "w4a8" else CF.W4A4_LAYOUT]
    g = torch.Generator().manual_seed(3)
    w = (torch.randn(48, 512, generator=g) * 0.02).to(torch.bfloat16)
    qdata, params = layout.quantize(w)
    assert params.orig_shape == (48, 512) and params.orig_dtype == torch.bfloat16
    wd = layout.dequantize(qdata, params)
    assert wd.dtype == torch.bfloat16 and wd.shape == w.shape
    # the group quantizer's error bound (half a step per element, rotation is orthogonal) on the
    # rotated weight carries over to W: ||W - Wd|| = ||W H - Wd H||
    wr = weights.fwht(w.float(), params.convrot_groupsize)
    step = params.scale.float().repeat_interleave(64, dim=1)
    err_rot = (weights.fwht(wd.float(), params.convrot_groupsize) - wr).abs()
    assert (err_rot <= 0.5 * step + 2e-3 * wr.abs().max()).all()
    rel = ((wd.float() - w.float()).norm() / w.float().norm()).item()
    assert rel < 0.12          # step / sqrt(12) relative to the std of a Gaussian group: ~0.09-0.10
    sd = layout.state_dict_tensors(qdata, params)
    assert sd[""] is qdata and sd["_scale"] is params.scale
    assert ("_zero" in sd) == (fmt == "w4a8")


def test_layout_linear_calls_the_quantized_ops(monkeypatch):
    quant_ops, base, _ = _fake_comfy()
    classes = CF.register(quant_ops, base)
    calls = []
    monkeypatch.setattr(ops, "w4a8_int8_linear", lambda *a, **k: calls.append(("w4a8", a, k)) or "y")
    monkeypatch.setattr(ops, "convrot_w4a4_linear", lambda *a, **k: calls.append(("w4a4", a, k)) or "y")
    x = torch.zeros(2, 256, dtype=torch.float16)
    p8 = classes[CF.W4A8_LAYOUT].Params(scale="s", orig_dtype=torch.bfloat16, orig_shape=(8, 256), zero="z")
    classes[CF.W4A8_LAYOUT].linear(x, "q", p8, bias="b")
    name, a, _ = calls[-1]
    assert name == "w4a8" and a[1:] == ("q", "s", None, None, "z", "b", 64, 256, torch.float16)
    p4 = classes[CF.W4A4_LAYOUT].Params(scale="s", orig_dtype=torch.bfloat16, orig_shape=(8, 256))
    classes[CF.W4A4_LAYOUT].linear(x, "q", p4)
    name, a, k = calls[-1]
    assert name == "w4a4" and k == {"convrot_groupsize": 64, "quant_group_size": 64, "linear_dtype": "int4"}


# ---- torch.compile support for comfy-kitchen's QuantizedTensor (compile_support.py:38-72,120-165)

@dataclasses.dataclass(frozen=True)
class _Params:
    scale: torch.Tensor
    orig_dtype: torch.dtype
    orig_shape: tuple
    group_size: int = 64
    convrot_groupsize: int = 256


def _fake_kitchen_base():
    """A QuantizedTensor shaped like comfy-kitchen's (a wrapper subclass over _qdata and _params)
    whose __tensor_unflatten__ ignores the outer size, the defect the patch fixes."""

    class QuantizedTensor(torch.Tensor):
        @staticmethod
        def __new__(cls, qdata, layout_cls, params):
            return torch.Tensor._make_wrapper_subclass(cls, params.orig_shape, device=qdata.device,
                                                       dtype=params.orig_dtype, requires_grad=False)

        def __init__(self, qdata, layout_cls, params):
            self._qdata, self._layout_cls, self._params = qdata, layout_cls, params

        def __tensor_flatten__(self):
            ctx = {"layout_cls": self._layout_cls, "params_class": type(self._params),
                   "tensor_fields": {"scale": "_scale"},
                   "non_tensor_fields": {f.name: getattr(self._params, f.name)
                                         for f in dataclasses.fields(self._params) if f.name != "scale"}}
            return ["_qdata", "_scale"], ctx

        @staticmethod
        def __tensor_unflatten__(inner_tensors, ctx, outer_size, outer_stride):
            fields = dict(ctx["non_tensor_fields"], scale=inner_tensors["_scale"])
            return QuantizedTensor(inner_tensors["_qdata"], ctx["layout_cls"], ctx["params_class"](**fields))

        @classmethod
        def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
            raise NotImplementedError(f"{func} on a stand-in QuantizedTensor")

    return types.SimpleNamespace(QuantizedTensor=QuantizedTensor)


def test_compile_support_dynamic_shapes_and_stable_hash():
    base = _fake_kitchen_base()
    qt = base.QuantizedTensor
    q = torch.zeros(8, 128, dtype=torch.uint8)
    p = _Params(scale=torch.ones(8, 4), orig_dtype=torch.bfloat16, orig_shape=(8, 256))
    t = qt(q, "KitchenAMDW4A8AsymG64Layout", p)
    inner = {"_qdata": q, "_scale": p.scale}
    _, ctx = t.__tensor_flatten__()
    # before: the outer size torch.compile passes is dropped
    assert qt.__tensor_unflatten__(inner, ctx, (4, 256), (256, 1)).shape == (8, 256)
    assert not hasattr(qt, "_stable_hash_for_caching")
    assert G.install_compile_support(base) == {"stable_hash": True, "dynamic_shapes": True}
    assert G.install_compile_support(base) == {"stable_hash": False, "dynamic_shapes": False}   # idempotent
    t2 = qt.__tensor_unflatten__(inner, ctx, (4, 256), (256, 1))
    assert t2.shape == (4, 256) and t2.stride() == (256, 1) and t2._params.orig_shape == (4, 256)
    # scalar placeholders keep the stored shape
    assert qt.__tensor_unflatten__(inner, ctx, 0, 0).shape == (8, 256)
    t = qt(q, "KitchenAMDW4A8AsymG64Layout", p)
    h = t._stable_hash_for_caching()
    assert "KitchenAMDW4A8AsymG64Layout" in h and "torch.uint8" in h and "(8, 256)" in h
    assert "convrot_groupsize=256" in h and "scale" not in h
    other = qt(q, "KitchenAMDW4A8AsymG64Layout", dataclasses.replace(p, convrot_groupsize=64))
    assert other._stable_hash_for_caching() != h
    assert qt(q, "KitchenAMDW4A8AsymG64Layout", p)._stable_hash_for_caching() == h
