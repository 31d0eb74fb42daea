"""Caller-side glue on the CPU: the custom ops' fakes (the torch.compile contract of
compile_support.py:75-117), the backend swap, and the format -> op mapping of the loader."""
import types

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from kitchen_amd import comfy_glue as G
from kitchen_amd import convert as C
from kitchen_amd import ops


def test_fakes_give_output_shapes_without_running_kernels():
    G.register_custom_ops()
    with FakeTensorMode():
        x = torch.empty(2, 7, 512, dtype=torch.bfloat16)
        h = torch.empty(5, 1024, dtype=torch.bfloat16)
        y = torch.ops.kitchen_amd.convrot_w4a4_linear(x, torch.empty(96, 256, dtype=torch.int8),
                                                      torch.empty(96), None, 256, 64, "int4", None)
        assert y.shape == (2, 7, 96) and y.dtype == torch.bfloat16
        y = torch.ops.kitchen_amd.convrot_w4a4_linear(h, torch.empty(64, 256, dtype=torch.int8),
                                                      torch.empty(64, 8, dtype=torch.float16), None, 64, 64, "int4",
                                                      "swiglu")
        assert y.shape == (5, 64)
        y = torch.ops.kitchen_amd.w4a8_int8_linear(x, torch.empty(48, 256, dtype=torch.uint8),
                                                   torch.empty(48, 8, dtype=torch.float16), None, None,
                                                   torch.empty(48, 4, dtype=torch.uint8), None, 64, 256, torch.float16)
        assert y.shape == (2, 7, 48) and y.dtype == torch.float16
        y = torch.ops.kitchen_amd.int8_linear(x, torch.empty(32, 512, dtype=torch.int8), torch.empty(32, 1), None,
                                              torch.bfloat16, True, 256, None)
        assert y.shape == (2, 7, 32)
    assert G.register_custom_ops().keys() == {"convrot_w4a4_linear", "w4a8_int8_linear", "int8_linear"}


def test_install_backend_sets_every_name():
    ck = types.SimpleNamespace()
    names = G.install_backend(ck)
    for n in names:
        assert callable(getattr(ck, n))
    assert ck.w4a8_int8_linear is G.register_custom_ops()["w4a8_int8_linear"]
    ck2 = types.SimpleNamespace()
    G.install_backend(ck2, compile_safe=False)
    assert ck2.convrot_w4a4_linear is ops.convrot_w4a4_linear


@pytest.fixture
def record(monkeypatch):
    calls = []
    for name in G.BACKEND_OPS:
        monkeypatch.setattr(ops, name, lambda *a, _n=name, **k: calls.append((_n, a, k)) or "y")
    return calls


def test_layer_linear_maps_each_format(record):
    x = torch.zeros(3, 512)
    w4 = {"l.weight": torch.zeros(8, 256, dtype=torch.int8), "l.weight_scale": torch.zeros(8)}
    G.layer_linear(w4, "l", {"format": "convrot_w4a4", "convrot_groupsize": 128})(x)
    name, a, k = record[-1]
    assert name == "convrot_w4a4_linear" and k == {"convrot_groupsize": 128, "quant_group_size": 64,
                                                   "linear_dtype": "int4", "input_act": None}
    w8 = {"l.weight": torch.zeros(8, 256, dtype=torch.uint8), "l.weight_scale": torch.zeros(8, 8, dtype=torch.float16),
          "l.weight_zero": torch.zeros(8, 4, dtype=torch.uint8)}
    G.layer_linear(w8, "l", {"format": "w4a8_asym_g64", "group_size": 64, "convrot_groupsize": 256})(x)
    name, a, k = record[-1]
    assert name == "w4a8_int8_linear" and a[5] is w8["l.weight_zero"] and k["group_size"] == 64
    ship = {"l.weight": torch.zeros(8, 256, dtype=torch.int8), "l.weight_s_rel": torch.zeros(8, 32, dtype=torch.uint8),
            "l.weight_s_channel": torch.zeros(8), "l.weight_codebook": torch.zeros(16)}
    G.layer_linear(ship, "l", {"format": "asym_w4a8_int8", "group_size": 16, "convrot_groupsize": 256})(x)
    name, a, k = record[-1]
    assert name == "w4a8_int8_linear" and a[3] is ship["l.weight_s_channel"] and a[4] is ship["l.weight_codebook"]
    i8 = {"l.weight": torch.zeros(8, 512, dtype=torch.int8), "l.weight_scale": torch.zeros(8, 1)}
    G.layer_linear(i8, "l", {"format": "int8_tensorwise", "convrot": False, "convrot_groupsize": 0})(x)
    name, a, k = record[-1]
    assert name == "int8_linear" and a[5] is False
    # quant_int8.py --no-convrot writes neither "convrot" nor "convrot_groupsize"
    # (tools/_formats.py:148-152): absence means no rotation (tools/verify_w4a4.py:313-315,338)
    G.layer_linear(i8, "l", {"format": "int8_tensorwise"})(x)
    name, a, k = record[-1]
    assert name == "int8_linear" and a[5] is False
    G.layer_linear(i8, "l", {"format": "int8_tensorwise", "convrot": True})(x)
    name, a, k = record[-1]
    assert a[5] is True and a[6] == 256
    G.layer_linear(i8, "l", {"format": "int8_tensorwise", "convrot": True, "convrot_groupsize": 64})(x)
    name, a, k = record[-1]
    assert a[5] is True and a[6] == 64
    with pytest.raises(NotImplementedError):
        G.layer_linear(i8, "l", {"format": "nvfp4"})
    with pytest.raises(KeyError):
        G.layer_linear({}, "l", {"format": "convrot_w4a4"})


def test_load_quantized_reads_the_converters_output(tmp_path, record):
    from safetensors.torch import save_file

    src, out = tmp_path / "m.safetensors", tmp_path / "q.safetensors"
    save_file({"a.weight": torch.randn(16, 256), "b.weight": torch.randn(32, 512), "b.bias": torch.zeros(32)}, str(src))
    C.convert(src, out, C.make_format("w4a8_asym_g64"), "cpu")
    layers = G.load_quantized(out, device="cpu")
    assert set(layers) == {"a", "b"}
    layers["b"](torch.zeros(2, 512))
    name, a, k = record[-1]
    assert name == "w4a8_int8_linear" and a[1].shape == (32, 256) and a[2].dtype == torch.float16
