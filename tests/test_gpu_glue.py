"""GPU checks of the caller-side glue: the opaque custom ops under torch.compile (no tracing into
the kernels, same result as eager), and a checkpoint converted on the GPU equals the CPU
conversion byte for byte and runs through the loader mapping to the oracle's result."""
import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import kitchen_amd as ck
from kitchen_amd import comfy_glue as G
from kitchen_amd import convert as C
from kitchen_amd import synth
from oracle import gemm, linear, quant

pytestmark = pytest.mark.gpu


def test_custom_op_under_torch_compile(gpu_device):
    print("[glue] torch.compile over kitchen_amd::w4a8_int8_linear", flush=True)
    lin = G.register_custom_ops()
    m, n, k = 256, 1024, 3072
    w = torch.from_numpy(synth.weight(n, k, seed=1)).to(gpu_device)
    qd, s16, zp = ck.quantize_w4a8_asym_weight(w, 64, 256)
    x = synth.to_bf16_tensor(synth.activations(m, k, seed=2), gpu_device)

    def f(x):
        return lin["w4a8_int8_linear"](x, qd, s16, None, None, zp, None, 64, 256, torch.bfloat16).float() * 2.0

    eager = f(x)
    compiled = torch.compile(f, fullgraph=True, backend="aot_eager")
    got = compiled(x)
    torch.cuda.synchronize()
    assert torch.equal(got, eager)
    assert torch.equal(eager, ck.w4a8_int8_linear(x, qd, s16, None, None, zp, None, 64, 256).float() * 2.0)


def test_gpu_conversion_matches_cpu_and_runs(gpu_device, tmp_path):
    print("[glue] convert on cuda vs cpu, then load and run", flush=True)
    g = torch.Generator().manual_seed(3)
    src = tmp_path / "m.safetensors"
    tensors = {"blk.fc1.weight": (torch.randn(512, 3072, generator=g) * 0.02).to(torch.bfloat16),
               "blk.fc1.bias": torch.zeros(512, dtype=torch.bfloat16),
               "blk.norm.weight": torch.ones(3072, dtype=torch.bfloat16)}
    save_file(tensors, str(src))
    fmt = C.make_format("w4a8_asym_g64")
    C.convert(src, tmp_path / "gpu.safetensors", fmt, device="cuda")
    C.convert(src, tmp_path / "cpu.safetensors", fmt, device="cpu")
    assert (tmp_path / "gpu.safetensors").read_bytes() == (tmp_path / "cpu.safetensors").read_bytes()
    layers = G.load_quantized(tmp_path / "gpu.safetensors", device=gpu_device)
    xb = synth.activations(128, 3072, seed=4)
    y = layers["blk.fc1"](synth.to_bf16_tensor(xb, gpu_device))
    torch.cuda.synchronize()
    w = tensors["blk.fc1.weight"].float().numpy()
    q0, s0, z0 = quant.quant_weight_u4_asym(linear.rotate_weight(w, 256), 64)
    ref = linear.w4a8_asym_linear(synth.bf16_bits_to_f32(xb), q0, s0, z0, None, 256, 64)
    assert gemm.rel_l2(ref.y, y.float().cpu().numpy()) < 4e-3


def test_layout_op_linear_runs_the_kernels(gpu_device):
    """F.linear on a QuantizedTensor weight of each registered layout reaches the layout's
    aten.linear handler and runs the HIP linear: the output equals the op's bit for bit."""
    from kitchen_amd import comfy_formats as CF
    from test_comfy_formats import StandInQuantizedTensor, _fake_comfy

    print("[glue] layout-op aten.linear handler on the GPU", flush=True)
    quant_ops, base, _ = _fake_comfy()
    classes = CF.register(quant_ops, base)
    w = torch.from_numpy(synth.weight(1024, 3072, seed=5)).to(gpu_device)
    x = synth.to_bf16_tensor(synth.activations(192, 3072, seed=6), gpu_device)
    b = torch.randn(1024, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16).to(gpu_device)
    for layout in (CF.W4A8_LAYOUT, CF.W4A4_LAYOUT):
        cls = classes[layout]
        qdata, params = cls.quantize(w)
        wq = StandInQuantizedTensor(qdata, cls, params, quant_ops.LAYOUT_OPS)
        y = torch.nn.functional.linear(x, wq, b)
        want = cls.linear(x, qdata, params, b)
        torch.cuda.synchronize()
        assert y.dtype == torch.bfloat16 and torch.equal(y, want)
        # and the quantized result is the dequantized weight's product to within the activation
        # codes' error (on the CPU oracle for these inputs: 0.009 with int8 codes, 0.207 with int4)
        ref = x.float() @ cls.dequantize(qdata, params).float().T + b.float()
        assert gemm.rel_l2(ref.cpu().numpy(), y.float().cpu().numpy()) < (2e-2 if layout == CF.W4A8_LAYOUT else 0.3)
