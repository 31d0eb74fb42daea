"""The whole-linear entry points (mq_linear_w4_group, mq_linear_rowscale: rotate + quantize and
the GEMM in one library call, codes and scales in the caller's workspace) give the same bits as
the two separate entry points they chain, for every path the linears take: group and row scales,
int8 and int4 activations, the SwiGLU prologue, few-row, 128-tile, split-K and wide GEMMs."""
import numpy as np
import pytest
import torch

import kitchen_amd as ck
from kitchen_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu


def _x(m, k, dev, dtype, seed):
    return synth.to_bf16_tensor(synth.activations(m, k, seed=seed), dev).to(dtype)


@pytest.mark.parametrize("m", [1, 77, 256, 1000])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_w4a8_group_linear_equals_two_steps(gpu_device, m, dtype):
    k, n = 3072, 1024
    print(f"[fused] w4a8 group M={m} {dtype}", flush=True)
    qd, s16, zp = ck.quantize_w4a8_asym_weight(torch.from_numpy(synth.weight(n, k, seed=3)).to(gpu_device), 64, 256)
    x = _x(m, k, gpu_device, dtype, seed=m)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(1)).to(dtype).to(gpu_device)
    y = ck.w4a8_int8_linear(x, qd, s16, None, None, zp, bias, 64, 256, dtype)
    qa, sa = ops.rotate_quantize(x, 256, 8)
    y2 = ops.gemm_w4_group(qa, sa, qd.view(torch.uint8), s16, zp.view(torch.uint8), bias, n, out_dtype=dtype)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)


@pytest.mark.parametrize("m", [3, 256, 700])
@pytest.mark.parametrize("hb", [16, 64, 256])
def test_w4a4_group_linear_swiglu_equals_two_steps(gpu_device, m, hb):
    k, n = 2048, 768
    print(f"[fused] w4a4 group swiglu M={m} H{hb}", flush=True)
    qw, s16 = ck.quantize_w4a4_group_weight(torch.from_numpy(synth.weight(n, k, seed=4)).to(gpu_device), 64, hb)
    rng = np.random.default_rng(m)
    h = torch.from_numpy(rng.standard_normal((m, 2 * k)).astype(np.float32) * 2).to(torch.bfloat16).to(gpu_device)
    y = ck.convrot_w4a4_linear(h, qw, s16, None, convrot_groupsize=hb, input_act="swiglu")
    # comfy-kitchen fuses (one rounding) under H256 only; H16 / H64 take its eager two roundings
    mode = _lib.SWIGLU_FUSED if hb == 256 else _lib.SWIGLU_EAGER
    qa, sa = ops.rotate_quantize(h, hb, 4, _lib.Q_X16ALT, swiglu=mode)
    y2 = ops.gemm_w4_group(qa, sa, qw, s16, None, None, n, act_mode=_lib.ACT_X16ALT)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)


@pytest.mark.parametrize("m", [2, 100, 256, 900])
def test_rowscale_linears_equal_two_steps(gpu_device, m):
    k, n = 3072, 640
    print(f"[fused] rowscale M={m}", flush=True)
    x = _x(m, k, gpu_device, torch.bfloat16, seed=m + 5)
    # shipped ConvRot W4A4: int4 activations, per-row F32 weight scale
    qw4, ws4 = ck.quantize_convrot_w4a4_weight(torch.from_numpy(synth.weight(n, k, seed=6)).to(gpu_device), 256)
    y = ck.convrot_w4a4_linear(x, qw4, ws4, None, convrot_groupsize=256)
    qa, sa = ops.rotate_quantize(x, 256, 4)
    y2 = ops.gemm_rowscale(qa, sa, qw4, ws4.reshape(-1).float(), None, n, 4)
    # int8_tensorwise with the SwiGLU prologue
    qw8, ws8 = ck.quantize_int8_convrot_weight(torch.from_numpy(synth.weight(n, k, seed=7)).to(gpu_device), 256)
    h = torch.cat([x, x.flip(1)], dim=1)
    y3 = ck.int8_linear(h, qw8, ws8, None, torch.float16, True, 256, input_act="swiglu")
    qa8, sa8 = ops.rotate_quantize(h, 256, 8, swiglu=True)
    y4 = ops.gemm_rowscale(qa8, sa8, qw8, ws8.reshape(-1).float(), None, n, 8, out_dtype=torch.float16)
    torch.cuda.synchronize()
    assert torch.equal(y, y2) and torch.equal(y3, y4)
