"""End-to-end GPU parity of the drop-in linears (rotate + quantize + GEMM + epilogue) at the
benchmark configurations, through the comfy-kitchen call surface."""
import numpy as np
import pytest
import torch

import kitchen_amd as ck
from kitchen_amd import synth, weights
from oracle import gemm, linear, quant

pytestmark = pytest.mark.gpu


def _setup(m, n, k, seed, spikes=0.0):
    xb = synth.activations(m, k, seed=seed, spike_frac=spikes)
    w = synth.weight(n, k, seed=seed + 1)
    rng = np.random.default_rng(seed + 2)
    bias = synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(rng.standard_normal(n).astype(np.float32) * 0.1))
    return xb, w, bias


def _rows(m):
    return np.r_[0:min(m, 256), max(0, m - 256):m] if m > 512 else np.arange(m)


@pytest.mark.parametrize("m,n,k", [(1024, 3072, 3072), (4352, 3072, 3072), (4096, 12288, 3072)])
def test_w4a8_linear_configs(gpu_device, m, n, k):
    """C0 (1024x3072x3072), C1 attn-out at M=4352, and the north-star shape (rows checked:
    first and last 256, as g64_bench6.py:71-79)."""
    print(f"[linear] w4a8 M={m} N={n} K={k}", flush=True)
    xb, w, bias = _setup(m, n, k, seed=0)
    qd, s16, zp = ck.quantize_w4a8_asym_weight(torch.from_numpy(w).to(gpu_device), 64, 256)
    x = synth.to_bf16_tensor(xb, gpu_device)
    y = ck.w4a8_int8_linear(x, qd, s16, None, None, zp, torch.from_numpy(bias).to(gpu_device), 64, 256,
                            torch.bfloat16)
    torch.cuda.synchronize()
    assert y.shape == (m, n) and y.dtype == torch.bfloat16
    # oracle on the same inputs; weights through the oracle quantizer must equal the device's
    q0, s0, z0 = quant.quant_weight_u4_asym(linear.rotate_weight(w, 256), 64)
    assert np.array_equal(qd.cpu().numpy(), quant.pack_u4(q0)), "weight codes differ"
    assert np.array_equal(zp.cpu().numpy(), quant.pack_u4(z0)), "zero-points differ"
    rows = _rows(m)
    ref = linear.w4a8_asym_linear(synth.bf16_bits_to_f32(xb[rows]), q0, s0, z0, bias, 256, 64)
    err = gemm.rel_l2(ref.y, y.float().cpu().numpy()[rows])
    print(f"[linear] rel L2 {err:.2e}", flush=True)
    assert err < 1e-2
    # the activation codes the linear fed its GEMM are the oracle's, bit for bit
    qa, sa = ck.quantize_int8_rowwise_convrot(x, 256)
    assert np.array_equal(qa.cpu().numpy()[rows], ref.qa) and np.array_equal(sa.cpu().numpy()[rows], ref.sa)


@pytest.mark.parametrize("hblock", [16, 64, 256])
def test_w4a4_group_linear_c2(gpu_device, hblock):
    m, n, k = 1024, 3072, 3072
    print(f"[linear] w4a4 group hblock={hblock}", flush=True)
    xb, w, bias = _setup(m, n, k, seed=2, spikes=0.001)
    qw, s16 = ck.quantize_w4a4_group_weight(torch.from_numpy(w).to(gpu_device), 64, hblock)
    x = synth.to_bf16_tensor(xb, gpu_device)
    y = ck.convrot_w4a4_linear(x, qw, s16, torch.from_numpy(bias).to(gpu_device), convrot_groupsize=hblock)
    torch.cuda.synchronize()
    q0, s0 = quant.quant_weight_i4_sym_group(linear.rotate_weight(w, hblock), 64)
    rows = _rows(m)
    ref = linear.w4a4_group_linear(synth.bf16_bits_to_f32(xb[rows]), q0, s0, bias, hblock, 64)
    assert gemm.rel_l2(ref.y, y.float().cpu().numpy()[rows]) < 1e-2


@pytest.mark.parametrize("linear_dtype", ["int4", "int8"])
def test_convrot_w4a4_shipped_rowscale(gpu_device, linear_dtype):
    m, n, k = 512, 3072, 3072
    print(f"[linear] convrot shipped {linear_dtype}", flush=True)
    xb, w, bias = _setup(m, n, k, seed=4)
    qw, ws = ck.quantize_convrot_w4a4_weight(torch.from_numpy(w).to(gpu_device), 256, 64)
    x = synth.to_bf16_tensor(xb, gpu_device)
    y = ck.convrot_w4a4_linear(x, qw, ws, torch.from_numpy(bias).to(gpu_device), 256, 64, linear_dtype)
    torch.cuda.synchronize()
    q0, s0 = quant.quant_weight_i4_rowwise(linear.rotate_weight(w, 256))
    ref = linear.w4a4_row_linear(synth.bf16_bits_to_f32(xb), q0, s0, bias, 256, 4 if linear_dtype == "int4" else 8)
    assert gemm.rel_l2(ref.y, y.float().cpu().numpy()) < 1e-2


@pytest.mark.parametrize("convrot", [True, False])
def test_int8_linear(gpu_device, convrot):
    m, n, k = 256, 12288, 3072
    print(f"[linear] int8 convrot={convrot}", flush=True)
    xb, w, bias = _setup(m, n, k, seed=6)
    q8, s8 = ck.quantize_int8_convrot_weight(torch.from_numpy(w).to(gpu_device), 256 if convrot else None)
    x = synth.to_bf16_tensor(xb, gpu_device)
    y = ck.int8_linear(x, q8, s8, torch.from_numpy(bias).to(gpu_device), torch.bfloat16, convrot, 256)
    torch.cuda.synchronize()
    wr = linear.rotate_weight(w, 256) if convrot else w
    q0, s1 = quant.quant_weight_i8_rowwise(wr)
    ref = linear.w8a8_linear(synth.bf16_bits_to_f32(xb), q0, s1, bias, 256 if convrot else None)
    assert gemm.rel_l2(ref.y, y.float().cpu().numpy()) < 1e-2


def test_leading_dims_and_m1(gpu_device):
    print("[linear] 3-D input and M=1", flush=True)
    n, k = 18432, 3072
    xb, w, bias = _setup(2, n, k, seed=8)
    qd, s16, zp = ck.quantize_w4a8_asym_weight(torch.from_numpy(w).to(gpu_device), 64, 256)
    x = synth.to_bf16_tensor(xb, gpu_device).reshape(2, 1, k)
    y = ck.w4a8_int8_linear(x, qd, s16, None, None, zp, None, 64, 256, torch.bfloat16)
    assert y.shape == (2, 1, n)
    q0, s0, z0 = quant.quant_weight_u4_asym(linear.rotate_weight(w, 256), 64)
    ref = linear.w4a8_asym_linear(synth.bf16_bits_to_f32(xb), q0, s0, z0, None, 256, 64)
    assert gemm.rel_l2(ref.y, y.reshape(2, n).float().cpu().numpy()) < 1e-2


def test_empty_batch(gpu_device):
    # zero tokens (a leading dimension of 0) give an empty output of the right shape on every op
    print("[linear] empty batch", flush=True)
    n, k = 384, 512
    w = torch.from_numpy(synth.weight(n, k, seed=9)).to(gpu_device)
    qd, s16, zp = ck.quantize_w4a8_asym_weight(w, 64, 256)
    qw, ws = ck.quantize_convrot_w4a4_weight(w, 256, 64)
    q8, s8 = weights.quantize_int8_convrot_weight(w, 256)
    for shape in ((0, k), (2, 0, k)):
        x = torch.empty(shape, dtype=torch.bfloat16, device=gpu_device)
        out = (*shape[:-1], n)
        assert ck.w4a8_int8_linear(x, qd, s16, None, None, zp, None, 64, 256, torch.bfloat16).shape == out
        assert ck.convrot_w4a4_linear(x, qw, ws, None).shape == out
        assert ck.int8_linear(x, q8, s8, None, torch.bfloat16, True, 256).shape == out
