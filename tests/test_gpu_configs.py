"""The BASELINE configurations' shapes end to end (rotate + quantize + GEMM + epilogue) against a
float64 reference built from the oracle's activation codes and the dequantized packed weights:
config 1 (W4A8 MMDiT shapes at M = 4352 and 8192, adaLN at M = 1), config 2 (W4A4 with Hadamard
16 / 64 / 256, token spikes) and config 3 (video tokens, M = 32760). Rows checked: the first and
last 64 of each output; every output is also checked finite. Bar: rel-L2 < 4e-3 (north star 1e-2)."""
import numpy as np
import pytest
import torch

import kitchen_amd as ck
from kitchen_amd import synth
from oracle import gemm, quant

pytestmark = pytest.mark.gpu

C1_KN = [(3072, 3072), (3072, 9216), (3072, 12288), (12288, 3072)]


def _rows(m):
    return np.r_[0:64, m - 64:m] if m > 128 else np.arange(m)


def _ref_w4a8(x_rows, qd, s16, zp, bias, hb):
    qa, sa = quant.rotquant(x_rows, hb, 8)
    q = quant.unpack_u4(qd.cpu().numpy()).astype(np.float64)
    z = quant.unpack_u4(zp.cpu().numpy())[:, : s16.shape[1]].astype(np.float64)
    wdq = (q.reshape(q.shape[0], -1, 64) - z[..., None]) * s16.cpu().numpy().astype(np.float64)[..., None]
    return (qa.astype(np.float64) * sa.astype(np.float64)[:, None]) @ wdq.reshape(q.shape[0], -1).T + bias


def _ref_w4a4(x_rows, qw, s16, bias, hb):
    qa, sa = quant.rotquant(x_rows, hb, 4)
    q = quant.unpack_i4(qw.cpu().numpy()).astype(np.float64)
    wdq = q.reshape(q.shape[0], -1, 64) * s16.cpu().numpy().astype(np.float64)[..., None]
    return (qa.astype(np.float64) * sa.astype(np.float64)[:, None]) @ wdq.reshape(q.shape[0], -1).T + bias


def _bias(n, seed):
    rng = np.random.default_rng(seed)
    return synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(rng.standard_normal(n).astype(np.float32) * 0.1))


@pytest.mark.parametrize("k,n", C1_KN)
def test_config1_w4a8_shapes(gpu_device, k, n):
    w = torch.from_numpy(synth.weight(n, k, seed=k + n)).to(gpu_device)
    qd, s16, zp = ck.quantize_w4a8_asym_weight(w, 64, 256)
    del w
    bias = _bias(n, k)
    for m in (4352, 8192):
        print(f"[config1] w4a8 M={m} K={k} N={n}", flush=True)
        xb = synth.activations(m, k, seed=m + k)
        y = ck.w4a8_int8_linear(synth.to_bf16_tensor(xb, gpu_device), qd, s16, None, None, zp,
                                torch.from_numpy(bias).to(gpu_device), 64, 256, torch.bfloat16)
        torch.cuda.synchronize()
        assert torch.isfinite(y).all()
        rows = _rows(m)
        ref = _ref_w4a8(synth.bf16_bits_to_f32(xb[rows]), qd, s16, zp, bias, 256)
        err = gemm.rel_l2(ref, y.float().cpu().numpy()[rows])
        print(f"[config1] rel L2 {err:.2e}", flush=True)
        assert err < 4e-3


def test_config1_adaln_m1(gpu_device):
    k, n = 3072, 18432
    print(f"[config1] adaLN M=1 K={k} N={n}", flush=True)
    qd, s16, zp = ck.quantize_w4a8_asym_weight(torch.from_numpy(synth.weight(n, k, seed=9)).to(gpu_device), 64, 256)
    xb = synth.activations(1, k, seed=10)
    bias = _bias(n, 11)
    y = ck.w4a8_int8_linear(synth.to_bf16_tensor(xb, gpu_device), qd, s16, None, None, zp,
                            torch.from_numpy(bias).to(gpu_device), 64, 256, torch.bfloat16)
    ref = _ref_w4a8(synth.bf16_bits_to_f32(xb), qd, s16, zp, bias, 256)
    assert gemm.rel_l2(ref, y.float().cpu().numpy()) < 4e-3


@pytest.mark.parametrize("hb", [16, 64, 256])
@pytest.mark.parametrize("k,n", C1_KN)
def test_config2_w4a4_shapes(gpu_device, k, n, hb):
    qw, s16 = ck.quantize_w4a4_group_weight(torch.from_numpy(synth.weight(n, k, seed=k + n + hb)).to(gpu_device),
                                            64, hb)
    bias = _bias(n, hb)
    for m in (4352, 8192):
        print(f"[config2] w4a4 H{hb} M={m} K={k} N={n}", flush=True)
        xb = synth.activations(m, k, seed=m + hb, spike_frac=0.001)
        y = ck.convrot_w4a4_linear(synth.to_bf16_tensor(xb, gpu_device), qw, s16,
                                   torch.from_numpy(bias).to(gpu_device), convrot_groupsize=hb)
        torch.cuda.synchronize()
        assert torch.isfinite(y).all()
        rows = _rows(m)
        ref = _ref_w4a4(synth.bf16_bits_to_f32(xb[rows]), qw, s16, bias, hb)
        err = gemm.rel_l2(ref, y.float().cpu().numpy()[rows])
        print(f"[config2] rel L2 {err:.2e}", flush=True)
        assert err < 4e-3
        del y
    torch.cuda.empty_cache()


@pytest.mark.parametrize("hb", [16, 64, 256])
def test_config2_adaln_m1(gpu_device, hb):
    """Config 2 on config 1's M = 1 adaLN shape (3072 -> 18432): the few-row kernel with int4
    activations in the group GEMM's x16 layout."""
    k, n = 3072, 18432
    print(f"[config2] w4a4 adaLN H{hb} M=1 K={k} N={n}", flush=True)
    qw, s16 = ck.quantize_w4a4_group_weight(torch.from_numpy(synth.weight(n, k, seed=12 + hb)).to(gpu_device), 64, hb)
    xb = synth.activations(1, k, seed=13 + hb)
    bias = _bias(n, 14 + hb)
    y = ck.convrot_w4a4_linear(synth.to_bf16_tensor(xb, gpu_device), qw, s16, torch.from_numpy(bias).to(gpu_device),
                               convrot_groupsize=hb)
    torch.cuda.synchronize()
    ref = _ref_w4a4(synth.bf16_bits_to_f32(xb), qw, s16, bias, hb)
    err = gemm.rel_l2(ref, y.float().cpu().numpy())
    print(f"[config2] rel L2 {err:.2e}", flush=True)
    assert err < 4e-3


@pytest.mark.parametrize("k,n", [(3072, 9216), (3072, 14336), (14336, 3072)])
def test_config3_video_gemms(gpu_device, k, n):
    m = 32760
    print(f"[config3] w4a8 M={m} K={k} N={n}", flush=True)
    qd, s16, zp = ck.quantize_w4a8_asym_weight(torch.from_numpy(synth.weight(n, k, seed=n)).to(gpu_device), 64, 256)
    xb = synth.activations(m, k, seed=3)
    y = ck.w4a8_int8_linear(synth.to_bf16_tensor(xb, gpu_device), qd, s16, None, None, zp, None, 64, 256,
                            torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    rows = _rows(m)
    ref = _ref_w4a8(synth.bf16_bits_to_f32(xb[rows]), qd, s16, zp, 0.0, 256)
    err = gemm.rel_l2(ref, y.float().cpu().numpy()[rows])
    print(f"[config3] rel L2 {err:.2e}", flush=True)
    assert err < 4e-3
    del y
    torch.cuda.empty_cache()
