"""The few-row path (M <= 4: the adaLN modulation linear and single-token calls) against the
oracle, for every weight kind, epilogue and activation layout it serves."""
import numpy as np
import pytest
import torch

from kitchen_amd import _lib, ops
from oracle import gemm, quant

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("n,k", [(18432, 3072), (1000, 640), (3072, 12288)])
def test_u4_asym_group(gpu_device, m, n, k):
    print(f"[gemv] u4 group M={m} N={n} K={k}", flush=True)
    rng = np.random.default_rng(m * n + k)
    qa = rng.integers(-127, 128, (m, k)).astype(np.int8)
    q = rng.integers(0, 16, (n, k)).astype(np.uint8)
    z = rng.integers(0, 16, (n, k // 64)).astype(np.uint8)
    s16 = rng.uniform(1e-3, 4e-3, (n, k // 64)).astype(np.float16)
    sa = rng.uniform(0.001, 0.01, m).astype(np.float32)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16)
    y = ops.gemm_w4_group(_t(qa, gpu_device), _t(sa, gpu_device), _t(quant.pack_u4(q), gpu_device),
                          _t(s16, gpu_device), _t(quant.pack_u4(z), gpu_device), bias.to(gpu_device), n)
    torch.cuda.synchronize()
    p = gemm.partials(qa, gemm.zero_adjusted(q, z, 64), 64)
    ref = gemm.epilogue_group(p, sa, s16.astype(np.float64), bias.float().numpy())
    assert gemm.rel_l2(ref, y.float().cpu().numpy()) < 4e-3


@pytest.mark.parametrize("act_mode", [_lib.ACT_I8, _lib.ACT_I4, _lib.ACT_X16ALT])
def test_i4_sym_group_activation_layouts(gpu_device, act_mode):
    m, n, k = 2, 3072, 3072
    print(f"[gemv] i4 group act_mode={act_mode}", flush=True)
    rng = np.random.default_rng(act_mode)
    codes = rng.integers(-7, 8, (m, k)).astype(np.int8) if act_mode else rng.integers(-127, 128, (m, k)).astype(np.int8)
    stored = codes
    if act_mode == _lib.ACT_X16ALT:
        sign = np.where((np.arange(k) // 64) % 2 == 1, -1, 1)
        stored = (16 * codes.astype(np.int16) * sign[None, :]).astype(np.int8)
    qw = rng.integers(-8, 8, (n, k)).astype(np.int8)
    s16 = rng.uniform(1e-3, 4e-3, (n, k // 64)).astype(np.float16)
    sa = rng.uniform(0.01, 0.1, m).astype(np.float32)
    y = ops.gemm_w4_group(_t(stored, gpu_device), _t(sa, gpu_device), _t(quant.pack_i4(qw), gpu_device),
                          _t(s16, gpu_device), None, None, n, act_mode=act_mode)
    torch.cuda.synchronize()
    ref = gemm.epilogue_group(gemm.partials(codes, qw, 64), sa, s16.astype(np.float64))
    assert gemm.rel_l2(ref, y.float().cpu().numpy()) < 4e-3


@pytest.mark.parametrize("wbits", [4, 8])
@pytest.mark.parametrize("m", [1, 4])
def test_rowscale_exact_sums(gpu_device, wbits, m):
    n, k = 3072, 3072
    print(f"[gemv] rowscale wbits={wbits} M={m}", flush=True)
    rng = np.random.default_rng(wbits * 10 + m)
    qa = rng.integers(-127, 128, (m, k)).astype(np.int8)
    lo, hi = (-8, 8) if wbits == 4 else (-127, 128)
    qw = rng.integers(lo, hi, (n, k)).astype(np.int8)
    sa = rng.uniform(0.001, 0.01, m).astype(np.float32)
    ws = rng.uniform(0.001, 0.01, n).astype(np.float32)
    packed = quant.pack_i4(qw) if wbits == 4 else qw
    y = ops.gemm_rowscale(_t(qa, gpu_device), _t(sa, gpu_device), _t(packed, gpu_device), _t(ws, gpu_device), None,
                          n, wbits)
    torch.cuda.synchronize()
    acc = gemm.partials(qa, qw, k)[0]
    # the exact int32 sum through the same fp32 expression: bit-exact bf16
    want = (acc.astype(np.float32) * sa[:, None] * ws[None, :]).astype(np.float32)
    assert np.array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16), quant.f32_to_bf16_bits(want))
