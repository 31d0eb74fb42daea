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


def _act_codes(rng, m, k, act_mode):
    """(codes, stored): the activation codes and the bytes the kernel reads for act_mode, with
    the extreme codes planted in the first row."""
    if act_mode == _lib.ACT_I8:
        codes = rng.integers(-127, 128, (m, k)).astype(np.int8)
        codes[0, :64] = 127
        codes[0, 64:128] = -127
    else:
        codes = rng.integers(-7, 8, (m, k)).astype(np.int8)
        codes[0, :64] = 7
        codes[0, 64:128] = -7
    stored = codes
    if act_mode == _lib.ACT_X16ALT:
        sign = np.where((np.arange(k) // 64) % 2 == 1, -1, 1)
        stored = (16 * codes.astype(np.int16) * sign[None, :]).astype(np.int8)
    return codes, stored


@pytest.mark.parametrize("act_mode", [_lib.ACT_I8, _lib.ACT_I4, _lib.ACT_X16ALT])
@pytest.mark.parametrize("wkind", ["u4", "i4"])
@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_group_partials_bitexact(gpu_device, m, wkind, act_mode):
    """The few-row kernel's integer path: its exact per-group int32 sums (the parity entry runs the
    same kernel, loads and dot4 chains at M <= 4) against the int64 oracle, extreme weights and
    codes included."""
    n, k = 1000, 3072
    print(f"[gemv] partials {wkind} act_mode={act_mode} M={m}", flush=True)
    rng = np.random.default_rng(100 * m + 10 * act_mode + (wkind == "u4"))
    codes, stored = _act_codes(rng, m, k, act_mode)
    if wkind == "u4":
        q = rng.integers(0, 16, (n, k)).astype(np.uint8)
        z = rng.integers(0, 16, (n, k // 64)).astype(np.uint8)
        q[0, :128] = 15
        z[0, :2] = 0
        q[1, :128] = 0
        z[1, :2] = 15
        part = ops.gemm_w4_group_partials(_t(stored, gpu_device), _t(quant.pack_u4(q), gpu_device),
                                          _t(quant.pack_u4(z), gpu_device), n, act_mode=act_mode)
        want = gemm.partials(codes, gemm.zero_adjusted(q, z, 64), 64)
    else:
        qw = rng.integers(-8, 8, (n, k)).astype(np.int8)
        qw[0, :128] = -8
        qw[1, :128] = 7
        part = ops.gemm_w4_group_partials(_t(stored, gpu_device), _t(quant.pack_i4(qw), gpu_device), None, n,
                                          act_mode=act_mode)
        want = gemm.partials(codes, qw, 64)
    torch.cuda.synchronize()
    assert np.array_equal(part.cpu().numpy().astype(np.int64), want)


@pytest.mark.parametrize("wbits", [4, 8])
@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_rowscale_acc_bitexact(gpu_device, wbits, m):
    """The few-row kernel's full-K int32 sums (row-scale parity entry at M <= 4)."""
    n, k = 777, 4096
    print(f"[gemv] row acc wbits={wbits} M={m}", flush=True)
    rng = np.random.default_rng(wbits * 7 + m)
    qa = rng.integers(-127, 128, (m, k)).astype(np.int8)
    qa[0] = 127
    lo, hi = (-8, 8) if wbits == 4 else (-127, 128)
    qw = rng.integers(lo, hi, (n, k)).astype(np.int8)
    qw[0] = lo
    packed = quant.pack_i4(qw) if wbits == 4 else qw
    acc = ops.gemm_rowscale_acc(_t(qa, gpu_device), _t(packed, gpu_device), n, wbits)
    torch.cuda.synchronize()
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), gemm.partials(qa, qw, k)[0])
