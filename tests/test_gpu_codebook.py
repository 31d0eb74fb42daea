"""GPU parity of the shipped asym_w4a8_int8 decode (mq_decode_w4a8_codebook) against the CPU
oracle (bit-exact int8 codes and row scales), and of w4a8_int8_linear on that layout (rel-L2 of
the bf16 output against the oracle's fp64 result < 4e-3). Each case prints its name first."""
import numpy as np
import pytest
import torch

import kitchen_amd as ck
from kitchen_amd import _lib, synth
from oracle import codebook as cbk
from oracle import gemm, linear

pytestmark = pytest.mark.gpu


def _case(n, k, gs, seed, with_codebook=True, saturate=False):
    """Random codes; s_rel in int8 units (fp8 32..120 with levels in [-1, 1], 1..15 with signed
    int4 levels), or up to 448 with saturate (then |level * s_rel| can pass 127)."""
    rng = np.random.default_rng(seed)
    qdata = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    lo, hi = (0x60, 0x70) if with_codebook else (0x38, 0x58)
    if saturate:
        lo, hi = 0x20, 0x7F                                                 # finite positive fp8
    s_rel = rng.integers(lo, hi, (n, k // gs), dtype=np.uint8)
    s_ch = rng.uniform(0.001, 0.05, n).astype(np.float32)
    cb = np.sort(rng.uniform(-1, 1, 16)).astype(np.float32) if with_codebook else None
    return qdata, s_rel, s_ch, cb


def _dev(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t.view(dtype) if dtype is not None else t


@pytest.mark.parametrize("gs", [4, 8, 16, 32, 64])
@pytest.mark.parametrize("with_codebook", [True, False])
@pytest.mark.parametrize("saturate", [False, True])
def test_decode_bitexact(gpu_device, gs, with_codebook, saturate):
    n, k = 96, 3072
    print(f"[codebook] decode N={n} K={k} gs={gs} codebook={with_codebook} saturate={saturate}", flush=True)
    qdata, s_rel, s_ch, cb = _case(n, k, gs, seed=gs + with_codebook, saturate=saturate)
    qdata[5] = 0                                                       # all-zero row (with levels[0] = 0)
    if cb is not None:
        cb[0] = 0.0
        cb[1] = 0.5                                                    # ties: 0.5 * odd s_rel
    s_rel[7, :] = 0x7F                                                 # fp8 NaN scales -> zero codes
    q8, rs = ck.decode_w4a8_codebook_weight(_dev(qdata, gpu_device, torch.int8),
                                            _dev(s_rel, gpu_device).view(torch.float8_e4m3fn),
                                            _dev(s_ch, gpu_device), None if cb is None else _dev(cb, gpu_device), gs)
    torch.cuda.synchronize()
    q0, r0 = cbk.decode_w4a8_codebook(qdata, s_rel, s_ch, cb, gs)
    assert np.array_equal(q8.cpu().numpy(), q0)
    assert np.array_equal(rs.cpu().numpy().view(np.uint32), r0.view(np.uint32))


def test_decode_large_shape(gpu_device):
    n, k = 12288, 3072
    print(f"[codebook] decode N={n} K={k}", flush=True)
    qdata, s_rel, s_ch, cb = _case(n, k, 16, seed=7)
    q8, rs = ck.decode_w4a8_codebook_weight(_dev(qdata, gpu_device), _dev(s_rel, gpu_device), _dev(s_ch, gpu_device),
                                            _dev(cb, gpu_device), 16)
    torch.cuda.synchronize()
    rows = np.r_[0:128, n - 128:n]
    q0, r0 = cbk.decode_w4a8_codebook(qdata[rows], s_rel[rows], s_ch[rows], cb, 16)
    assert np.array_equal(q8.cpu().numpy()[rows], q0) and np.array_equal(rs.cpu().numpy()[rows], r0)
    assert np.array_equal(rs.cpu().numpy().view(np.uint32), s_ch.view(np.uint32))   # s_channel unchanged


@pytest.mark.parametrize("m,n,k", [(512, 3072, 3072), (4096, 1024, 3072)])
def test_w4a8_int8_linear_shipped_layout(gpu_device, m, n, k):
    print(f"[codebook] w4a8_int8_linear shipped layout M={m} N={n} K={k}", flush=True)
    qdata, s_rel, s_ch, cb = _case(n, k, 16, seed=m + n)
    xb = synth.activations(m, k, seed=3)
    rng = np.random.default_rng(4)
    bias = synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(rng.standard_normal(n).astype(np.float32) * 0.1))
    x = synth.to_bf16_tensor(xb, gpu_device)
    y = ck.w4a8_int8_linear(x, _dev(qdata, gpu_device, torch.int8), _dev(s_rel, gpu_device), _dev(s_ch, gpu_device),
                            codebook=_dev(cb, gpu_device), correction=None, bias=torch.from_numpy(bias).to(gpu_device),
                            group_size=16, convrot_groupsize=256, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    rows = np.r_[0:128, m - 128:m] if m > 256 else np.arange(m)
    q0, r0 = cbk.decode_w4a8_codebook(qdata, s_rel, s_ch, cb, 16)
    ref = linear.w8a8_linear(synth.bf16_bits_to_f32(xb[rows]), q0, r0, bias, 256)
    err = gemm.rel_l2(ref.y, y.float().cpu().numpy()[rows])
    print(f"[codebook] rel L2 {err:.2e}", flush=True)
    assert err < 4e-3
    # and against the weight the tensors describe (rotated x times level * s_rel * s_channel)
    from oracle.hadamard import fwht_pinned
    w = cbk.dequant_rotated(qdata, s_rel, s_ch, cb, 16)
    xr = fwht_pinned(synth.bf16_bits_to_f32(xb[rows]), 256).astype(np.float64)
    assert gemm.rel_l2(xr @ w.T + bias[None, :], y.float().cpu().numpy()[rows]) < 2e-2


def test_shipped_layout_errors(gpu_device):
    print("[codebook] argument errors", flush=True)
    qdata, s_rel, s_ch, cb = _case(8, 256, 16, seed=1)
    x = torch.zeros(4, 256, dtype=torch.bfloat16, device=gpu_device)
    with pytest.raises(NotImplementedError):
        ck.w4a8_int8_linear(x, _dev(qdata, gpu_device), _dev(s_rel, gpu_device), _dev(s_ch, gpu_device),
                            _dev(cb, gpu_device), correction=_dev(s_rel, gpu_device), group_size=16)
    with pytest.raises(ValueError):
        ck.w4a8_int8_linear(x, _dev(qdata, gpu_device), _dev(s_rel, gpu_device), _dev(s_ch, gpu_device),
                            _dev(cb, gpu_device), group_size=32)
    with pytest.raises(ValueError):                        # group size 12 is refused by the C ABI
        _lib.call("mq_decode_w4a8_codebook", 0, 128, 0, 16, 0, 0, 12, 8, 192, 0, 192, 0, 0)
