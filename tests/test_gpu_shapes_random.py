"""Seeded random shapes against the oracle. GEMM: every entry point (the few-row kernels, the wide
kernel on 128 x 128 tiles and split-K are reached; the wide kernel's large tiles are covered by
tests/test_gpu_gemm.py and tests/test_gpu_configs.py), exact int32 partials / accumulators where the entry point exposes
them, and the bf16 outputs (with and without the split-K workspace) against a float64 product of the
same codes. Rotate + quantize, plain and with the SwiGLU prologue: codes and scales bit-exact. Sizes
are drawn so the oracle finishes in seconds."""
import numpy as np
import pytest
import torch

from kitchen_amd import _lib, ops, synth
from oracle import gemm, quant, swiglu

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(2027)
CASES = []
for i in range(12):
    m = int(RNG.choice([1, 2, 3, 4, 5, 37, 128, 129, 200, 256, 300, 513]))
    n = int(RNG.integers(1, 9)) * int(RNG.choice([16, 48, 100, 128]))
    k = 64 * int(RNG.integers(1, 33))
    CASES.append((i, m, n, k))


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _plain_group(qa_d, sa_d, qw_d, s_d, z_d, bias, n, m, k, act_mode=0):
    y = torch.empty((m, n), dtype=torch.bfloat16, device=qa_d.device)
    _lib.call("mq_gemm_w4_group", qa_d.data_ptr(), qa_d.stride(0), sa_d.data_ptr(), qw_d.data_ptr(), qw_d.stride(0),
              s_d.data_ptr(), s_d.stride(0), _lib.ptr(z_d), z_d.stride(0) if z_d is not None else 0, 64, act_mode,
              _lib.ptr(bias), _lib.DT_BF16, y.data_ptr(), _lib.DT_BF16, n, m, n, k, _lib.stream_of(qa_d))
    return y


@pytest.mark.parametrize("case,m,n,k", CASES)
def test_u4_asym_group(gpu_device, case, m, n, k):
    print(f"[random] u4 group case {case} M={m} N={n} K={k}", flush=True)
    rng = np.random.default_rng(100 + case)
    qa = rng.integers(-127, 128, (m, k)).astype(np.int8)
    q = rng.integers(0, 16, (n, k)).astype(np.uint8)
    z = rng.integers(0, 16, (n, k // 64)).astype(np.uint8)
    s16 = rng.uniform(1e-3, 4e-3, (n, k // 64)).astype(np.float16)
    sa = rng.uniform(0.001, 0.01, m).astype(np.float32)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(case)).to(torch.bfloat16)
    qa_d, sa_d = _t(qa, gpu_device), _t(sa, gpu_device)
    qw_d, z_d, s_d = _t(quant.pack_u4(q), gpu_device), _t(quant.pack_u4(z), gpu_device), _t(s16, gpu_device)
    b_d = bias.to(gpu_device)
    p = gemm.partials(qa, gemm.zero_adjusted(q, z, 64), 64)
    part = ops.gemm_w4_group_partials(qa_d, qw_d, z_d, n)
    y_ws = ops.gemm_w4_group(qa_d, sa_d, qw_d, s_d, z_d, b_d, n)
    y_plain = _plain_group(qa_d, sa_d, qw_d, s_d, z_d, b_d, n, m, k)
    torch.cuda.synchronize()
    assert np.array_equal(part.cpu().numpy().astype(np.int64), p)
    ref = gemm.epilogue_group(p, sa, s16.astype(np.float64), bias.float().numpy())
    for y in (y_ws, y_plain):
        assert torch.isfinite(y).all()
        assert gemm.rel_l2(ref, y.float().cpu().numpy()) < 4e-3


@pytest.mark.parametrize("case,m,n,k", CASES)
def test_i4_sym_group_x16alt(gpu_device, case, m, n, k):
    print(f"[random] i4 group x16alt case {case} M={m} N={n} K={k}", flush=True)
    rng = np.random.default_rng(200 + case)
    codes = rng.integers(-7, 8, (m, k)).astype(np.int8)
    sign = np.where((np.arange(k) // 64) % 2 == 1, -1, 1)
    stored = (16 * codes.astype(np.int16) * sign[None, :]).astype(np.int8)
    qw = rng.integers(-8, 8, (n, k)).astype(np.int8)
    s16 = rng.uniform(1e-3, 4e-3, (n, k // 64)).astype(np.float16)
    sa = rng.uniform(0.01, 0.1, m).astype(np.float32)
    qa_d, sa_d, qw_d, s_d = _t(stored, gpu_device), _t(sa, gpu_device), _t(quant.pack_i4(qw), gpu_device), \
        _t(s16, gpu_device)
    y = ops.gemm_w4_group(qa_d, sa_d, qw_d, s_d, None, None, n, act_mode=_lib.ACT_X16ALT)
    torch.cuda.synchronize()
    p = gemm.partials(codes, qw, 64)
    ref = gemm.epilogue_group(p, sa, s16.astype(np.float64))
    assert gemm.rel_l2(ref, y.float().cpu().numpy()) < 4e-3


@pytest.mark.parametrize("wbits", [4, 8])
@pytest.mark.parametrize("case,m,n,k", CASES[:8])
def test_rowscale(gpu_device, wbits, case, m, n, k):
    print(f"[random] rowscale w{wbits} case {case} M={m} N={n} K={k}", flush=True)
    rng = np.random.default_rng(300 + case + wbits)
    lim = 7 if wbits == 4 else 127
    qa = rng.integers(-lim, lim + 1, (m, k)).astype(np.int8)
    qw = rng.integers(-lim, lim + 1, (n, k)).astype(np.int8)
    sa = rng.uniform(0.001, 0.01, m).astype(np.float32)
    ws = rng.uniform(0.001, 0.01, n).astype(np.float32)
    qa_d, sa_d, ws_d = _t(qa, gpu_device), _t(sa, gpu_device), _t(ws, gpu_device)
    qw_d = _t(quant.pack_i4(qw) if wbits == 4 else qw, gpu_device)
    acc = ops.gemm_rowscale_acc(qa_d, qw_d, n, wbits)
    y = ops.gemm_rowscale(qa_d, sa_d, qw_d, ws_d, None, n, wbits)
    torch.cuda.synchronize()
    p = gemm.partials(qa, qw, k)[0]
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), p)
    ref = p.astype(np.float64) * sa.astype(np.float64)[:, None] * ws.astype(np.float64)[None, :]
    assert gemm.rel_l2(ref, y.float().cpu().numpy()) < 4e-3


# Rotate + quantize (plain and SwiGLU prologue): seeded random M (both sides of the 512-row switch
# between four waves per row and one), K, Hadamard block and code layout; codes and scales bit-exact.
RQ_MODES = [(8, _lib.Q_BYTES), (4, _lib.Q_BYTES), (4, _lib.Q_PACKED), (4, _lib.Q_X16ALT)]
RQ_CASES = []
for i in range(12):
    hb = int(RNG.choice([0, 16, 64, 256]))
    bits, layout = RQ_MODES[int(RNG.integers(0, 4))]
    unit = max(hb, 64)                                   # K: whole Hadamard blocks and 64-column groups
    k = unit * int(RNG.choice([1, 3, 5, 12, 47, 48, 129, 256])) % 16384 or 16384
    m = int(RNG.choice([1, 7, 64, 300, 512, 513, 1100]))
    RQ_CASES.append((i, m, k, hb, bits, layout))


def _check_codes(q, s, q0, s0, layout):
    assert np.array_equal(s.view(np.uint32), s0.view(np.uint32)), "scales differ"
    if layout == _lib.Q_X16ALT:
        sign = np.where((np.arange(q0.shape[1]) // 64) % 2 == 1, -1, 1).astype(np.int16)
        assert np.array_equal(q.astype(np.int16), 16 * q0.astype(np.int16) * sign[None, :]), "x16alt codes differ"
    elif layout == _lib.Q_PACKED:
        assert np.array_equal(q, quant.pack_i4(q0)), "packed codes differ"
    else:
        assert np.array_equal(q, q0), "codes differ"


@pytest.mark.parametrize("case,m,k,hb,bits,layout", RQ_CASES)
def test_rotquant(gpu_device, case, m, k, hb, bits, layout):
    print(f"[random] rotquant case {case} M={m} K={k} hblock={hb} bits={bits} layout={layout}", flush=True)
    xb = synth.activations(m, k, seed=400 + case)
    q, s = ops.rotate_quantize(synth.to_bf16_tensor(xb, gpu_device), hb, bits, layout)
    torch.cuda.synchronize()
    xf = synth.bf16_bits_to_f32(xb)
    q0, s0 = quant.rotquant(xf, hb, bits) if hb else quant.quant_per_token(xf, 127 if bits == 8 else 7)
    _check_codes(q.cpu().numpy(), s.cpu().numpy(), q0, s0, layout)


@pytest.mark.parametrize("case,m,k,hb,bits,layout", RQ_CASES[:8])
def test_swiglu_rotquant(gpu_device, case, m, k, hb, bits, layout):
    m = min(m, 300)
    print(f"[random] swiglu rotquant case {case} M={m} K={k} hblock={hb} bits={bits} layout={layout}", flush=True)
    rng = np.random.default_rng(500 + case)
    g = rng.standard_normal((m, k)).astype(np.float32) * 3.0
    u = synth.bf16_bits_to_f32(synth.activations(m, k, seed=600 + case))
    hb_bits = synth.f32_to_bf16_bits(np.concatenate([g, u], axis=1))
    q, s = ops.rotate_quantize(synth.to_bf16_tensor(hb_bits, gpu_device), hb, bits, layout, swiglu=True)
    torch.cuda.synchronize()
    hf = synth.bf16_bits_to_f32(hb_bits)
    if hb:
        q0, s0 = swiglu.swiglu_rotquant(hf, hb, bits)
    else:
        q0, s0 = quant.quant_per_token(swiglu.swiglu_bf16(*np.split(hf, 2, axis=1)), 127 if bits == 8 else 7)
    _check_codes(q.cpu().numpy(), s.cpu().numpy(), q0, s0, layout)
