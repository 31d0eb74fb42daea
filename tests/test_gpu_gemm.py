"""GPU parity of the quantized GEMMs against the oracle.

Bars: per-group int32 partials and full-K int32 accumulators bit-exact; bf16 outputs within
relative L2 1e-2 of the oracle's fp64 epilogue (the kernels land near the bf16 rounding floor,
so the tests also require < 4e-3)."""
import numpy as np
import pytest
import torch

from kitchen_amd import _lib, ops
from oracle import gemm, quant

pytestmark = pytest.mark.gpu
TOL = 1e-2
TIGHT = 4e-3


def _bf16_round(x):
    from kitchen_amd import synth

    return synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(np.asarray(x, np.float32)))


def _t(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.view(dtype)


def _case_u4(m, n, k, seed, dev):
    rng = np.random.default_rng(seed)
    qa = rng.integers(-127, 128, (m, k)).astype(np.int8)
    sa = rng.uniform(0.005, 0.015, m).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    q, s16, z = quant.quant_weight_u4_asym(w, 64)
    bias = _bf16_round(rng.standard_normal(n) * 0.5)
    return qa, sa, q, s16, z, bias


@pytest.mark.parametrize("m,n,k", [(128, 128, 64), (130, 200, 192), (1, 128, 3072), (257, 384, 1024),
                                   (64, 1000, 640)])
def test_u4_asym_partials_bitexact(gpu_device, m, n, k):
    print(f"[gemm] u4 partials M={m} N={n} K={k}", flush=True)
    qa, sa, q, s16, z, bias = _case_u4(m, n, k, m + n + k, gpu_device)
    part = ops.gemm_w4_group_partials(_t(qa, gpu_device), _t(quant.pack_u4(q), gpu_device),
                                      _t(quant.pack_u4(z), gpu_device), n)
    torch.cuda.synchronize()
    p0 = gemm.partials(qa, gemm.zero_adjusted(q, z, 64), 64)
    assert np.array_equal(part.cpu().numpy().astype(np.int64), p0)


@pytest.mark.parametrize("m,n,k", [(128, 128, 128), (77, 256, 3072)])
def test_i4_sym_partials_bitexact(gpu_device, m, n, k):
    print(f"[gemm] i4 partials M={m} N={n} K={k}", flush=True)
    rng = np.random.default_rng(m * n)
    qa = rng.integers(-7, 8, (m, k)).astype(np.int8)
    qw = rng.integers(-8, 8, (n, k)).astype(np.int8)           # full signed nibble range incl. -8
    part = ops.gemm_w4_group_partials(_t(qa, gpu_device), _t(quant.pack_i4(qw), gpu_device), None, n)
    torch.cuda.synchronize()
    assert np.array_equal(part.cpu().numpy().astype(np.int64), gemm.partials(qa, qw, 64))


def test_extreme_partials(gpu_device):
    print("[gemm] extreme partials", flush=True)
    m, n, k = 128, 128, 128
    qa = np.full((m, k), 127, np.int8)
    qa[1::2] = -127
    q = np.full((n, k), 15, np.uint8)
    z = np.zeros((n, 2), np.uint8)
    q[1::2] = 0
    z[1::2] = 15
    part = ops.gemm_w4_group_partials(_t(qa, gpu_device), _t(quant.pack_u4(q), gpu_device),
                                      _t(quant.pack_u4(z), gpu_device), n).cpu().numpy()
    p0 = gemm.partials(qa, gemm.zero_adjusted(q, z, 64), 64)
    assert np.abs(p0).max() == 64 * 127 * 15
    assert np.array_equal(part.astype(np.int64), p0)


@pytest.mark.parametrize("m,n,k", [(256, 256, 3072), (130, 384, 1024), (1, 3072, 3072), (300, 1000, 12288)])
def test_u4_asym_group_scale_output(gpu_device, m, n, k):
    print(f"[gemm] u4 y M={m} N={n} K={k}", flush=True)
    qa, sa, q, s16, z, bias = _case_u4(m, n, k, 7 * m + n, gpu_device)
    y = ops.gemm_w4_group(_t(qa, gpu_device), _t(sa, gpu_device), _t(quant.pack_u4(q), gpu_device),
                          _t(s16, gpu_device), _t(quant.pack_u4(z), gpu_device),
                          torch.from_numpy(bias).to(gpu_device, torch.bfloat16), n)
    torch.cuda.synchronize()
    y0 = gemm.epilogue_group(gemm.partials(qa, gemm.zero_adjusted(q, z, 64), 64), sa, s16, bias)
    err = gemm.rel_l2(y0, y.float().cpu().numpy())
    assert err < TOL and err < TIGHT, err
    y2 = ops.gemm_w4_group(_t(qa, gpu_device), _t(sa, gpu_device), _t(quant.pack_u4(q), gpu_device),
                           _t(s16, gpu_device), _t(quant.pack_u4(z), gpu_device),
                           torch.from_numpy(bias).to(gpu_device, torch.bfloat16), n)
    assert torch.equal(y, y2), "not deterministic"


@pytest.mark.parametrize("wbits", [4, 8])
@pytest.mark.parametrize("m,n,k", [(128, 128, 64), (200, 300, 3072), (1, 256, 12288)])
def test_rowscale_acc_and_output(gpu_device, wbits, m, n, k):
    print(f"[gemm] rowscale w{wbits} M={m} N={n} K={k}", flush=True)
    rng = np.random.default_rng(wbits * 1000 + m)
    lim = 7 if wbits == 4 else 127
    qa = rng.integers(-lim, lim + 1, (m, k)).astype(np.int8)
    qw = rng.integers(-lim, lim + 1, (n, k)).astype(np.int8)
    wpk = quant.pack_i4(qw) if wbits == 4 else qw
    acc = ops.gemm_rowscale_acc(_t(qa, gpu_device), _t(wpk, gpu_device), n, wbits)
    torch.cuda.synchronize()
    p0 = gemm.partials(qa, qw, k)[0]
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), p0)
    sa = rng.uniform(0.01, 0.02, m).astype(np.float32)
    sw = rng.uniform(0.001, 0.002, n).astype(np.float32)
    bias = _bf16_round(rng.standard_normal(n))
    y = ops.gemm_rowscale(_t(qa, gpu_device), _t(sa, gpu_device), _t(wpk, gpu_device), _t(sw, gpu_device),
                          torch.from_numpy(bias).to(gpu_device, torch.bfloat16), n, wbits)
    torch.cuda.synchronize()
    err = gemm.rel_l2(gemm.epilogue_row(p0, sa, sw, bias), y.float().cpu().numpy())
    assert err < TIGHT, err


# ---------------------------------------------------------------- activation layouts and tile paths
# M <= 128 runs the few-row 128 x 128-tile kernel; larger M the wide kernel, on 128 x 128 tiles for
# small products and 256 x 256 or 256 x 192 tiles for large ones: all are covered.

def _x16alt(qa):
    """The group GEMM's int4 operand layout (mq_rotquant MQ_Q_X16ALT): 16 * q, odd groups negated."""
    sign = np.where((np.arange(qa.shape[1]) // 64) % 2 == 1, -1, 1).astype(np.int16)
    return (16 * qa.astype(np.int16) * sign[None, :]).astype(np.int8)


@pytest.mark.parametrize("act_mode", [_lib.ACT_I4, _lib.ACT_X16ALT])
@pytest.mark.parametrize("wkind", ["u4", "i4"])
@pytest.mark.parametrize("m,n,k", [(96, 128, 256), (300, 384, 1024), (513, 256, 3072)])
def test_int4_activation_layouts_partials_bitexact(gpu_device, act_mode, wkind, m, n, k):
    print(f"[gemm] int4 act mode={act_mode} w={wkind} M={m} N={n} K={k}", flush=True)
    rng = np.random.default_rng(m + n + act_mode)
    qa = rng.integers(-7, 8, (m, k)).astype(np.int8)
    qa_dev = _x16alt(qa) if act_mode == _lib.ACT_X16ALT else qa
    if wkind == "u4":
        q = rng.integers(0, 16, (n, k)).astype(np.uint8)
        z = rng.integers(0, 16, (n, k // 64)).astype(np.uint8)
        wpk, zpk, wq = quant.pack_u4(q), quant.pack_u4(z), gemm.zero_adjusted(q, z, 64)
    else:
        wq = rng.integers(-8, 8, (n, k)).astype(np.int8)
        wpk, zpk = quant.pack_i4(wq), None
    part = ops.gemm_w4_group_partials(_t(qa_dev, gpu_device), _t(wpk, gpu_device),
                                      None if zpk is None else _t(zpk, gpu_device), n, 64, act_mode)
    torch.cuda.synchronize()
    assert np.array_equal(part.cpu().numpy().astype(np.int64), gemm.partials(qa, wq, 64))


@pytest.mark.parametrize("act_mode", [_lib.ACT_I4, _lib.ACT_X16ALT])
@pytest.mark.parametrize("m", [64, 1024])
def test_int4_activation_layouts_output(gpu_device, act_mode, m):
    """W4A4 group scheme (int4 per-token activations, int4 sym g64 fp16 weights): the fp32 group
    accumulation stays at the bf16 rounding floor with int4-sized partials."""
    n, k = 768, 3072
    print(f"[gemm] int4 act output mode={act_mode} M={m}", flush=True)
    rng = np.random.default_rng(11 * m + act_mode)
    qa = rng.integers(-7, 8, (m, k)).astype(np.int8)
    sa = rng.uniform(0.05, 0.2, m).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    qw, s16 = quant.quant_weight_i4_sym_group(w, 64)
    bias = _bf16_round(rng.standard_normal(n) * 0.5)
    qa_dev = _x16alt(qa) if act_mode == _lib.ACT_X16ALT else qa
    y = ops.gemm_w4_group(_t(qa_dev, gpu_device), _t(sa, gpu_device), _t(quant.pack_i4(qw), gpu_device),
                          _t(s16, gpu_device), None, torch.from_numpy(bias).to(gpu_device, torch.bfloat16), n, 64,
                          act_mode)
    torch.cuda.synchronize()
    y0 = gemm.epilogue_group(gemm.partials(qa, qw, 64), sa, s16, bias)
    err = gemm.rel_l2(y0, y.float().cpu().numpy())
    assert err < TIGHT, err


@pytest.mark.parametrize("m,n,k", [(300, 1000, 640), (257, 200, 128), (1000, 520, 3072)])
def test_wide_tile_ragged_edges(gpu_device, m, n, k):
    """Ragged M and N (N % 8 != 0 takes the element-wise store path) on the wide kernel's 128 x 128
    tiles, int8 activations with full-range signed int4 weights (nibble -8 included)."""
    print(f"[gemm] ragged M={m} N={n} K={k}", flush=True)
    rng = np.random.default_rng(m * 7 + n)
    qa = rng.integers(-127, 128, (m, k)).astype(np.int8)
    qw = rng.integers(-8, 8, (n, k)).astype(np.int8)
    part = ops.gemm_w4_group_partials(_t(qa, gpu_device), _t(quant.pack_i4(qw), gpu_device), None, n)
    torch.cuda.synchronize()
    assert np.array_equal(part.cpu().numpy().astype(np.int64), gemm.partials(qa, qw, 64))
    sa = rng.uniform(0.005, 0.015, m).astype(np.float32)
    s16 = rng.uniform(0.001, 0.01, (n, k // 64)).astype(np.float16)
    y = ops.gemm_w4_group(_t(qa, gpu_device), _t(sa, gpu_device), _t(quant.pack_i4(qw), gpu_device),
                          _t(s16, gpu_device), None, None, n)
    torch.cuda.synchronize()
    err = gemm.rel_l2(gemm.epilogue_group(gemm.partials(qa, qw, 64), sa, s16), y.float().cpu().numpy())
    assert err < TIGHT, err


# Products large enough for the wide kernel's large tiles on 256 compute units, with ragged M and N
# and K / 64 = 5 (a block of four groups that runs past the last): 2900 x 3000 runs 256 x 192 tiles
# (one round of 192 tiles instead of 144 of 256), 4300 x 3000 256 x 256 tiles.
WIDE_RAGGED = [(2900, 3000, 320), (4300, 3000, 320)]


@pytest.mark.parametrize("m,n,k", WIDE_RAGGED)
def test_large_tiles_group_ragged(gpu_device, m, n, k):
    print(f"[gemm] large-tile group M={m} N={n} K={k}", flush=True)
    rng = np.random.default_rng(m + n + k)
    qa = rng.integers(-127, 128, (m, k)).astype(np.int8)
    q = rng.integers(0, 16, (n, k)).astype(np.uint8)
    z = rng.integers(0, 16, (n, k // 64)).astype(np.uint8)
    qa_d, qw_d, z_d = _t(qa, gpu_device), _t(quant.pack_u4(q), gpu_device), _t(quant.pack_u4(z), gpu_device)
    part = ops.gemm_w4_group_partials(qa_d, qw_d, z_d, n)
    torch.cuda.synchronize()
    part = part.cpu().numpy()
    wq = gemm.zero_adjusted(q, z, 64).astype(np.float64)
    a64 = qa.astype(np.float64)
    p = np.empty((k // 64, m, n), dtype=np.int64)
    for g in range(k // 64):   # float64 products of these integers are exact
        p[g] = (a64[:, 64 * g:64 * g + 64] @ wq[:, 64 * g:64 * g + 64].T).astype(np.int64)
        assert np.array_equal(part[g].astype(np.int64), p[g]), g
    sa = rng.uniform(0.001, 0.01, m).astype(np.float32)
    s16 = rng.uniform(1e-3, 4e-3, (n, k // 64)).astype(np.float16)
    bias = _bf16_round(rng.standard_normal(n) * 0.5)
    y = ops.gemm_w4_group(qa_d, _t(sa, gpu_device), qw_d, _t(s16, gpu_device), z_d,
                          torch.from_numpy(bias).to(gpu_device, torch.bfloat16), n)
    torch.cuda.synchronize()
    err = gemm.rel_l2(gemm.epilogue_group(p, sa, s16.astype(np.float64), bias), y.float().cpu().numpy())
    assert err < TIGHT, err


@pytest.mark.parametrize("wbits", [4, 8])
@pytest.mark.parametrize("m,n,k", WIDE_RAGGED)
def test_large_tiles_rowscale_ragged(gpu_device, wbits, m, n, k):
    print(f"[gemm] large-tile rowscale w{wbits} M={m} N={n} K={k}", flush=True)
    rng = np.random.default_rng(wbits + m + n)
    lim = 7 if wbits == 4 else 127
    qa = rng.integers(-127, 128, (m, k)).astype(np.int8)
    qw = rng.integers(-lim - (wbits == 4), lim + 1, (n, k)).astype(np.int8)   # int4 nibble -8 included
    wpk = quant.pack_i4(qw) if wbits == 4 else qw
    acc = ops.gemm_rowscale_acc(_t(qa, gpu_device), _t(wpk, gpu_device), n, wbits)
    torch.cuda.synchronize()
    p0 = (qa.astype(np.float64) @ qw.astype(np.float64).T).astype(np.int64)   # exact in float64
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), p0)
    sa = rng.uniform(0.01, 0.02, m).astype(np.float32)
    sw = rng.uniform(0.001, 0.002, n).astype(np.float32)
    bias = _bf16_round(rng.standard_normal(n))
    y = ops.gemm_rowscale(_t(qa, gpu_device), _t(sa, gpu_device), _t(wpk, gpu_device), _t(sw, gpu_device),
                          torch.from_numpy(bias).to(gpu_device, torch.bfloat16), n, wbits)
    torch.cuda.synchronize()
    err = gemm.rel_l2(gemm.epilogue_row(p0, sa, sw, bias), y.float().cpu().numpy())
    assert err < TIGHT, err
