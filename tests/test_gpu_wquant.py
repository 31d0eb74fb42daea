"""HIP weight quantizer (mq_quantize_weight, reached through kitchen_amd.weights on a GPU weight)
against the numpy oracle: packed codes, scales and zero-points bit for bit, for every format,
Hadamard block and input dtype, with the edge cases the quantizer formulas have (zero groups and
rows, one-signed and constant groups, an odd number of groups, the K limit, strided rows, fp16
scale overflow)."""
import numpy as np
import pytest
import torch

from kitchen_amd import weights
from oracle import linear, quant

pytestmark = pytest.mark.gpu

DEV = "cuda"
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _weight(n, k, seed, dtype, edge=True):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[:, :: 97] *= 25.0                                   # outlier columns
    if edge and n >= 4 and k >= 256:
        w[0, :256] = 0.0                                  # zero Hadamard block -> zero groups
        w[1, :64] = np.abs(w[1, :64])                     # one-signed group (before rotation)
        w[2, 64:128] = 0.5                                # constant group (before rotation)
        w[3, :] = 0.0                                     # zero row
    t = torch.from_numpy(w).to(dtype)
    return t, t.to(torch.float32).numpy()                 # the exact values the kernel reads


def _rot(w32, cg):
    return linear.rotate_weight(w32, cg) if cg else w32


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("cg", [0, 16, 64, 256])
def test_u4_asym_g64_bitexact(dtype, cg):
    wt, w32 = _weight(24, 1024, 31, dtype)
    qd, s16, z = weights.quantize_w4a8_asym_weight(wt.to(DEV), 64, cg)
    q0, s0, z0 = quant.quant_weight_u4_asym(_rot(w32, cg), 64)
    assert np.array_equal(qd.cpu().numpy(), quant.pack_u4(q0))
    assert np.array_equal(s16.cpu().numpy().view(np.uint16), s0.view(np.uint16))
    assert np.array_equal(z.cpu().numpy(), quant.pack_u4(z0))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("cg", [0, 16, 64, 256])
def test_i4_sym_g64_bitexact(dtype, cg):
    wt, w32 = _weight(24, 1024, 32, dtype)
    qw, s16 = weights.quantize_w4a4_group_weight(wt.to(DEV), 64, cg)
    q0, s0 = quant.quant_weight_i4_sym_group(_rot(w32, cg), 64)
    assert np.array_equal(qw.cpu().numpy(), quant.pack_i4(q0))
    assert np.array_equal(s16.cpu().numpy().view(np.uint16), s0.view(np.uint16))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("cg", [0, 64, 256])
def test_row_formats_bitexact(dtype, cg):
    wt, w32 = _weight(24, 1024, 33, dtype)
    qw, s = weights.quantize_convrot_w4a4_weight(wt.to(DEV), cg if cg else 256, 64) if cg else (None, None)
    if cg:
        q0, s0 = quant.quant_weight_i4_rowwise(_rot(w32, cg))
        assert np.array_equal(qw.cpu().numpy(), quant.pack_i4(q0))
        assert np.array_equal(s.cpu().numpy().view(np.uint32), s0.view(np.uint32))
    q8, s8 = weights.quantize_int8_convrot_weight(wt.to(DEV), cg if cg else None)
    q1, s1 = quant.quant_weight_i8_rowwise(_rot(w32, cg))
    assert q8.shape == q1.shape and s8.shape == s1.shape
    assert np.array_equal(q8.cpu().numpy(), q1)
    assert np.array_equal(s8.cpu().numpy().view(np.uint32), s1.view(np.uint32))


def test_odd_group_count_packs_last_zero_point():
    wt, w32 = _weight(8, 192, 34, torch.float32, edge=False)     # 3 groups of 64
    qd, s16, z = weights.quantize_w4a8_asym_weight(wt.to(DEV), 64, 64)
    q0, s0, z0 = quant.quant_weight_u4_asym(_rot(w32, 64), 64)
    assert z.shape == (8, 2)
    assert np.array_equal(z.cpu().numpy(), quant.pack_u4(z0))
    assert np.array_equal(qd.cpu().numpy(), quant.pack_u4(q0))


@pytest.mark.parametrize("k", [12288, 32768])
def test_large_k(k):
    wt, w32 = _weight(3, k, 35, torch.bfloat16, edge=False)
    qd, s16, z = weights.quantize_w4a8_asym_weight(wt.to(DEV), 64, 256)
    q0, s0, z0 = quant.quant_weight_u4_asym(_rot(w32, 256), 64)
    assert np.array_equal(qd.cpu().numpy(), quant.pack_u4(q0))
    assert np.array_equal(s16.cpu().numpy().view(np.uint16), s0.view(np.uint16))
    assert np.array_equal(z.cpu().numpy(), quant.pack_u4(z0))


def test_strided_rows():
    wt, w32 = _weight(16, 1536, 36, torch.float32, edge=False)
    wide = torch.zeros((16, 2048), dtype=torch.float32)
    wide[:, 256:1792] = wt
    view = wide.to(DEV)[:, 256:1792]                              # row stride 2048
    q8, s8 = weights.quantize_int8_convrot_weight(view, 256)
    q1, s1 = quant.quant_weight_i8_rowwise(_rot(w32, 256))
    assert np.array_equal(q8.cpu().numpy(), q1)
    assert np.array_equal(s8.cpu().numpy().view(np.uint32), s1.view(np.uint32))


def test_matches_torch_cpu_quantizer():
    """The two implementations behind kitchen_amd.weights agree (GPU -> HIP, CPU -> torch)."""
    wt, _ = _weight(32, 768, 37, torch.bfloat16)
    for fn, args in ((weights.quantize_w4a8_asym_weight, (64, 256)), (weights.quantize_w4a4_group_weight, (64, 64)),
                     (weights.quantize_convrot_w4a4_weight, (256, 64)), (weights.quantize_int8_convrot_weight, (256,))):
        got = fn(wt.to(DEV), *args)
        ref = fn(wt.to(torch.float32), *args)
        for g, r in zip(got, ref):
            assert g.dtype == r.dtype and g.shape == r.shape
            assert torch.equal(g.cpu(), r), fn.__name__


def test_fp16_scale_overflow_raises():
    w = torch.full((4, 256), 4.0e6, dtype=torch.float32)
    w[:, ::2] = -4.0e6
    with pytest.raises(ValueError, match="overflows the fp16 scale"):
        weights.quantize_w4a8_asym_weight(w.to(DEV), 64, 0)
