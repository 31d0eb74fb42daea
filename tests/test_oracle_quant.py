"""Pins oracle.quant: known answers, rounding semantics, packing, statistics (CPU only)."""
import numpy as np
import pytest

from oracle import quant
from oracle.hadamard import fwht_pinned

F32 = np.float32


def test_per_token_known_answers():
    # row 0: absmax 127 -> s = 1, codes are the values rounded half-to-even
    # row 1: all zero -> s = 1e-10 (fp32), q = 0
    # row 2: absmax 254 -> s = 2; 5 / 2 = 2.5 ties to 2, 7 / 2 = 3.5 ties to 4, -3/2 -> -2
    x = np.array([[127.0, 2.5, -3.5, 0.5, 1.5, -127.0],
                  [0.0] * 6,
                  [254.0, 5.0, 7.0, -3.0, 0.0, 1.0]], dtype=F32)
    q, s = quant.quant_per_token(x, 127)
    assert s.dtype == np.float32
    assert s[0] == 1.0 and s[1] == F32(1e-10) and s[2] == 2.0
    assert q[0].tolist() == [127, 2, -4, 0, 2, -127]
    assert q[1].tolist() == [0] * 6
    assert q[2].tolist() == [127, 2, 4, -2, 0, 0]


def test_per_token_int4_saturates_only_at_limit():
    x = np.array([[7.0, -7.0, 3.5, 2.5, 0.49]], dtype=F32)
    q, s = quant.quant_per_token(x, 7)
    assert s[0] == 1.0
    assert q[0].tolist() == [7, -7, 4, 2, 0]


def test_division_not_reciprocal_product():
    # x / s and x * (1/s) differ for some fp32 pairs; the oracle must use division
    # (activation_balance.py:69-70). Find such a pair and check the oracle's code follows x / s.
    rng = np.random.default_rng(3)
    s = F32(3.0) / F32(127)
    xs = rng.uniform(-3, 3, 200000).astype(F32)
    div = np.rint(xs / s)
    mul = np.rint(xs * (F32(1) / s))
    idx = np.nonzero(div != mul)[0]
    assert idx.size > 0
    row = np.zeros((1, 8), F32)
    row[0, 0] = F32(3.0)          # absmax -> s = 3/127
    row[0, 1] = xs[idx[0]]
    q, sc = quant.quant_per_token(row, 127)
    assert sc[0] == s
    assert q[0, 1] == div[idx[0]]


def test_rotquant_is_fwht_then_quant():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 512)).astype(F32)
    q, s = quant.rotquant(x, 256, 8)
    q2, s2 = quant.quant_per_token(fwht_pinned(x, 256), 127)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


@pytest.mark.parametrize("bits,expect", [(8, 0.009), (4, 0.17)])
def test_roundtrip_error_matches_published(bits, expect):
    # README.md:448-452,466-473: int8 per-token ~0.009, int4 ~0.17 relative L2 after rotation
    rng = np.random.default_rng(5)
    x = rng.standard_normal((256, 3072)).astype(F32)
    xr = fwht_pinned(x, 256)
    q, s = quant.rotquant(x, 256, bits)
    rec = q.astype(np.float64) * s[:, None]
    err = np.linalg.norm(rec - xr) / np.linalg.norm(xr)
    assert abs(err - expect) / expect < 0.25, err


def test_pack_i4_hand_bytes_and_roundtrip():
    q = np.array([[1, 2, -1, 7, -7, 0, -8, 3]], dtype=np.int8)
    p = quant.pack_i4(q)
    # byte j = (q[2j] & 0xF) | (q[2j+1] & 0xF) << 4
    assert p.view(np.uint8).tolist() == [[0x21, 0x7F, 0x09, 0x38]]
    assert np.array_equal(quant.unpack_i4(p), q)
    rng = np.random.default_rng(6)
    r = rng.integers(-8, 8, (5, 64)).astype(np.int8)
    assert np.array_equal(quant.unpack_i4(quant.pack_i4(r)), r)


def test_pack_u4_roundtrip_and_order():
    q = np.array([[0, 15, 3, 12]], dtype=np.uint8)
    assert quant.pack_u4(q).tolist() == [[0xF0, 0xC3]]
    rng = np.random.default_rng(7)
    r = rng.integers(0, 16, (3, 32)).astype(np.uint8)
    assert np.array_equal(quant.unpack_u4(quant.pack_u4(r)), r)


def test_bf16_roundtrip():
    rng = np.random.default_rng(8)
    x = rng.standard_normal(1000).astype(F32)
    b = quant.f32_to_bf16_bits(x)
    xb = quant.bf16_bits_to_f32(b)
    assert np.array_equal(quant.f32_to_bf16_bits(xb), b)
    assert np.max(np.abs(xb - x) / np.abs(x)) <= 2.0**-8  # half of the 2^-7 ulp
    # ties to even: 1 + 2^-8 (exactly half a bf16 ulp) rounds down to 1
    assert quant.bf16_bits_to_f32(quant.f32_to_bf16_bits(np.array([1 + 2**-8], F32)))[0] == 1.0


# ---------------------------------------------------------------- weights

def test_u4_asym_known_groups():
    g = 4
    w = np.array([[0.0, 0.0, 0.0, 0.0,          # all-zero group -> s = 0, q = z = 0
                   1.5, 1.5, 1.5, 1.5,          # constant positive: range [0, 1.5], s = 0.1
                   -0.3, 0.0, 0.3, 0.45,        # straddles zero
                   -1.0, -1.0, 0.5, 0.5]],      # two-valued
                 dtype=F32)
    q, s, z = quant.quant_weight_u4_asym(w, g)
    sf = s.astype(np.float64)
    assert s[0, 0] == 0 and z[0, 0] == 0 and (q[0, :4] == 0).all()
    assert s[0, 1] == np.float16(0.1) and z[0, 1] == 0 and (q[0, 4:8] == 15).all()
    s2 = np.float16(np.float32(0.75) / np.float32(15))
    assert s[0, 2] == s2
    z2 = np.rint(np.float32(0.3) / np.float32(s2))
    assert z[0, 2] == z2
    deq = quant.dequant_u4_asym(q, s, z)
    assert np.max(np.abs(deq - w)[0, 4:]) <= 0.5 * sf[0, 1:].max() + 1e-6
    # two-valued group: both values are reproduced to within half a step
    assert np.allclose(deq[0, 12:], w[0, 12:], atol=0.5 * sf[0, 3] + 1e-6)


def test_u4_asym_random_error_bound():
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((32, 256)) * 0.02).astype(F32)
    q, s, z = quant.quant_weight_u4_asym(w, 64)
    assert q.max() <= 15 and z.max() <= 15
    deq = quant.dequant_u4_asym(q, s, z)
    step = np.repeat(s.astype(np.float64), 64, axis=1)
    # each element within half a step (+ the zero-point rounding of half a step)
    assert np.all(np.abs(deq - w) <= step + 1e-9)


def test_i4_sym_group_and_rowwise():
    w = np.array([[0.7, -0.7, 0.35, 0.05, 0, 0, 0, 0]], dtype=F32)
    q, s = quant.quant_weight_i4_sym_group(w, 4)
    assert s[0, 0] == np.float16(0.1) and s[0, 1] == 0
    s0 = np.float32(np.float16(0.1))
    assert q[0, :4].tolist() == [int(np.rint(F32(0.7) / s0)), -int(np.rint(F32(0.7) / s0)),
                                 int(np.rint(F32(0.35) / s0)), int(np.rint(F32(0.05) / s0))]
    assert (q[0, 4:] == 0).all()
    q2, s2 = quant.quant_weight_i4_rowwise(np.array([[7.0, -3.5, 0.0, 2.5]], F32))
    assert s2[0] == 1.0 and q2[0].tolist() == [7, -4, 0, 2]
    q3, s3 = quant.quant_weight_i8_rowwise(np.array([[127.0, -63.5, 0.5]], F32))
    assert s3.shape == (1, 1) and s3[0, 0] == 1.0 and q3[0].tolist() == [127, -64, 0]


def test_quant_per_token_non_finite_rows():
    """A row holding +-inf (an overflowed activation) gets scale +inf and code 0 everywhere; NaN
    entries get code 0 and do not count in the absmax; finite rows are unchanged."""
    x = np.array([[1.0, -2.0, np.inf, 0.5],
                  [1.0, np.nan, -4.0, 2.0],
                  [1.0, -2.0, 3.0, 0.5]], np.float32)
    q, s = quant.quant_per_token(x, 7)
    assert np.isinf(s[0]) and (q[0] == 0).all()
    # s = fp32(4 / 7) lies above 4 / 7, so 2 / s = 3.4999998 rounds to 3
    assert s[1] == np.float32(4.0) / np.float32(7) and q[1].tolist() == [2, 0, -7, 3]
    q2, s2 = quant.quant_per_token(x[2:], 7)
    assert np.array_equal(q[2], q2[0]) and s[2] == s2[0]
    # an fp16 SwiGLU product that overflows spreads inf / NaN over its Hadamard block
    from oracle import swiglu
    g = np.full((1, 64), 300.0, np.float32)
    u = np.full((1, 64), 1.0, np.float32)
    u[0, 5] = 240.0                                     # silu(300) * 240 = 72000 > 65504
    h = np.concatenate([g, u], axis=1)
    q, s = swiglu.swiglu_rotquant(h, 16, 4, dtype="f16")
    assert np.isinf(s[0]) and (q == 0).all()
