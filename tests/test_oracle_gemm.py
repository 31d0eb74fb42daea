"""Pins oracle.gemm / oracle.linear: exactness, closed forms, linearity (CPU only)."""
import numpy as np

from oracle import gemm, linear, quant


def test_partials_float64_equals_int64_bruteforce():
    rng = np.random.default_rng(10)
    qa = rng.integers(-127, 128, (7, 256)).astype(np.int8)
    wq = rng.integers(-15, 16, (5, 256)).astype(np.int16)
    assert np.array_equal(gemm.partials(qa, wq, 64), gemm.partials_int64(qa, wq, 64))


def test_partials_extreme_values_exact():
    qa = np.full((2, 128), 127, np.int8)
    qa[1] = -127
    wq = np.full((3, 128), 15, np.int16)
    wq[2] = -15
    p = gemm.partials(qa, wq, 64)
    assert p.shape == (2, 2, 3)
    assert p[0, 0, 0] == 64 * 127 * 15 and p[1, 1, 2] == 64 * 127 * 15 and p[0, 1, 0] == -64 * 127 * 15


def test_partials_one_hot_selects_single_weight():
    rng = np.random.default_rng(11)
    wq = rng.integers(-15, 16, (4, 128)).astype(np.int16)
    qa = np.zeros((128, 128), np.int8)
    np.fill_diagonal(qa, 1)
    p = gemm.partials(qa, wq, 64)
    # P[g, m, n] = wq[n, m] if m in group g else 0
    for g in range(2):
        for m in range(128):
            expect = wq[:, m] if m // 64 == g else np.zeros(4)
            assert np.array_equal(p[g, m], expect)


def test_zero_adjusted_and_epilogue_match_dequantized_matmul():
    rng = np.random.default_rng(12)
    w = (rng.standard_normal((6, 128)) * 0.02).astype(np.float32)
    q, s, z = quant.quant_weight_u4_asym(w, 64)
    qa = rng.integers(-127, 128, (5, 128)).astype(np.int8)
    sa = rng.uniform(0.01, 0.02, 5)
    bias = rng.standard_normal(6)
    p = gemm.partials(qa, gemm.zero_adjusted(q, z, 64), 64)
    y = gemm.epilogue_group(p, sa, s.astype(np.float64), bias)
    ref = (qa.astype(np.float64) * sa[:, None]) @ quant.dequant_u4_asym(q, s, z).T + bias
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-12)


def test_zero_point_only_weight_gives_minus_z_times_rowsum():
    q = np.zeros((2, 128), np.uint8)
    z = np.array([[3, 5], [0, 15]], np.uint8)
    qa = np.arange(-64, 64, dtype=np.int64).reshape(1, 128).astype(np.int8)
    p = gemm.partials(qa, gemm.zero_adjusted(q, z, 64), 64)
    rs = [int(qa[0, :64].astype(np.int64).sum()), int(qa[0, 64:].astype(np.int64).sum())]
    assert p[:, 0, :].tolist() == [[-3 * rs[0], 0], [-5 * rs[1], -15 * rs[1]]]


def test_linearity_in_activation_codes():
    rng = np.random.default_rng(13)
    a1 = rng.integers(-60, 60, (3, 192)).astype(np.int8)
    a2 = rng.integers(-60, 60, (3, 192)).astype(np.int8)
    wq = rng.integers(-15, 16, (4, 192)).astype(np.int16)
    p = gemm.partials((a1.astype(np.int16) + a2).astype(np.int8), wq, 64)
    assert np.array_equal(p, gemm.partials(a1, wq, 64) + gemm.partials(a2, wq, 64))


def test_w4a8_linear_approximates_float_linear():
    rng = np.random.default_rng(14)
    m, k, n = 16, 512, 24
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wr = linear.rotate_weight(w, 256)
    q, s, z = quant.quant_weight_u4_asym(wr, 64)
    res = linear.w4a8_asym_linear(x, q, s, z, None, 256, 64)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    # (xH)(WH)^T = xW^T; the error is the uint4 weight quantization noise (~8 %)
    assert gemm.rel_l2(ref, res.y) < 0.15
    # and the exact dequantized computation agrees to fp64 rounding
    deq = quant.dequant_u4_asym(q, s, z)
    exact = (res.qa.astype(np.float64) * res.sa[:, None]) @ deq.T
    assert gemm.rel_l2(exact, res.y) < 1e-12


def test_w4a4_and_w8a8_linears():
    rng = np.random.default_rng(15)
    m, k, n = 8, 256, 16
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wr = linear.rotate_weight(w, 64)
    q4, s4 = quant.quant_weight_i4_sym_group(wr, 64)
    r = linear.w4a4_group_linear(x, q4, s4, None, 64, 64)
    assert r.qa.min() >= -7 and r.qa.max() <= 7
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    assert gemm.rel_l2(ref, r.y) < 0.35
    q8, s8 = quant.quant_weight_i8_rowwise(linear.rotate_weight(w, 256))
    r8 = linear.w8a8_linear(x, q8, s8, None, 256)
    assert gemm.rel_l2(ref, r8.y) < 0.02
    qr, sr = quant.quant_weight_i4_rowwise(linear.rotate_weight(w, 256))
    rr = linear.w4a4_row_linear(x, qr, sr, None, 256, 4)
    assert rr.partials.shape == (1, m, n) and gemm.rel_l2(ref, rr.y) < 0.4
