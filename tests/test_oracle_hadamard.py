"""Pins oracle.hadamard against closed forms and invariants (CPU only)."""
import numpy as np
import pytest

from oracle.hadamard import BLOCKS, fwht_pinned, h4_half, hadamard, rotate_matmul64


def test_h4_half_rows_match_reference_comment():
    # g64_quant.cu:7: y_i = (x0 + x1 + x2 + x3)/2 - x_{3-i}
    expect = np.array([[0.5, 0.5, 0.5, -0.5],
                       [0.5, 0.5, -0.5, 0.5],
                       [0.5, -0.5, 0.5, 0.5],
                       [-0.5, 0.5, 0.5, 0.5]])
    assert np.array_equal(h4_half(), expect)


@pytest.mark.parametrize("b", BLOCKS)
def test_hadamard_invariants(b):
    h = hadamard(b)
    assert h.shape == (b, b)
    assert np.array_equal(h, h.T)
    assert np.allclose(h @ h, np.eye(b), atol=1e-12)
    assert np.allclose(np.abs(h), 1 / np.sqrt(b))


def test_hadamard_kronecker_recursion():
    assert np.array_equal(hadamard(64), np.kron(h4_half(), hadamard(16)))
    assert np.array_equal(hadamard(256), np.kron(hadamard(16), hadamard(16)))


@pytest.mark.parametrize("b", BLOCKS)
def test_one_hot_gives_columns_exactly(b):
    # A one-hot row passes through every stage with values +-2^-j: exact in fp32.
    x = np.eye(b, dtype=np.float32)
    y = fwht_pinned(x, b)
    assert np.array_equal(y.astype(np.float64), hadamard(b))


@pytest.mark.parametrize("b", BLOCKS)
def test_fwht_matches_matmul_form(b):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((8, 3 * b)).astype(np.float32)
    y = fwht_pinned(x, b).astype(np.float64)
    ref = rotate_matmul64(x, b)
    # fp32 rounding of log4(b) stages of 4-term sums
    assert np.max(np.abs(y - ref)) < 1e-5 * np.max(np.abs(ref))


def test_fwht_is_an_involution_and_norm_preserving():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 512)).astype(np.float32)
    y = fwht_pinned(x, 256)
    assert np.allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x, axis=1), rtol=1e-5)
    assert np.allclose(fwht_pinned(y, 256), x, atol=1e-5)


def test_blocks_do_not_mix():
    x = np.zeros((1, 512), np.float32)
    x[0, 300] = 1.0
    y = fwht_pinned(x, 256)
    assert np.all(y[0, :256] == 0)
    assert np.array_equal(y[0, 256:].astype(np.float64), hadamard(256)[:, 300 - 256])


def test_pinned_order_is_left_to_right_sum():
    """Hand-computed case where the reference's association ((x0+x1)+x2)+x3 (g64_quant.cu:79)
    gives a different fp32 result than any pairwise order: a wrong order fails this test."""
    e = np.float32(2.0**-24)
    xx = np.zeros((1, 16), np.float32)
    xx[0, :4] = [1.0, e, e, -1.0]
    out = fwht_pinned(xx, 16)
    # stage stride 1: h = 0.5*(((1 + e) + e) - 1) = 0 (each + e rounds back to 1)
    #   -> y = [1, -e, -e, -1]; stage stride 4 (other groups are 0): out[i + 4j] = 0.5*y_i
    #   for j < 3 and -0.5*y_i for j = 3.
    y1 = np.array([1.0, -e, -e, -1.0], np.float64)
    expect = np.zeros(16)
    for i in range(4):
        expect[i], expect[i + 4], expect[i + 8], expect[i + 12] = 0.5 * y1[i], 0.5 * y1[i], 0.5 * y1[i], -0.5 * y1[i]
    assert np.array_equal(out[0].astype(np.float64), expect)
    # pairwise association (x0 + x3) + (x1 + x2) would give h = 2^-24 and y_1 = 0 instead
    h_pair = np.float32(0.5) * ((np.float32(1.0) + np.float32(-1.0)) + (e + e))
    assert h_pair - e == 0.0 and expect[1] != 0.0
