"""The package's offline weight quantizers (torch) reproduce the oracle bit for bit (CPU only)."""
import numpy as np
import pytest
import torch

from kitchen_amd import weights
from oracle import linear, quant
from oracle.hadamard import fwht_pinned


@pytest.mark.parametrize("block", [16, 64, 256])
def test_torch_fwht_matches_oracle_bitwise(block):
    rng = np.random.default_rng(20)
    x = (rng.standard_normal((16, 1024)) * rng.uniform(0.001, 100, (16, 1))).astype(np.float32)
    got = weights.fwht(torch.from_numpy(x), block).numpy()
    assert np.array_equal(got.view(np.uint32), fwht_pinned(x, block).view(np.uint32))


def _w(n=48, k=512, seed=21):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((n, k)) * 0.02).astype(np.float32)


def test_w4a8_asym_weight_bitexact():
    w = _w()
    qd, s, z = weights.quantize_w4a8_asym_weight(torch.from_numpy(w), 64, 256)
    q0, s0, z0 = quant.quant_weight_u4_asym(linear.rotate_weight(w, 256), 64)
    assert np.array_equal(qd.numpy(), quant.pack_u4(q0))
    assert np.array_equal(s.numpy().view(np.uint16), s0.view(np.uint16))
    assert np.array_equal(z.numpy(), quant.pack_u4(z0))


def test_w4a4_group_weight_bitexact():
    w = _w(seed=22)
    qw, s = weights.quantize_w4a4_group_weight(torch.from_numpy(w), 64, 64)
    q0, s0 = quant.quant_weight_i4_sym_group(linear.rotate_weight(w, 64), 64)
    assert np.array_equal(qw.numpy(), quant.pack_i4(q0))
    assert np.array_equal(s.numpy().view(np.uint16), s0.view(np.uint16))


def test_convrot_w4a4_and_int8_weights_bitexact():
    w = _w(seed=23)
    qw, s = weights.quantize_convrot_w4a4_weight(torch.from_numpy(w), 256, 64)
    q0, s0 = quant.quant_weight_i4_rowwise(linear.rotate_weight(w, 256))
    assert np.array_equal(qw.numpy(), quant.pack_i4(q0)) and np.array_equal(s.numpy(), s0)
    q8, s8 = weights.quantize_int8_convrot_weight(torch.from_numpy(w), 256)
    q1, s1 = quant.quant_weight_i8_rowwise(linear.rotate_weight(w, 256))
    assert np.array_equal(q8.numpy(), q1) and np.array_equal(s8.numpy(), s1)
    with pytest.raises(ValueError, match="quant_group_size"):
        weights.quantize_convrot_w4a4_weight(torch.from_numpy(w), 256, 32)


def test_rejects_bad_shapes():
    with pytest.raises(ValueError, match="convrot"):
        weights.fwht(torch.zeros(2, 96), 32)
    with pytest.raises(ValueError, match="multiple"):
        weights.fwht(torch.zeros(2, 96), 64)


def test_ops_refuse_host_tensors():
    from kitchen_amd import ops

    with pytest.raises(ValueError, match="linear_dtype"):
        ops.convrot_w4a4_linear(torch.zeros(2, 256), torch.zeros(4, 128, dtype=torch.int8),
                                torch.ones(4), linear_dtype="fp8")
    with pytest.raises(ValueError, match="quant_group_size"):
        ops.convrot_w4a4_linear(torch.zeros(2, 256), torch.zeros(4, 128, dtype=torch.int8),
                                torch.ones(4), quant_group_size=32)
    with pytest.raises(ValueError, match="does not match"):
        ops.convrot_w4a4_linear(torch.zeros(2, 256), torch.zeros(4, 64, dtype=torch.int8), torch.ones(4))
    with pytest.raises(ValueError, match="device"):
        ops.rotate_quantize(torch.zeros(2, 256), 256, 8)
