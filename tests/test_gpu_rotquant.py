"""GPU parity of the fused rotate + per-token quantizer (mq_rotquant) against the CPU oracle.

Bar: activation codes and scales bit-exact. Each case prints its name before the GPU step."""
import numpy as np
import pytest
import torch

from kitchen_amd import _lib, ops, synth
from oracle import quant

pytestmark = pytest.mark.gpu


def _run(xbits, hblock, bits, packed, dev):
    x = synth.to_bf16_tensor(xbits, dev)
    q, s = ops.rotate_quantize(x, hblock, bits, packed)
    torch.cuda.synchronize()
    return q.cpu().numpy(), s.cpu().numpy()


def _oracle(xbits, hblock, bits):
    xf = synth.bf16_bits_to_f32(xbits)
    if hblock:
        return quant.rotquant(xf, hblock, bits)
    return quant.quant_per_token(xf, 127 if bits == 8 else 7)


def _check(xbits, hblock, bits, packed, dev, label):
    print(f"[rotquant] {label} M={xbits.shape[0]} K={xbits.shape[1]} hblock={hblock} bits={bits} packed={packed}",
          flush=True)
    q, s = _run(xbits, hblock, bits, packed, dev)
    q0, s0 = _oracle(xbits, hblock, bits)
    assert np.array_equal(s.view(np.uint32), s0.view(np.uint32)), "scales differ"
    if packed == _lib.Q_X16ALT:
        # the group GEMM's int4 operand layout: 16 * q, negated in odd 64-column groups
        sign = np.where((np.arange(q0.shape[1]) // 64) % 2 == 1, -1, 1).astype(np.int16)
        assert np.array_equal(q.astype(np.int16), 16 * q0.astype(np.int16) * sign[None, :]), "x16alt codes differ"
    elif packed:
        assert np.array_equal(q, quant.pack_i4(q0)), "packed codes differ"
    else:
        diff = np.nonzero(q != q0)
        assert diff[0].size == 0, f"{diff[0].size} codes differ, first at {diff[0][0]},{diff[1][0]}"


MODES = [(8, False), (4, False), (4, True), (4, _lib.Q_X16ALT)]


@pytest.mark.parametrize("hblock", [0, 16, 64, 256])
@pytest.mark.parametrize("bits,packed", MODES)
def test_config0_shape_bitexact(gpu_device, hblock, bits, packed):
    # C0 activations: [1024, 3072] N(0,1) with 1 % outlier channels x20, seed 0
    xb = synth.activations(1024, 3072, seed=0)
    _check(xb, hblock, bits, packed, gpu_device, "C0")


@pytest.mark.parametrize("hblock", [16, 64, 256])
def test_config2_spikes_bitexact(gpu_device, hblock):
    # C2: outliers x20 plus 0.1 % token spikes x50, int4 activations
    xb = synth.activations(2048, 3072, seed=2, spike_frac=0.001)
    _check(xb, hblock, 4, True, gpu_device, "C2")


@pytest.mark.parametrize("k", [256, 512, 768, 1024, 1280, 2048, 9216, 12288, 14336, 16384])
def test_k_range_bitexact(gpu_device, k):
    xb = synth.activations(37, k, seed=k)
    for hb in (64, 256):
        _check(xb, hb, 8, False, gpu_device, f"K{k}")
    _check(xb, 256, 4, True, gpu_device, f"K{k}")
    _check(xb, 64, 4, _lib.Q_X16ALT, gpu_device, f"K{k}")


@pytest.mark.parametrize("m", [1, 2, 3, 5, 63, 65])
def test_m_tails(gpu_device, m):
    _check(synth.activations(m, 3072, seed=m), 256, 8, False, gpu_device, "Mtail")
    _check(synth.activations(m, 3072, seed=m), 64, 4, True, gpu_device, "Mtail")


def test_small_k_no_rotation_and_block16(gpu_device):
    xb = synth.activations(9, 16, seed=3)
    _check(xb, 0, 8, False, gpu_device, "K16")
    _check(xb, 16, 4, True, gpu_device, "K16")
    _check(xb, 16, 4, _lib.Q_X16ALT, gpu_device, "K16")


def test_zero_rows_and_exact_ties(gpu_device):
    # hblock 0 keeps the values, so exact half-integer quotients reach the tie path:
    # row 1: absmax 127 -> s = 1; 2.5 -> 2, 3.5 -> 4, -0.5 -> 0 (ties to even)
    m, k = 4, 64
    x = np.zeros((m, k), np.float32)
    x[1, :8] = [127.0, 2.5, 3.5, -0.5, 1.5, -2.5, 0.5, 126.5]
    x[2, :] = np.arange(k, dtype=np.float32) - 31.5         # many exact halves after scaling
    x[2, 0] = 127.0
    x[3, :] = 1e-39                                           # subnormal row -> s = 1e-10 clamp
    xb = synth.f32_to_bf16_bits(x)
    _check(xb, 0, 8, False, gpu_device, "ties")
    _check(xb, 0, 4, False, gpu_device, "ties")
    _check(xb, 16, 8, False, gpu_device, "ties-rot")


@pytest.mark.parametrize("hblock", [0, 256])
def test_extreme_row_magnitudes(gpu_device, hblock):
    # Rows scaled across the float range pin the row scale (formed without a division) and the
    # reciprocal behind the codes at every exponent: subnormal-scale rows (the 1e-10 clamp), tiny,
    # ordinary and huge rows. Without rotation the largest row reaches 1e38; with it, rows stay
    # below 1e36 so no butterfly sum overflows.
    rng = np.random.default_rng(21)
    exps = [-39, -36, -30, -20, -12, -10, -8, -3, 0, 3, 10, 20, 30, 35, 38]
    m, k = len(exps), 1024
    x = rng.standard_normal((m, k)).astype(np.float32)
    for r, e in enumerate(exps):
        top = 1.0e38 if hblock == 0 else 1.0e35
        x[r] *= np.float32(min(10.0 ** e, top) / 4.0)
    xb = synth.f32_to_bf16_bits(x)
    for bits, packed in ((8, False), (4, False)):
        _check(xb, hblock, bits, packed, gpu_device, "magnitudes")


def test_near_tie_window_exercised(gpu_device):
    # Rotated fp32 values have full mantissas, so some quotients x*(1/s) land within 2^-16 of a
    # half-integer, where the kernel recomputes x / s exactly. Count them with the oracle's
    # arithmetic to make sure this case is really exercised, then require bit-exact codes.
    xb = synth.activations(4096, 3072, seed=9)
    xf = synth.bf16_bits_to_f32(xb)
    from oracle.hadamard import fwht_pinned

    xr = fwht_pinned(xf, 256).astype(np.float64)
    s = np.maximum(np.abs(xr).max(axis=1) / 127, 1e-10)
    t = xr / s[:, None]
    near = np.abs(np.abs(t - np.floor(t)) - 0.5) < 2.0**-15
    print(f"[rotquant] near-tie elements: {int(near.sum())}", flush=True)
    assert near.sum() > 10
    _check(xb, 256, 8, False, gpu_device, "near-ties")


def test_strided_input_c_abi(gpu_device):
    print("[rotquant] strided ldx", flush=True)
    xb = synth.activations(33, 1024, seed=11)
    wide = np.zeros((33, 1536), np.uint16)
    wide[:, :1024] = xb
    xw = synth.to_bf16_tensor(wide, gpu_device)
    q = torch.full((33, 1040), 99, dtype=torch.int8, device=gpu_device)   # ldq 1040 > K
    s = torch.empty(33, dtype=torch.float32, device=gpu_device)
    _lib.call("mq_rotquant", xw.data_ptr(), _lib.DT_BF16, 33, 1024, 1536, 256, 8, 0, q.data_ptr(), 1040, s.data_ptr(),
              _lib.stream_of(xw))
    torch.cuda.synchronize()
    q0, s0 = _oracle(xb, 256, 8)
    qn = q.cpu().numpy()
    assert np.array_equal(qn[:, :1024], q0) and np.array_equal(s.cpu().numpy(), s0)
    assert (qn[:, 1024:] == 99).all(), "wrote past K"


def test_config3_video_tokens_subset(gpu_device):
    # C3: [32760, 3072]; compare a deterministic subset of rows, and check the size-independent
    # properties on all rows (codes within +-127, every row has a code at +-127 unless all-zero).
    m, k = 32760, 3072
    xb = synth.activations(m, k, seed=3)
    print(f"[rotquant] C3 M={m} K={k}", flush=True)
    q, s = _run(xb, 256, 8, False, gpu_device)
    assert np.abs(q.astype(np.int16)).max(axis=1).min() == 127
    rows = np.r_[0:256, m - 256:m, np.random.default_rng(0).choice(m, 256, replace=False)]
    q0, s0 = _oracle(xb[rows], 256, 8)
    assert np.array_equal(q[rows], q0) and np.array_equal(s[rows], s0)


@pytest.fixture(scope="module")
def large_x():
    # [9600, 14336] (C3's MLP-down width): generated once for the cases below (about 17 s)
    return synth.activations(9600, 14336, seed=4)


@pytest.mark.parametrize("bits,packed", [(8, False), (4, True), (4, _lib.Q_X16ALT)])
def test_large_output_rows_subset(gpu_device, large_x, bits, packed):
    # outputs of 64 MiB and more take the non-temporal code stores: [9600, 14336] gives 137.6 MB
    # of one-byte codes or 68.8 MB packed (four waves per row); a subset of rows against the
    # oracle, and the code range on all rows
    xb = large_x
    m, k = xb.shape
    print(f"[rotquant] large output M={m} K={k} bits={bits} packed={packed}", flush=True)
    q, s = _run(xb, 256, bits, packed, gpu_device)
    rows = np.r_[0:128, m - 128:m, np.random.default_rng(1).choice(np.arange(128, m - 128), 128, replace=False)]
    q0, s0 = _oracle(xb[rows], 256, bits)
    assert np.array_equal(s[rows].view(np.uint32), s0.view(np.uint32)), "scales differ"
    if packed == _lib.Q_X16ALT:
        sign = np.where((np.arange(k) // 64) % 2 == 1, -1, 1).astype(np.int16)
        assert np.array_equal(q[rows].astype(np.int16), 16 * q0.astype(np.int16) * sign[None, :])
        assert (q.view(np.int8) % 16 == 0).all()
    elif packed:
        assert np.array_equal(q[rows], quant.pack_i4(q0)), "packed codes differ"
    else:
        assert np.array_equal(q[rows], q0), "codes differ"
        assert np.abs(q.astype(np.int16)).max(axis=1).min() == 127


def test_deterministic(gpu_device):
    xb = synth.activations(512, 3072, seed=5)
    a = _run(xb, 256, 8, False, gpu_device)
    b = _run(xb, 256, 8, False, gpu_device)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
