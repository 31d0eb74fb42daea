"""int8 weights in the 16-row tile layout (MQ_W8_TILE16, ops.tile_int8_weight): the layout itself,
the full-K int32 sums against the oracle, and whole linears bit-identical to the same weights as
[N, K] rows at every M path (GEMV, the wide kernel's 128 / 192 / 256 tiles, trailing rows,
split-K). Each case prints its name before the GPU step."""
import numpy as np
import pytest
import torch

from kitchen_amd import _lib, ops, synth
from oracle import gemm

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _untile(wt: np.ndarray, n: int) -> np.ndarray:
    """[ceil(N/16), K/64, 16, 64] -> [N, K]: block [b, g] is bytes 64 g .. of rows 16 b .. 16 b + 15."""
    nb, g = wt.shape[:2]
    return wt.transpose(0, 2, 1, 3).reshape(nb * 16, g * 64)[:n]


@pytest.mark.parametrize("n,k", [(17, 192), (3000, 1024), (3072, 3072)])
def test_layout(gpu_device, n, k):
    print(f"[tile16] layout N={n} K={k}", flush=True)
    rng = np.random.default_rng(n + k)
    w = rng.integers(-128, 128, (n, k)).astype(np.int8)
    wt = ops.tile_int8_weight(_t(w, gpu_device)).cpu().numpy()
    assert wt.shape == ((n + 15) // 16, k // 64, 16, 64)
    assert np.array_equal(_untile(wt, n), w)
    # block [b, g] row r is the 64 bytes at row 16 b + r, columns 64 g ..
    b, g, r = (n - 1) // 16, k // 64 - 1, (n - 1) % 16
    assert np.array_equal(wt[b, g, r], w[n - 1, 64 * g:64 * g + 64])
    assert not wt.transpose(0, 2, 1, 3).reshape(-1, k)[n:].any()   # rows past N are zero


def test_layout_of_a_strided_weight(gpu_device):
    print("[tile16] strided [N, K] view", flush=True)
    rng = np.random.default_rng(3)
    wide = rng.integers(-128, 128, (40, 512)).astype(np.int8)
    w = _t(wide, gpu_device)[:, :256]                 # row stride 512 bytes
    wt = ops.tile_int8_weight(w).cpu().numpy()
    assert np.array_equal(_untile(wt, 40), wide[:, :256])


# M through every path: GEMV (1, 4), the wide kernel's 128 tiles at small M (5, 64, 129, 256), its
# ragged larger tiles (300, 2900)
@pytest.mark.parametrize("m,n,k", [(1, 3000, 3072), (4, 17, 192), (5, 3072, 1024), (64, 300, 448),
                                   (129, 3000, 3072), (256, 3072, 12288), (300, 2000, 512), (2900, 3000, 1024)])
def test_int32_sums_against_oracle(gpu_device, m, n, k):
    print(f"[tile16] acc M={m} N={n} K={k}", flush=True)
    rng = np.random.default_rng(m * 7 + n)
    qa = rng.integers(-127, 128, (m, k)).astype(np.int8)
    qw = rng.integers(-127, 128, (n, k)).astype(np.int8)
    wt = ops.tile_int8_weight(_t(qw, gpu_device))
    acc = ops.gemm_rowscale_acc(_t(qa, gpu_device), wt, n, 8)
    torch.cuda.synchronize()
    p0 = gemm.partials(qa, qw, k)[0]
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), p0)


@pytest.mark.parametrize("m,n,k", [(1, 18432, 3072), (3, 3072, 3072), (77, 3072, 3072), (256, 12288, 3072),
                                   (256, 3072, 12288), (4096, 3072, 3072), (4352, 12288, 3072)])
def test_linear_bitidentical_to_rows(gpu_device, m, n, k):
    # the whole W8A8 linear (rotate + quantize, GEMM, epilogue): tiled and [N, K] weights give the
    # same bf16 outputs bit for bit; K = 12288 at M = 256 runs split along K, M = 4352 against
    # N = 12288 runs its last 256 rows as a trailing product
    print(f"[tile16] linear M={m} N={n} K={k}", flush=True)
    x = synth.to_bf16_tensor(synth.activations(m, k, seed=m + 1), gpu_device)
    gen = torch.Generator(device=gpu_device).manual_seed(n + k)
    w = torch.randint(-127, 128, (n, k), generator=gen, device=gpu_device, dtype=torch.int8)
    s = torch.rand(n, 1, generator=gen, device=gpu_device) * 2e-4 + 3e-4
    bias = (torch.randn(n, generator=gen, device=gpu_device) * 0.02).to(torch.bfloat16)
    y_rows = ops.int8_linear(x, w, s, bias, torch.bfloat16, True, 256)
    y_tile = ops.int8_linear(x, ops.tile_int8_weight(w), s, bias, torch.bfloat16, True, 256)
    torch.cuda.synchronize()
    assert torch.equal(y_rows.view(torch.int16), y_tile.view(torch.int16))


def test_rejects_what_the_layout_does_not_cover(gpu_device):
    print("[tile16] argument checks", flush=True)
    qa = torch.zeros(8, 192, dtype=torch.int8, device=gpu_device)
    wt = ops.tile_int8_weight(torch.zeros(16, 192, dtype=torch.int8, device=gpu_device))
    with pytest.raises(ValueError, match="int8 weights"):
        ops.gemm_rowscale_acc(qa, wt, 16, 4)
    with pytest.raises(ValueError, match="must be contiguous"):
        ops.gemm_rowscale_acc(qa, wt, 40, 8)            # shape of another N
    with pytest.raises(ValueError, match="K >= 192"):
        _lib.call("mq_tile_weight_i8", wt.data_ptr(), 128, 16, 128, wt.data_ptr(), _lib.stream_of(wt))


# The whole-linear entries write the activation codes in 16-row tiles wherever the wide kernel runs
# their product (MQ_W8_TILE16's layout, for A); the same linear in two steps keeps them as rows.
# Both give the same output bits: W8A8 (rows and tiled weights), W4A8 group scale, W4A4 group scale
# (int4 x16 codes), including trailing rows (M = 4352, N = 12288) and split-K (M = 256, K = 12288).
@pytest.mark.parametrize("m,n,k", [(129, 3000, 3072), (300, 2000, 512), (256, 3072, 12288), (4096, 3072, 3072),
                                   (4352, 12288, 3072)])
def test_w8a8_linear_matches_two_steps(gpu_device, m, n, k):
    print(f"[tile16] w8a8 two-step M={m} N={n} K={k}", flush=True)
    x = synth.to_bf16_tensor(synth.activations(m, k, seed=m), gpu_device)
    gen = torch.Generator(device=gpu_device).manual_seed(k)
    w = torch.randint(-127, 128, (n, k), generator=gen, device=gpu_device, dtype=torch.int8)
    s = torch.rand(n, generator=gen, device=gpu_device) * 2e-4 + 3e-4
    bias = (torch.randn(n, generator=gen, device=gpu_device) * 0.02).to(torch.bfloat16)
    qa, sa = ops.rotate_quantize(x, 256, 8, _lib.Q_BYTES)
    y2 = ops.gemm_rowscale(qa, sa, w, s, bias, n, 8)
    for wl in (w, ops.tile_int8_weight(w)):
        y1 = ops.int8_linear(x, wl, s, bias, torch.bfloat16, True, 256)
        torch.cuda.synchronize()
        assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))


@pytest.mark.parametrize("m,n,k", [(300, 2000, 512), (4096, 3072, 3072), (4352, 12288, 3072)])
@pytest.mark.parametrize("act_bits", [8, 4])
def test_w4_group_linear_matches_two_steps(gpu_device, m, n, k, act_bits):
    print(f"[tile16] w4 group two-step act{act_bits} M={m} N={n} K={k}", flush=True)
    x = synth.to_bf16_tensor(synth.activations(m, k, seed=m + 5), gpu_device)
    gen = torch.Generator(device=gpu_device).manual_seed(k + 1)
    qd = torch.randint(0, 256, (n, k // 2), generator=gen, device=gpu_device, dtype=torch.uint8)
    s16 = (torch.rand(n, k // 64, generator=gen, device=gpu_device) * 0.004 + 0.004).to(torch.float16)
    zp = torch.randint(0, 256, (n, (k // 64 + 1) // 2), generator=gen, device=gpu_device, dtype=torch.uint8)
    bias = (torch.randn(n, generator=gen, device=gpu_device) * 0.02).to(torch.bfloat16)
    hb = 256 if act_bits == 8 else 64
    y1 = ops._linear_w4_group(x, False, hb, act_bits, qd, s16, zp, bias, n, k, torch.bfloat16)
    layout, mode = (_lib.Q_BYTES, _lib.ACT_I8) if act_bits == 8 else (_lib.Q_X16ALT, _lib.ACT_X16ALT)
    qa, sa = ops.rotate_quantize(x, hb, act_bits, layout)
    y2 = ops.gemm_w4_group(qa, sa, qd, s16, zp, bias, n, act_mode=mode)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
