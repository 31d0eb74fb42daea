"""4-bit weights expanded once to int8 16-row tiles (mq_expand_weight_w4, ops.ExpandedW4).

The expansion is this library's layout, not the reference's: its bytes are checked against a numpy
restatement of the packed kernels' unpack (q - z or the signed nibble; negated in odd K groups
for int8 activations, x16 for signed weights under the x16 int4 activation layout), and every
GEMM and linear that reads it against the same call on the packed weights, bit for bit. The
packed calls are themselves pinned against the oracle (test_gpu_gemm, test_gpu_linear,
test_gpu_configs), so equality carries that parity over."""
import numpy as np
import pytest
import torch

import kitchen_amd as ck
from kitchen_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu


def _expand_np(qw: np.ndarray, wz, n: int, k: int, layout: int) -> np.ndarray:
    """int8 [ceil(n / 16), k / 64, 16, 64] from packed bytes qw [n, k / 2] (low nibble = even k)."""
    q = np.stack([qw & 15, qw >> 4], axis=-1).reshape(n, k).astype(np.int32)
    g = np.arange(k) // 64
    if wz is not None:
        z = np.stack([wz & 15, wz >> 4], axis=-1).reshape(n, -1)[:, : k // 64].astype(np.int32)
        v = q - z[:, g]
    else:
        v = np.where(q >= 8, q - 16, q)
    if layout == _lib.ACT_I8:
        v = np.where(g % 2 == 1, -v, v)
    elif layout == _lib.ACT_X16ALT and wz is None:
        v = 16 * v
    nb = (n + 15) // 16
    out = np.zeros((nb * 16, k), dtype=np.int8)
    out[:n] = v.astype(np.int8)
    return out.reshape(nb, 16, k // 64, 64).transpose(0, 2, 1, 3)


def _scale_pairs_np(s16, n, k):
    """The group scales as the expansion carries them: uint32 [4 ceil(K/256)][16][ld], dword
    [g][c][u] = s[32u + c, g] | s[32u + 16 + c, g] << 16, zero past N and K/64."""
    g = k // 64
    g4, ld = (g + 3) // 4 * 4, ((n + 15) // 16 + 17) // 2
    bits = np.zeros((2 * ld * 16, g4), dtype=np.uint32)        # [column, group], columns padded
    bits[:n, :g] = s16.view(np.uint16)[:, :g]
    cols = bits.reshape(ld, 2, 16, g4)                           # [u][half][c][g]
    return (cols[:, 0] | (cols[:, 1] << 16)).transpose(2, 1, 0)  # [g][c][u]


@pytest.mark.parametrize("layout", [_lib.ACT_I8, _lib.ACT_X16ALT, _lib.W4X_ROW])
@pytest.mark.parametrize("asym", [True, False])
@pytest.mark.parametrize("n,k", [(16, 192), (40, 320), (1, 128), (77, 3072)])
def test_expansion_bytes(gpu_device, layout, asym, n, k):
    print(f"[expand] bytes n={n} k={k} asym={asym} layout={layout}", flush=True)
    rng = np.random.default_rng(n * 7 + k)
    qw = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    wz = rng.integers(0, 256, (n, (k // 64 + 1) // 2), dtype=np.uint8) if asym else None
    # fp16 scales from random bits (finite: exponent field below 31), a padded row stride
    s16 = rng.integers(0, 1 << 16, (n, k // 64 + 3), dtype=np.uint16)
    s16 = np.where((s16 & 0x7c00) == 0x7c00, s16 & 0x3fff, s16).view(np.float16)
    s16_t = torch.from_numpy(s16).to(gpu_device)[:, : k // 64]
    ex = ck.expand_w4_weight(torch.from_numpy(qw).to(gpu_device),
                             None if wz is None else torch.from_numpy(wz).to(gpu_device), layout,
                             None if layout == _lib.W4X_ROW else s16_t)
    torch.cuda.synchronize()
    assert ex.tiles.shape == ((n + 15) // 16, k // 64, 16, 64) and ex.asym == asym
    assert np.array_equal(ex.tiles.cpu().numpy(), _expand_np(qw, wz, n, k, layout))
    tiles = (n + 15) // 16 * 16 * k
    if layout == _lib.W4X_ROW:
        assert ex.buf.numel() == tiles
    else:
        pairs = ex.buf[tiles:].cpu().numpy().view(np.uint32)
        want = _scale_pairs_np(np.ascontiguousarray(s16[:, : k // 64]), n, k)
        assert pairs.size == want.size and np.array_equal(pairs, want.reshape(-1))


def _group_weights(n, k, asym, dev, seed):
    w = torch.from_numpy(synth.weight(n, k, seed=seed)).to(dev)
    if asym:
        return ck.quantize_w4a8_asym_weight(w, 64, 256)
    qw, s16 = ck.quantize_w4a4_group_weight(w, 64, 64)
    return qw, s16, None


# few rows (128 tiles, split-K), one round of 256 x 192 tiles, 256 x 256 tiles, trailing rows
SHAPES = [(5, 1024, 3072), (100, 768, 2048), (256, 1536, 3072), (700, 3072, 3072), (1000, 640, 256),
          (4096, 3072, 3072), (4096, 4096, 1024), (4352, 12288, 256)]


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("act_mode", [_lib.ACT_I8, _lib.ACT_X16ALT])
@pytest.mark.parametrize("asym", [True, False])
def test_group_gemm_expanded_equals_packed(gpu_device, m, n, k, act_mode, asym):
    print(f"[expand] group gemm M={m} N={n} K={k} act_mode={act_mode} asym={asym}", flush=True)
    qw, s16, zp = _group_weights(n, k, asym, gpu_device, seed=m + n)
    x = synth.to_bf16_tensor(synth.activations(m, k, seed=m), gpu_device)
    if act_mode == _lib.ACT_I8:
        qa, sa = ops.rotate_quantize(x, 256, 8)
    else:
        qa, sa = ops.rotate_quantize(x, 64, 4, _lib.Q_X16ALT)
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(n)) * 0.1).to(torch.bfloat16).to(gpu_device)
    out = torch.float32 if m == 700 else torch.bfloat16
    ex = ck.expand_w4_weight(qw.view(torch.uint8), None if zp is None else zp.view(torch.uint8), act_mode, s16)
    y = ops.gemm_w4_group(qa, sa, ex, s16, None, bias, n, act_mode=act_mode, out_dtype=out)
    y0 = ops.gemm_w4_group(qa, sa, qw.view(torch.uint8), s16, None if zp is None else zp.view(torch.uint8), bias, n,
                           act_mode=act_mode, out_dtype=out)
    torch.cuda.synchronize()
    if m > ops.FEW_ROWS:
        assert torch.equal(y, y0)
    else:
        # the packed weights' few rows run on the 128 x 128 kernel (int32 partials converted, then one
        # fp32 fma per group): the same exact partials, summed in fp32 in another order, so the
        # outputs agree to within a rounding step of the output type
        assert torch.allclose(y.float(), y0.float(), rtol=2 ** -7, atol=2e-2)


# K groups not a multiple of four (odd, and 2 mod 4) on the 256-row tiles (256 x 192, 256 x 256,
# trailing rows), whose lanes read the group scales the expansion carries (zero-padded past G),
# and on the 128 x 128 tile; the scale and zero-point rows padded to even strides, as the wide
# kernel loads them (so the packed weights run on it too)
ODD_G = [(2100, 4000, 320), (2100, 4000, 1472), (4096, 12288, 320), (4096, 12288, 448), (4352, 12288, 1920),
         (700, 3000, 192)]


@pytest.mark.parametrize("m,n,k", ODD_G)
@pytest.mark.parametrize("act_mode", [_lib.ACT_I8, _lib.ACT_X16ALT])
@pytest.mark.parametrize("asym", [True, False])
def test_expanded_equals_packed_uneven_groups(gpu_device, m, n, k, act_mode, asym):
    print(f"[expand] uneven groups M={m} N={n} K={k} act_mode={act_mode} asym={asym}", flush=True)
    g = k // 64
    w = torch.from_numpy(synth.weight(n, k, seed=k)).to(gpu_device)
    if asym:
        qw, s16, zp = ck.quantize_w4a8_asym_weight(w, 64, 64)
        zc = zp.shape[1]
        zpp = torch.zeros((n, zc + zc % 2), dtype=torch.uint8, device=gpu_device)
        zpp[:, :zc] = zp.view(torch.uint8)
        zp = zpp[:, :zc]
    else:
        (qw, s16), zp = ck.quantize_w4a4_group_weight(w, 64, 64), None
    sp = torch.zeros((n, g + g % 2), dtype=torch.float16, device=gpu_device)
    sp[:, :g] = s16
    s16 = sp[:, :g]
    x = synth.to_bf16_tensor(synth.activations(m, k, seed=m), gpu_device)
    qa, sa = ops.rotate_quantize(x, 64, 8) if act_mode == _lib.ACT_I8 else ops.rotate_quantize(x, 64, 4, _lib.Q_X16ALT)
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(n)) * 0.1).to(torch.bfloat16).to(gpu_device)
    ex = ck.expand_w4_weight(qw.view(torch.uint8), zp, act_mode, s16)
    y = ops.gemm_w4_group(qa, sa, ex, s16, None, bias, n, act_mode=act_mode)
    y0 = ops.gemm_w4_group(qa, sa, qw.view(torch.uint8), s16, zp, bias, n, act_mode=act_mode)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all() and torch.equal(y, y0)


def test_expanded_weights_refused_where_the_wide_kernel_does_not_run(gpu_device):
    w = torch.from_numpy(synth.weight(256, 192, seed=1)).to(gpu_device)
    qw, s16, zp = ck.quantize_w4a8_asym_weight(w, 64, 64)
    ex = ck.expand_w4_weight(qw.view(torch.uint8), zp.view(torch.uint8), _lib.ACT_I8, s16)
    x = synth.to_bf16_tensor(synth.activations(64, 192, seed=2), gpu_device)
    qa, sa = ops.rotate_quantize(x, 64, 8)
    # K = 192: three scale columns per row, not the pairs the wide kernel loads
    with pytest.raises(_lib.MQError, match="wide kernel only"):
        ops.gemm_w4_group(qa, sa, ex, s16, None, None, 256)
    qw, s16, zp = _group_weights(256, 256, True, gpu_device, seed=3)
    ex = ck.expand_w4_weight(qw.view(torch.uint8), zp.view(torch.uint8), _lib.ACT_I8, s16)
    x = synth.to_bf16_tensor(synth.activations(3, 256, seed=4), gpu_device)
    qa, sa = ops.rotate_quantize(x, 256, 8)
    with pytest.raises(_lib.MQError, match="wide kernel only"):   # M <= 4: the GEMV reads packed bytes
        ops.gemm_w4_group(qa, sa, ex, s16, None, None, 256)
    with pytest.raises(ValueError, match="do not serve act_mode"):
        ops.gemm_w4_group(qa, sa, ex, s16, None, None, 256, act_mode=_lib.ACT_X16ALT)


def _packed_only(fn):
    old = ops.EXPAND_W4
    ops.EXPAND_W4 = False
    try:
        return fn()
    finally:
        ops.EXPAND_W4 = old


@pytest.mark.parametrize("m", [1, 4, 5, 300, 4096])
def test_linears_run_on_the_expansion(gpu_device, m):
    """w4a8_int8_linear, convrot_w4a4_linear (group and shipped row scales): the same bits with the
    cached expansion (group scales above 128 rows, row scales above 4) as on the packed weights,
    one expansion per weight and layout."""
    print(f"[expand] linears M={m}", flush=True)
    assert ops.EXPAND_W4
    k, n = 3072, 1536
    x = synth.to_bf16_tensor(synth.activations(m, k, seed=m + 1), gpu_device)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(gpu_device)
    qd, s16, zp = ck.quantize_w4a8_asym_weight(torch.from_numpy(synth.weight(n, k, seed=5)).to(gpu_device), 64, 256)
    qg, sg = ck.quantize_w4a4_group_weight(torch.from_numpy(synth.weight(n, k, seed=6)).to(gpu_device), 64, 64)
    qr, sr = ck.quantize_convrot_w4a4_weight(torch.from_numpy(synth.weight(n, k, seed=7)).to(gpu_device), 256)
    calls = [
        lambda: ck.w4a8_int8_linear(x, qd, s16, None, None, zp, bias, 64, 256, torch.bfloat16),
        lambda: ck.convrot_w4a4_linear(x, qg, sg, bias, convrot_groupsize=64),
        lambda: ck.convrot_w4a4_linear(x, qr, sr, bias, convrot_groupsize=256),
    ]
    ops._EXPANDED.clear()
    ys = [c() for c in calls]
    cached = sum(len(v) for v in ops._EXPANDED.values())
    ys2 = [c() for c in calls]            # second calls: the cached expansions, no new ones
    want = (2 if m > ops.FEW_ROWS else 0) + (1 if m > ops.GEMV_ROWS else 0)
    assert sum(len(v) for v in ops._EXPANDED.values()) == cached == want
    y0 = [_packed_only(c) for c in calls]
    torch.cuda.synchronize()
    for a, b, c in zip(ys, ys2, y0):
        assert torch.equal(a, b) and torch.equal(a, c)


def test_expansion_follows_weight_updates(gpu_device):
    """An in-place update of the packed weight (its version changes) makes a new expansion."""
    k, n, m = 1024, 256, 200
    x = synth.to_bf16_tensor(synth.activations(m, k, seed=9), gpu_device)
    qd, s16, zp = ck.quantize_w4a8_asym_weight(torch.from_numpy(synth.weight(n, k, seed=10)).to(gpu_device), 64, 256)
    y1 = ck.w4a8_int8_linear(x, qd, s16, None, None, zp, None, 64, 256, torch.bfloat16)
    qd2, _, _ = ck.quantize_w4a8_asym_weight(torch.from_numpy(synth.weight(n, k, seed=11)).to(gpu_device), 64, 256)
    qd.copy_(qd2)
    y2 = ck.w4a8_int8_linear(x, qd, s16, None, None, zp, None, 64, 256, torch.bfloat16)
    y3 = _packed_only(lambda: ck.w4a8_int8_linear(x, qd, s16, None, None, zp, None, 64, 256, torch.bfloat16))
    torch.cuda.synchronize()
    assert not torch.equal(y1, y2) and torch.equal(y2, y3)
