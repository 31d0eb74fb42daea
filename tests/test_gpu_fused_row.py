"""One-row whole linears (M = 1, K <= 4096): the GEMV rotates and quantizes the row in its own
prologue (one launch). The output must equal, bit for bit, the two-launch path on the same
operands: mq_rotquant's codes and scale fed to the GEMM entry point. Covered: every activation
layout the whole-linear entries use (int8, int4 one per byte, the group GEMM's x16 layout), the
three input types, every Hadamard block, uint4 / int4 group weights and int8 / int4 row weights,
ragged N, K up to the fused limit and past it, and rows that pin the quantizer's edge cases (a zero
row, one dominant value, halves that land on rounding ties)."""
import pytest
import torch

from kitchen_amd import _lib, ops

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _row(k, dev, dtype, kind, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(1, k, generator=g)
    if kind == "zero":
        x.zero_()
    elif kind == "spike":
        x[0, k // 3] = 3000.0
    elif kind == "ties":
        # values on a grid of halves of the scale step: many products land next to half-integers
        x = (torch.randint(-254, 255, (1, k), generator=g).float() * 0.5)
    return x.to(dtype).to(dev)


def _group_weights(n, k, dev, asym, seed):
    g = torch.Generator().manual_seed(seed)
    qw = torch.randint(0, 256, (n, k // 2), generator=g, dtype=torch.uint8).to(dev)
    s16 = (torch.rand(n, k // 64, generator=g) * 0.004 + 0.002).to(torch.float16).to(dev)
    zp = torch.randint(0, 256, (n, (k // 64 + 1) // 2), generator=g, dtype=torch.uint8).to(dev) if asym else None
    bias = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16).to(dev)
    return qw, s16, zp, bias


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("hblock", [0, 16, 64, 256])
@pytest.mark.parametrize("act_bits", [8, 4])
@pytest.mark.parametrize("asym", [True, False])
def test_group_row_equals_two_launches(gpu_device, dtype, hblock, act_bits, asym):
    n, k = 1000, 3072
    print(f"[fused-row] group dtype={dtype} hblock={hblock} act_bits={act_bits} asym={asym}", flush=True)
    qw, s16, zp, bias = _group_weights(n, k, gpu_device, asym, seed=hblock + act_bits)
    layout = _lib.Q_X16ALT if act_bits == 4 else _lib.Q_BYTES
    act_mode = _lib.ACT_X16ALT if act_bits == 4 else _lib.ACT_I8
    for kind in ("rand", "spike", "zero", "ties"):
        x = _row(k, gpu_device, dtype, kind, seed=7)
        y1 = ops._linear_w4_group(x, 0, hblock, act_bits, qw, s16, zp, bias, n, k, torch.bfloat16)
        qa, sa = ops.rotate_quantize(x, hblock, act_bits, layout)
        y2 = ops.gemm_w4_group(qa, sa, qw, s16, zp, bias, n, act_mode=act_mode)
        torch.cuda.synchronize()
        assert torch.equal(y1, y2), f"row {kind}: fused and two-launch outputs differ"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("hblock", [0, 16, 64, 256])
@pytest.mark.parametrize("act_bits", [8, 4])
@pytest.mark.parametrize("wbits,tiled", [(8, False), (8, True), (4, False)])
def test_rowscale_row_equals_two_launches(gpu_device, dtype, hblock, act_bits, wbits, tiled):
    n, k = 1000, 3072
    print(f"[fused-row] rowscale dtype={dtype} hblock={hblock} act_bits={act_bits} wbits={wbits} tiled={tiled}",
          flush=True)
    g = torch.Generator().manual_seed(11)
    if wbits == 8:
        qw = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(gpu_device)
        if tiled:
            qw = ops.tile_int8_weight(qw)
    else:
        qw = torch.randint(0, 256, (n, k // 2), generator=g, dtype=torch.uint8).to(gpu_device)
    ws = (torch.rand(n, generator=g) * 0.01 + 0.001).to(gpu_device)
    bias = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16).to(gpu_device)
    for kind in ("rand", "spike", "zero", "ties"):
        x = _row(k, gpu_device, dtype, kind, seed=3)
        y1 = ops._linear_rowscale(x, 0, hblock, act_bits, qw, wbits, ws, bias, n, k, torch.bfloat16)
        qa, sa = ops.rotate_quantize(x, hblock, act_bits, _lib.Q_BYTES)
        y2 = ops.gemm_rowscale(qa, sa, qw, ws, bias, n, wbits)
        torch.cuda.synchronize()
        assert torch.equal(y1, y2), f"row {kind}: fused and two-launch outputs differ"


@pytest.mark.parametrize("k", [256, 3136, 4096, 4160])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_row_lengths_and_outputs(gpu_device, k, out_dtype):
    """K from one Hadamard block to the fused limit (4096) and past it (4160: the two-launch path),
    with a ragged N; every output type."""
    n = 333
    print(f"[fused-row] K={k} out={out_dtype}", flush=True)
    qw, s16, zp, bias = _group_weights(n, k, gpu_device, True, seed=k)
    x = _row(k, gpu_device, torch.bfloat16, "rand", seed=k)
    y1 = ops._linear_w4_group(x, 0, 64, 8, qw, s16, zp, bias, n, k, out_dtype)
    qa, sa = ops.rotate_quantize(x, 64, 8)
    y2 = ops.gemm_w4_group(qa, sa, qw, s16, zp, bias, n, out_dtype=out_dtype)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)


def test_public_ops_one_token(gpu_device):
    """The drop-in ops on one token ([1, 1, K], as the adaLN modulation linear calls them) equal the
    same ops on that token inside a two-token batch (the GEMV without the fused prologue)."""
    n, k = 1536, 3072
    print("[fused-row] public ops, one token", flush=True)
    qw, s16, zp, bias = _group_weights(n, k, gpu_device, True, seed=5)
    x2 = torch.randn(2, k, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16).to(gpu_device)
    y1 = ops.w4a8_int8_linear(x2[:1].reshape(1, 1, k), qw, s16, None, None, zp, bias)
    y2 = ops.w4a8_int8_linear(x2, qw, s16, None, None, zp, bias)
    torch.cuda.synchronize()
    assert y1.shape == (1, 1, n)
    assert torch.equal(y1.reshape(1, n), y2[:1])


@pytest.mark.parametrize("bias_kind", ["none", "f32", "f16"])
def test_row_bias_types(gpu_device, bias_kind):
    """No bias, and biases of other floating-point types than the output's."""
    n, k = 777, 3072
    print(f"[fused-row] bias {bias_kind}", flush=True)
    qw, s16, zp, bias = _group_weights(n, k, gpu_device, True, seed=21)
    b = None if bias_kind == "none" else bias.to(torch.float32 if bias_kind == "f32" else torch.float16)
    x = _row(k, gpu_device, torch.float16, "rand", seed=21)
    y1 = ops._linear_w4_group(x, 0, 256, 8, qw, s16, zp, b, n, k, torch.bfloat16)
    qa, sa = ops.rotate_quantize(x, 256, 8)
    y2 = ops.gemm_w4_group(qa, sa, qw, s16, zp, b, n)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
