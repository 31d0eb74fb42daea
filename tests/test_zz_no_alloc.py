"""mq_linear_w4_group_noalloc, the whole W4 group linear that allocates nothing (its codes, scales
and split-K partials live in the library's fixed per-device scratch array), against the ordinary
entry point mq_linear_w4_group with a caller workspace: bit-exact on two calls in a row, the
second with a smaller input, called through the C ABI; the trailing-rows product with the SwiGLU
prologue through the scratch; device memory unchanged across a call; and a shape whose split-K
partials do not fit beside its codes (then the product runs unsplit: same codes and int32
partials, fp32 group sums associated differently, both outputs within the oracle's tolerance)."""
import numpy as np
import pytest
import torch

import kitchen_amd as ck
from kitchen_amd import _lib, synth

SCRATCH_BYTES = _lib.NOALLOC_SCRATCH_BYTES


def _noalloc():
    return _lib.load().mq_linear_w4_group_noalloc


def _args(x, qd, s16, zp, bias, y, act_bits, swiglu=0):
    m, k = x.shape
    k = k // 2 if swiglu else k
    n = qd.shape[0]
    return [x.data_ptr(), _lib.dtype_code(x.dtype), x.stride(0), 256, act_bits, swiglu, qd.data_ptr(), qd.stride(0),
            s16.data_ptr(), s16.stride(0), _lib.ptr(zp), 0 if zp is None else zp.stride(0), _lib.ptr(bias),
            _lib.DT_BF16 if bias is None else _lib.dtype_code(bias.dtype), y.data_ptr(), _lib.dtype_code(y.dtype),
            y.stride(0), m, n, k]


def _reference(x, qd, s16, zp, bias, y, act_bits, swiglu=0):
    m, k = x.shape
    k = k // 2 if swiglu else k
    n = qd.shape[0]
    work = torch.empty(_lib.load().mq_linear_workspace_bytes(m, n, k), dtype=torch.uint8, device=x.device)
    _lib.call("mq_linear_w4_group", *_args(x, qd, s16, zp, bias, y, act_bits, swiglu), work.data_ptr(),
              work.numel(), _lib.stream_of(x))
    return work


def _w4a8_weight(n, k, dev, seed=1):
    w = torch.from_numpy(synth.weight(n, k, seed=seed)).to(dev)
    qd, s16, zp = ck.quantize_w4a8_asym_weight(w, 64, 256)
    return qd.view(torch.uint8), s16, zp.view(torch.uint8)


@pytest.mark.gpu
@pytest.mark.parametrize("act_bits", [8, 4])
def test_noalloc_equals_workspace_entry_point(gpu_device, act_bits):
    k, n = 3072, 3072
    fn = _noalloc()
    w = torch.from_numpy(synth.weight(n, k, seed=1)).to(gpu_device)
    if act_bits == 8:
        qd, s16, zp = ck.quantize_w4a8_asym_weight(w, 64, 256)
        qd, zp = qd.view(torch.uint8), zp.view(torch.uint8)
    else:
        qd, s16 = ck.quantize_w4a4_group_weight(w, 64, 256)
        qd, zp = qd.view(torch.uint8), None
    bias = torch.randn(n, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(gpu_device)
    # M = 256 runs the split-K path through the scratch's partials region; M = 64 (smaller, second)
    # the 128-tile kernel with only codes and scales in the scratch; M = 1 the one-launch GEMV that
    # quantizes its row itself (the scratch is not written)
    for m in (256, 64, 1):
        print(f"[noalloc] act_bits={act_bits} M={m} N={n} K={k}", flush=True)
        x = synth.to_bf16_tensor(synth.activations(m, k, seed=m), gpu_device)
        y0 = torch.empty((m, n), dtype=torch.bfloat16, device=gpu_device)
        y1 = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=gpu_device)
        work = _reference(x, qd, s16, zp, bias, y0, act_bits)
        rc = fn(*_args(x, qd, s16, zp, bias, y1, act_bits), _lib.stream_of(x))
        assert rc == 0, _lib.load().mq_last_error().decode()
        torch.cuda.synchronize()
        assert torch.equal(y0, y1)
        del work


@pytest.mark.gpu
def test_noalloc_trailing_rows_with_swiglu_prologue(gpu_device):
    # M = 4352 against N = 12288: the last 256 rows run as their own product (trailing rows) on the
    # 16-row code tiles, and the activation is the SwiGLU prologue of a [gate | up] input
    m, n, k = 4352, 12288, 3072
    print(f"[noalloc] trailing rows + swiglu M={m} N={n} K={k}", flush=True)
    qd, s16, zp = _w4a8_weight(n, k, gpu_device)
    g = torch.Generator(device=gpu_device).manual_seed(3)
    h = (torch.randn(m, 2 * k, generator=g, device=gpu_device) * 2).to(torch.bfloat16)
    bias = torch.randn(n, generator=g, device=gpu_device).to(torch.bfloat16)
    y0 = torch.empty((m, n), dtype=torch.bfloat16, device=gpu_device)
    y1 = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=gpu_device)
    work = _reference(h, qd, s16, zp, bias, y0, 8, swiglu=_lib.SWIGLU_FUSED)
    rc = _noalloc()(*_args(h, qd, s16, zp, bias, y1, 8, swiglu=_lib.SWIGLU_FUSED), _lib.stream_of(h))
    assert rc == 0, _lib.load().mq_last_error().decode()
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)
    # the call itself takes no device memory: free memory is unchanged across a repeat call
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info(gpu_device)[0]
    rc = _noalloc()(*_args(h, qd, s16, zp, bias, y1, 8, swiglu=_lib.SWIGLU_FUSED), _lib.stream_of(h))
    torch.cuda.synchronize()
    assert rc == 0 and torch.cuda.mem_get_info(gpu_device)[0] == free0
    assert torch.equal(y0, y1)
    del work


@pytest.mark.gpu
def test_noalloc_with_expanded_weights(gpu_device):
    # the weights' int8 expansion (act_bits | MQ_W4_EXPANDED) through the scratch: the workspace
    # entry's bits, and those of the packed weights (the wide kernel runs both at M = 300)
    m, n, k = 300, 1536, 3072
    print(f"[noalloc] expanded weights M={m} N={n} K={k}", flush=True)
    qd, s16, zp = _w4a8_weight(n, k, gpu_device, seed=4)
    ex = ck.expand_w4_weight(qd, zp, _lib.ACT_I8, s16)
    x = synth.to_bf16_tensor(synth.activations(m, k, seed=5), gpu_device)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).to(gpu_device)
    y0, y1, y2 = (torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=gpu_device) for _ in range(3))
    work = _reference(x, qd, s16, zp, bias, y0, 8)
    args = _args(x, qd, s16, zp, bias, y1, 8 | _lib.W4_EXPANDED)
    args[6], args[7] = ex.tiles.data_ptr(), k
    rc = _noalloc()(*args, _lib.stream_of(x))
    assert rc == 0, _lib.load().mq_last_error().decode()
    args = _args(x, qd, s16, zp, bias, y2, 8 | _lib.W4_EXPANDED)
    args[6], args[7] = ex.tiles.data_ptr(), k
    w2 = torch.empty(_lib.load().mq_linear_workspace_bytes(m, n, k), dtype=torch.uint8, device=gpu_device)
    _lib.call("mq_linear_w4_group", *args, w2.data_ptr(), w2.numel(), _lib.stream_of(x))
    torch.cuda.synchronize()
    assert torch.equal(y0, y1) and torch.equal(y1, y2)
    del work, w2


@pytest.mark.gpu
def test_noalloc_when_partials_do_not_fit(gpu_device):
    # codes and scales (57.4 MB) fit the scratch; whether the split-K partials fit beside them
    # decides whether the result is the workspace entry's bit for bit. Unsplit, the same int32
    # partials are summed in another fp32 order: both outputs are then checked against the oracle
    from oracle import gemm, linear, quant

    m, n, k = 3500, 512, 16384
    need = _lib.load().mq_linear_workspace_bytes(m, n, k)
    print(f"[noalloc] M={m} N={n} K={k}: workspace {need} bytes, scratch {SCRATCH_BYTES}", flush=True)
    w = synth.weight(n, k, seed=4)
    qd, s16, zp = ck.quantize_w4a8_asym_weight(torch.from_numpy(w).to(gpu_device), 64, 256)
    qd, zp = qd.view(torch.uint8), zp.view(torch.uint8)
    xb = synth.activations(m, k, seed=5)
    x = synth.to_bf16_tensor(xb, gpu_device)
    y0 = torch.empty((m, n), dtype=torch.bfloat16, device=gpu_device)
    y1 = torch.empty((m, n), dtype=torch.bfloat16, device=gpu_device)
    work = _reference(x, qd, s16, zp, None, y0, 8)
    rc = _noalloc()(*_args(x, qd, s16, zp, None, y1, 8), _lib.stream_of(x))
    assert rc == 0, _lib.load().mq_last_error().decode()
    torch.cuda.synchronize()
    if need <= SCRATCH_BYTES:
        assert torch.equal(y0, y1)
    else:
        rows = np.r_[0:32, m - 32:m]
        q0, s0, z0 = quant.quant_weight_u4_asym(linear.rotate_weight(w, 256), 64)
        ref = linear.w4a8_asym_linear(synth.bf16_bits_to_f32(xb[rows]), q0, s0, z0, None, 256, 64)
        for y in (y0, y1):
            assert gemm.rel_l2(ref.y, y.float().cpu().numpy()[rows]) < 4e-3
        a, b = y0.float(), y1.float()
        assert (torch.linalg.vector_norm(a - b) / torch.linalg.vector_norm(a)).item() < 4e-3
    del work


def test_noalloc_rejects_inputs_beyond_the_scratch():
    # codes [M, K] and scales [M] above the fixed scratch: refused before any HIP call (CPU only)
    fn = _noalloc()
    m, k, n = 8192, 16384, 64            # 128 MiB of codes
    assert m * k > SCRATCH_BYTES
    a = 1 << 20                          # never dereferenced: the size check fails first
    rc = fn(a, 0, k, 256, 8, 0, a, k // 2, a, k // 64, None, 0, None, 0, a, 0, n, m, n, k, None)
    assert rc == -1
    assert "scratch" in _lib.load().mq_last_error().decode()
