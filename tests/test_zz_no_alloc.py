"""mq_linear_w4_group_noalloc, the whole W4 group linear that allocates nothing (its codes, scales
and split-K partials live in the library's fixed per-device scratch array), against the ordinary
entry point mq_linear_w4_group with a caller workspace: bit-exact on two calls in a row, the
second with a smaller input, called through the C ABI."""
import numpy as np
import pytest
import torch

import kitchen_amd as ck
from kitchen_amd import _lib, synth

SCRATCH_BYTES = _lib.NOALLOC_SCRATCH_BYTES


def _noalloc():
    return _lib.load().mq_linear_w4_group_noalloc


def _args(x, qd, s16, zp, bias, y, act_bits):
    m, k = x.shape
    n = qd.shape[0]
    return [x.data_ptr(), _lib.dtype_code(x.dtype), x.stride(0), 256, act_bits, 0, qd.data_ptr(), qd.stride(0),
            s16.data_ptr(), s16.stride(0), _lib.ptr(zp), 0 if zp is None else zp.stride(0), _lib.ptr(bias),
            _lib.DT_BF16 if bias is None else _lib.dtype_code(bias.dtype), y.data_ptr(), _lib.dtype_code(y.dtype),
            y.stride(0), m, n, k]


def _reference(x, qd, s16, zp, bias, y, act_bits):
    m, k = x.shape
    n = qd.shape[0]
    work = torch.empty(_lib.load().mq_linear_workspace_bytes(m, n, k), dtype=torch.uint8, device=x.device)
    _lib.call("mq_linear_w4_group", *_args(x, qd, s16, zp, bias, y, act_bits), work.data_ptr(), work.numel(),
              _lib.stream_of(x))
    return work


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
    # the 128-tile kernel with only codes and scales in the scratch
    for m in (256, 64):
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


def test_noalloc_rejects_inputs_beyond_the_scratch():
    # codes [M, K] and scales [M] above the fixed scratch: refused before any HIP call (CPU only)
    fn = _noalloc()
    m, k, n = 8192, 16384, 64            # 128 MiB of codes
    assert m * k > SCRATCH_BYTES
    a = 1 << 20                          # never dereferenced: the size check fails first
    rc = fn(a, 0, k, 256, 8, 0, a, k // 2, a, k // 64, None, 0, None, 0, a, 0, n, m, n, k, None)
    assert rc == -1
    assert "scratch" in _lib.load().mq_last_error().decode()
