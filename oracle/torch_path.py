"""The reference's CPU torch path for the W4A8 linear, timed as the CPU baseline of bench.py.

It restates, with torch on the host cores, what the reference's torch code computes for this path:
the rotation as x.reshape(M, K/b, b) @ H_b in fp32 (experiments/qwen21-kernel/node/__init__.py:92,
g64_quant_test.py:63-64), the per-token int8 quantizer of tools/activation_balance.py:65-71, and
the GEMM with per-group weight scales as a dequantized fp32 matmul (g64_bench6.py:50-68 form:
per-group scales applied to the weight, row scales and bias after). The weight is dequantized
once, outside the timed region, as a resident weight would be.

Used only by bench.py's cpu_baseline leg; never by the product.
"""
from __future__ import annotations

import time

import numpy as np
import torch

from .hadamard import hadamard


class W4A8CpuLinear:
    def __init__(self, q_codes: np.ndarray, s16: np.ndarray, z: np.ndarray, bias, block: int = 256, group: int = 64):
        n, k = q_codes.shape
        wq = q_codes.astype(np.float32).reshape(n, k // group, group) - z.astype(np.float32)[..., None]
        w = wq * s16.astype(np.float32)[..., None]
        self.w_t = torch.from_numpy(w.reshape(n, k)).t().contiguous()
        self.h = torch.from_numpy(hadamard(block).astype(np.float32))
        self.block = block
        self.bias = None if bias is None else torch.as_tensor(bias, dtype=torch.float32)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        m, k = x.shape
        xr = (x.float().reshape(m, k // self.block, self.block) @ self.h).reshape(m, k)
        s = (xr.abs().amax(dim=1, keepdim=True) / 127).clamp(min=1e-10)
        qa = (xr / s).round().clamp(-127, 127)
        y = (qa @ self.w_t) * s
        if self.bias is not None:
            y = y + self.bias
        return y.to(torch.bfloat16)


def time_cpu(fn, x, runs: int = 5, min_seconds: float = 0.0) -> tuple[float, int]:
    """(median seconds per call, calls timed): at least `runs` calls after one warm-up, and more
    until `min_seconds` of timed work have run."""
    fn(x)
    ts = []
    total = 0.0
    while len(ts) < runs or total < min_seconds:
        t0 = time.perf_counter()
        fn(x)
        ts.append(time.perf_counter() - t0)
        total += ts[-1]
    ts.sort()
    return ts[len(ts) // 2], len(ts)
