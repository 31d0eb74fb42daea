"""Seeded synthetic DiT-shaped inputs of the benchmark configurations (numpy, CPU).

Activations: N(0, 1) with 1 % of K-channels scaled x20 (outlier channels) and, optionally, 0.1 %
of tokens scaled x50 (spikes); weights: N(0, 0.02). Values are rounded to bf16 and returned as
uint16 bit patterns (`to_bf16_tensor` turns them into a torch bfloat16 tensor).
"""
from __future__ import annotations

import numpy as np
import torch


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def activations(m: int, k: int, seed: int = 0, outlier_frac: float = 0.01, outlier_scale: float = 20.0,
                spike_frac: float = 0.0, spike_scale: float = 50.0) -> np.ndarray:
    """bf16 bit patterns [m, k] of N(0,1) activations with outlier channels and token spikes."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k), dtype=np.float32)
    n_out = int(round(outlier_frac * k))
    if n_out:
        x[:, rng.choice(k, n_out, replace=False)] *= np.float32(outlier_scale)
    n_spk = int(round(spike_frac * m))
    if n_spk:
        x[rng.choice(m, n_spk, replace=False), :] *= np.float32(spike_scale)
    return f32_to_bf16_bits(x)


def weight(n: int, k: int, seed: int = 1, std: float = 0.02) -> np.ndarray:
    """float32 [n, k] weights rounded to bf16 values."""
    rng = np.random.default_rng(seed)
    return bf16_bits_to_f32(f32_to_bf16_bits(rng.standard_normal((n, k), dtype=np.float32) * np.float32(std)))


def to_bf16_tensor(bits: np.ndarray, device="cpu") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)
