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


# --------------------------------------------------------------------------- config 4: linear stack

MMDIT_HIDDEN = 3072
MMDIT_LINEARS = (  # (name, K, N) of the 7 linear types of one stream of one dual-stream block
    ("q", 3072, 3072), ("k", 3072, 3072), ("v", 3072, 3072), ("out", 3072, 3072),
    ("mlp_up", 3072, 12288), ("mlp_down", 12288, 3072), ("mod", 3072, 18432))
MMDIT_TOKENS = {"image": 4096, "text": 256}


def w4a4_count(linears: int, w4a4_frac: float = 0.35) -> int:
    """W4A4 linears of a stack of `linears`: w4a4_frac of them, rounded half up (294 of 840)."""
    return int(linears * w4a4_frac + 0.5)


def mmdit_linear_stack(blocks: int = 60, w4a4_frac: float = 0.35, seed: int = 4, device="cuda"):
    """The linear stack of BASELINE config 4: `blocks` dual-stream MMDiT blocks (hidden 3072,
    MLP ratio 4), 7 linear types per stream (q, k, v, out, mlp up, mlp down, adaLN modulation at
    M = 1), image M = 4096 and text M = 256. Exactly round(w4a4_frac * linears) of the linears
    (294 of 840 at the defaults) go on W4A4 (int4 per-token activations after H_64, int4
    symmetric group-64 fp16-scale weights), placed by a seeded permutation; the rest on W8A8
    (int8 per-row weights, int8 per-token activations after H_256). Weights are random-init directly in the quantized domain (random codes,
    random positive scales), which is what quantizing random-init weights produces.

    Returns a list of dicts: {"name", "stream", "M", "K", "N", "fmt", "tensors"}."""
    from . import ops

    gen = torch.Generator(device="cpu").manual_seed(seed)
    total = blocks * 2 * len(MMDIT_LINEARS)
    pick = torch.zeros(total, dtype=torch.bool)
    pick[torch.randperm(total, generator=gen)[:w4a4_count(total, w4a4_frac)]] = True
    dgen = torch.Generator(device=device).manual_seed(seed + 1)
    layers = []
    i = 0
    for b in range(blocks):
        for stream, m_tok in MMDIT_TOKENS.items():
            for name, k, n in MMDIT_LINEARS:
                m = 1 if name == "mod" else m_tok
                bias = (torch.randn(n, generator=dgen, device=device) * 0.02).to(torch.bfloat16)
                if bool(pick[i]):
                    q = torch.randint(-128, 128, (n, k // 2), generator=dgen, device=device, dtype=torch.int8)
                    s = (torch.rand(n, k // 64, generator=dgen, device=device) * 0.004 + 0.004).to(torch.float16)
                    tensors = {"qweight": q, "wscales": s, "bias": bias}
                    fmt = "w4a4"
                else:
                    w = torch.randint(-127, 128, (n, k), generator=dgen, device=device, dtype=torch.int8)
                    s = torch.rand(n, 1, generator=dgen, device=device) * 2e-4 + 3e-4
                    # held in the 16-row tile layout a loader prepares (ops.tile_int8_weight)
                    tensors = {"weight": ops.tile_int8_weight(w), "weight_scale": s, "bias": bias}
                    fmt = "w8a8"
                layers.append({"name": f"blocks.{b}.{stream}.{name}", "stream": stream, "M": m, "K": k, "N": n,
                               "fmt": fmt, "tensors": tensors})
                i += 1
    return layers


def stack_ops(layers) -> float:
    """Integer operations of one pass over the stack (2 M N K per linear)."""
    return float(sum(2 * l["M"] * l["N"] * l["K"] for l in layers))


def stack_activations(device="cuda", seed: int = 5) -> dict:
    """bf16 input buffers of the stack, one per (M, K): resident inputs for every linear."""
    gen = torch.Generator(device=device).manual_seed(seed)
    out = {}
    for m in (*MMDIT_TOKENS.values(), 1):
        for k in (MMDIT_HIDDEN, 4 * MMDIT_HIDDEN):
            out[(m, k)] = torch.randn(m, k, generator=gen, device=device).to(torch.bfloat16)
    return out


def stack_pass(layers, acts, side=None):
    """One pass over the stack; returns the outputs in layer order. side=None: every linear in
    order on the current stream. With a side stream, the two token streams of each MMDiT block run
    concurrently (text linears on `side`, image linears on the current stream), joined where a
    block joins them: after mod / q / k / v (the joint attention reads both streams' q, k, v) and
    after out / mlp_up / mlp_down (the block's end). The text linears are small (M = 256) and
    latency-bound, so they fill compute units the image GEMMs leave between tiles."""
    outs = [None] * len(layers)
    if side is None:
        for i, layer in enumerate(layers):
            outs[i] = stack_layer(layer, acts[(layer["M"], layer["K"])])
        return outs
    main = torch.cuda.current_stream()
    blocks: dict = {}
    for i, layer in enumerate(layers):
        blocks.setdefault(layer["name"].split(".")[1], []).append(i)
    for idx in blocks.values():
        for phase in (("mod", "q", "k", "v"), ("out", "mlp_up", "mlp_down")):
            side.wait_stream(main)
            for i in idx:
                layer = layers[i]
                if layer["name"].rsplit(".", 1)[1] not in phase:
                    continue
                x = acts[(layer["M"], layer["K"])]
                if layer["stream"] == "text":
                    with torch.cuda.stream(side):
                        outs[i] = stack_layer(layer, x)
                else:
                    outs[i] = stack_layer(layer, x)
            main.wait_stream(side)
    return outs


def stack_layer(layer, x):
    """One linear of the stack through the drop-in ops."""
    from . import ops

    t = layer["tensors"]
    if layer["fmt"] == "w4a4":
        return ops.convrot_w4a4_linear(x, t["qweight"], t["wscales"], t["bias"], convrot_groupsize=64,
                                       quant_group_size=64, linear_dtype="int4")
    return ops.int8_linear(x, t["weight"], t["weight_scale"], t["bias"], torch.bfloat16, True, 256)
