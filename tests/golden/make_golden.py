"""Write the golden fixtures of the quantized-linear path from the CPU oracle.

    python tests/golden/make_golden.py        # -> tests/golden/linear_small.npz

Small, seeded cases: rotate + quantize (every Hadamard block and bit width, with a zero row, exact
ties and an outlier row), the configs' weight quantizers, exact int32 group partials and the fp64
linear outputs. The fixture is data only (numpy arrays, no pickles); the oracle that produced it
is restated from the reference in oracle/ (see its module docstrings for the file:line anchors).
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from oracle import SPEC_VERSION, gemm, linear, quant  # noqa: E402

OUT = os.path.join(HERE, "linear_small.npz")
M, K, N = 8, 256, 16
ROT_CASES = [(0, 8), (16, 4), (64, 4), (64, 8), (256, 8), (256, 4)]


def inputs():
    rng = np.random.default_rng(20261201)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[:, rng.choice(K, 3, replace=False)] *= 20.0           # outlier channels
    x[1] = 0.0                                                # zero row -> s = 1e-10, q = 0
    x[2, :] = 0.0
    x[2, :8] = [127.0, 2.5, -3.5, 0.5, 1.5, -2.5, 126.5, -0.5]  # exact ties with hblock 0
    x[5] *= 50.0                                              # token spike
    xb = quant.f32_to_bf16_bits(x)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w[3, :64] = 0.0                                           # all-zero group -> s = z = q = 0
    w = quant.bf16_bits_to_f32(quant.f32_to_bf16_bits(w))
    bias = quant.bf16_bits_to_f32(quant.f32_to_bf16_bits(rng.standard_normal(N).astype(np.float32) * 0.1))
    return xb, w, bias


def build() -> dict:
    xb, w, bias = inputs()
    xf = quant.bf16_bits_to_f32(xb)
    out = {"spec": np.array(SPEC_VERSION), "x_bf16": xb, "w": w, "bias": bias}
    for hb, bits in ROT_CASES:
        q, s = quant.rotquant(xf, hb, bits) if hb else quant.quant_per_token(xf, 127 if bits == 8 else 7)
        out[f"rq_h{hb}_b{bits}_q"] = q
        out[f"rq_h{hb}_b{bits}_s"] = s
    # configs' W4A8 weight: rotate by H256, uint4 asym per group of 64
    q, s16, z = quant.quant_weight_u4_asym(linear.rotate_weight(w, 256), 64)
    out["w4a8_q_packed"], out["w4a8_s16"], out["w4a8_z_packed"] = quant.pack_u4(q), s16, quant.pack_u4(z)
    res = linear.w4a8_asym_linear(xf, q, s16, z, bias, 256, 64)
    out["w4a8_partials"], out["w4a8_y"] = res.partials.astype(np.int32), res.y
    # configs' W4A4 weight: rotate by H64, int4 sym per group of 64, int4 activations
    q4, s4 = quant.quant_weight_i4_sym_group(linear.rotate_weight(w, 64), 64)
    out["w4a4_q_packed"], out["w4a4_s16"] = quant.pack_i4(q4), s4
    res4 = linear.w4a4_group_linear(xf, q4, s4, bias, 64, 64)
    out["w4a4_partials"], out["w4a4_y"] = res4.partials.astype(np.int32), res4.y
    return out


if __name__ == "__main__":
    data = build()
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(data)} arrays)")
