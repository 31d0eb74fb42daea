"""Operand types at the boundary: fp16 / fp32 activations, the fp16 SwiGLU prologue, bias and
output types of every GEMM kernel, input_act="gelu_tanh", and the shipped W4A8 weight decoded once.

Bars: activation codes and scales bit-exact against the oracle on the same fp16 / fp32 values
(the reference quantizer takes bf16 or fp16 and rotates in fp32, g64_quant.cu:27-108,
swiglu_quant.cu:124-132); outputs of exact integer sums bit-exact against the same fp32 expression
rounded to the output type; one kernel's fp32, fp16 and bf16 outputs the roundings of one fp32
value; linears within 4e-3 rel-L2 of the oracle's fp64 result. Each case prints its name first."""
import numpy as np
import pytest
import torch

import kitchen_amd as ck
from kitchen_amd import _lib, ops, synth
from oracle import gemm, quant, swiglu

pytestmark = pytest.mark.gpu
F32 = np.float32


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _codes_check(q, s, q0, s0, packed):
    assert np.array_equal(s.view(np.uint32), s0.view(np.uint32)), "scales differ"
    if packed == _lib.Q_X16ALT:
        sign = np.where((np.arange(q0.shape[1]) // 64) % 2 == 1, -1, 1).astype(np.int16)
        assert np.array_equal(q.astype(np.int16), 16 * q0.astype(np.int16) * sign[None, :]), "x16alt codes differ"
    elif packed:
        assert np.array_equal(q, quant.pack_i4(q0)), "packed codes differ"
    else:
        assert np.array_equal(q, q0), f"{np.count_nonzero(q != q0)} codes differ"


MODES = [(8, False), (4, False), (4, True), (4, _lib.Q_X16ALT)]


@pytest.mark.parametrize("hblock", [0, 16, 64, 256])
@pytest.mark.parametrize("bits,packed", MODES)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_rotquant_config0_shape_f16_f32(gpu_device, dtype, hblock, bits, packed):
    # C0 activations [1024, 3072] (outlier channels x20) in fp16 / fp32: rotated from the exact
    # value, so the codes are the oracle's on the same values
    print(f"[dtypes] rotquant {dtype} C0 hblock={hblock} bits={bits} packed={packed}", flush=True)
    xf = synth.bf16_bits_to_f32(synth.activations(1024, 3072, seed=0))
    if dtype == "f16":
        xf = xf.astype(np.float16).astype(F32)
        x = _t(xf.astype(np.float16), gpu_device)
    else:
        xf = xf + np.random.default_rng(1).standard_normal(xf.shape).astype(F32) * F32(1e-3)   # not bf16 values
        x = _t(xf, gpu_device)
    q, s = ops.rotate_quantize(x, hblock, bits, packed)
    torch.cuda.synchronize()
    q0, s0 = quant.rotquant(xf, hblock, bits) if hblock else quant.quant_per_token(xf, 127 if bits == 8 else 7)
    _codes_check(q.cpu().numpy(), s.cpu().numpy(), q0, s0, packed)


def _f16_h(m, k, seed, gate_scale=3.0):
    rng = np.random.default_rng(seed)
    g = rng.standard_normal((m, k)).astype(F32) * gate_scale
    u = synth.bf16_bits_to_f32(synth.activations(m, k, seed=seed + 1))
    return np.concatenate([g, u], axis=1).astype(np.float16)


def test_swiglu_f16_every_gate_bitexact(gpu_device):
    # one nonzero column per row (hblock 0, K = 16): the row's scale max(|a| / 127, 1e-10) carries
    # the fp16 activation a = swiglu(g, u) itself; every finite fp16 gate, several up values
    bits = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
    g = bits.view(np.float16)
    g = g[np.isfinite(g)]
    rng = np.random.default_rng(0)
    for up in (1.0, -0.3125, 7.5, None):
        u = (rng.standard_normal(g.size) * 4).astype(np.float16) if up is None else np.full(g.size, up, np.float16)
        h = np.zeros((g.size, 32), np.float16)
        h[:, 0], h[:, 16] = g, u
        for mode in (_lib.SWIGLU_FUSED, _lib.SWIGLU_EAGER):
            print(f"[dtypes] swiglu f16 gate sweep up={up} mode={mode}", flush=True)
            q, s = ops.rotate_quantize(_t(h, gpu_device), 0, 8, False, swiglu=mode)
            torch.cuda.synchronize()
            act = swiglu.swiglu_f16_eager if mode == _lib.SWIGLU_EAGER else swiglu.swiglu_f16
            a = act(h[:, :16].astype(F32), h[:, 16:].astype(F32))
            # rows whose product overflows fp16 (inf) are compared too: scale +inf, codes 0
            q0, s0 = quant.quant_per_token(a, 127)
            _codes_check(q.cpu().numpy(), s.cpu().numpy(), q0, s0, False)


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("hblock,bits,packed", [(64, 4, True), (256, 8, False), (16, 4, 2)])
def test_swiglu_f16_product_overflow_rows(gpu_device, mode, hblock, bits, packed):
    # rows whose fp16 product silu(g) * u passes 65504 become inf in the input type; the rotation
    # spreads inf / NaN over that Hadamard block: the row is quantized with scale +inf and codes 0
    # (oracle.quant.quant_per_token), the other rows as usual
    print(f"[dtypes] swiglu f16 overflow mode={mode} hblock={hblock} bits={bits} packed={packed}", flush=True)
    h = _f16_h(64, 3072, seed=9)
    h[3, 100], h[3, 3072 + 100] = 300.0, 240.0          # 72000 -> inf
    h[10, 7], h[10, 3072 + 7] = 200.0, -400.0           # -80000 -> -inf
    q, s = ops.rotate_quantize(_t(h, gpu_device), hblock, bits, packed, swiglu=mode)
    torch.cuda.synchronize()
    with np.errstate(invalid="ignore", over="ignore"):
        q0, s0 = swiglu.swiglu_rotquant(h.astype(F32), hblock, bits, dtype="f16", eager=mode == 2)
    assert np.isinf(s0[[3, 10]]).all() and np.isfinite(np.delete(s0, [3, 10])).all()
    _codes_check(q.cpu().numpy(), s.cpu().numpy(), q0, s0, packed)


@pytest.mark.parametrize("hblock", [16, 64, 256])
@pytest.mark.parametrize("bits,packed", MODES)
def test_swiglu_f16_mlp_down_input(gpu_device, hblock, bits, packed):
    print(f"[dtypes] swiglu f16 C1-down hblock={hblock} bits={bits} packed={packed}", flush=True)
    h = _f16_h(256, 12288, seed=7)
    q, s = ops.rotate_quantize(_t(h, gpu_device), hblock, bits, packed, swiglu=True)
    torch.cuda.synchronize()
    q0, s0 = swiglu.swiglu_rotquant(h.astype(F32), hblock, bits, dtype="f16")
    _codes_check(q.cpu().numpy(), s.cpu().numpy(), q0, s0, packed)


def test_swiglu_fp32_pairs_are_formed_eagerly(gpu_device):
    # the fused prologue takes bf16 / fp16; an fp32 gate | up pair is formed by torch in fp32 first
    print("[dtypes] swiglu fp32 eager", flush=True)
    h = _t(_f16_h(64, 1024, seed=3).astype(F32), gpu_device)
    q, s = ops.rotate_quantize(h, 256, 8, False, swiglu=True)
    gate, up = h.chunk(2, dim=-1)
    q2, s2 = ops.rotate_quantize(torch.nn.functional.silu(gate) * up, 256, 8, False)
    torch.cuda.synchronize()
    assert torch.equal(q, q2) and torch.equal(s, s2)


OUT_TYPES = [torch.bfloat16, torch.float16, torch.float32]


def _round_to(y32: np.ndarray, dt) -> np.ndarray:
    if dt == torch.float32:
        return y32
    if dt == torch.float16:
        return y32.astype(np.float16).astype(F32)
    return synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(y32))


@pytest.mark.parametrize("m", [1, 3, 77, 256, 1000])
@pytest.mark.parametrize("bias_dtype", [None, torch.bfloat16, torch.float16, torch.float32])
def test_rowscale_output_types_exact(gpu_device, m, bias_dtype):
    # exact int32 sums, so every kernel's output is the fp32 expression ((acc * sa) * ws) + bias
    # rounded to the output type, bit for bit: M = 1 / 3 the few-row kernel, 77 the 128-tile
    # kernel, 256 the split-K wide kernel, 1000 the wide kernel
    n, k = 640, 3072
    rng = np.random.default_rng(m)
    qa = rng.integers(-127, 128, (m, k)).astype(np.int8)
    qw = rng.integers(-127, 128, (n, k)).astype(np.int8)
    sa = rng.uniform(0.001, 0.01, m).astype(F32)
    ws = rng.uniform(0.001, 0.01, n).astype(F32)
    bias = None
    bias_f = np.zeros(n, F32)
    if bias_dtype is not None:
        bias = torch.from_numpy(rng.standard_normal(n).astype(F32)).to(bias_dtype)
        bias_f = bias.float().numpy()
        bias = bias.to(gpu_device)
    acc = gemm.partials(qa, qw, k)[0].astype(F32)
    y32 = ((acc * sa[:, None]) * ws[None, :]) + bias_f[None, :]
    for dt in OUT_TYPES:
        print(f"[dtypes] rowscale M={m} bias={bias_dtype} out={dt}", flush=True)
        y = ops.gemm_rowscale(_t(qa, gpu_device), _t(sa, gpu_device), _t(qw, gpu_device), _t(ws, gpu_device), bias,
                              n, 8, out_dtype=dt)
        torch.cuda.synchronize()
        assert y.dtype == dt
        got = y.float().cpu().numpy()
        want = _round_to(y32, dt)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{np.count_nonzero(got != want)} differ"


@pytest.mark.parametrize("m", [2, 77, 256, 1000])
@pytest.mark.parametrize("act_mode", [_lib.ACT_I8, _lib.ACT_X16ALT])
def test_group_output_types_are_roundings_of_one_value(gpu_device, m, act_mode):
    # one group GEMM kernel's fp32, fp16 and bf16 outputs are the roundings of the same fp32 value
    n, k = 640, 3072
    rng = np.random.default_rng(10 * m + act_mode)
    if act_mode == _lib.ACT_I8:
        codes = rng.integers(-127, 128, (m, k)).astype(np.int8)
        stored = codes
        q = rng.integers(0, 16, (n, k)).astype(np.uint8)
        z = rng.integers(0, 16, (n, k // 64)).astype(np.uint8)
        qw_d, z_d, wq = _t(quant.pack_u4(q), gpu_device), _t(quant.pack_u4(z), gpu_device), gemm.zero_adjusted(q, z, 64)
    else:
        codes = rng.integers(-7, 8, (m, k)).astype(np.int8)
        sign = np.where((np.arange(k) // 64) % 2 == 1, -1, 1)
        stored = (16 * codes.astype(np.int16) * sign[None, :]).astype(np.int8)
        wq = rng.integers(-8, 8, (n, k)).astype(np.int8)
        qw_d, z_d = _t(quant.pack_i4(wq), gpu_device), None
    s16 = rng.uniform(1e-3, 4e-3, (n, k // 64)).astype(np.float16)
    sa = rng.uniform(0.001, 0.01, m).astype(F32)
    bias = torch.from_numpy(rng.standard_normal(n).astype(F32)).to(torch.float16)
    ys = {}
    for dt in OUT_TYPES:
        print(f"[dtypes] group M={m} act_mode={act_mode} out={dt}", flush=True)
        ys[dt] = ops.gemm_w4_group(_t(stored, gpu_device), _t(sa, gpu_device), qw_d, _t(s16, gpu_device), z_d,
                                   bias.to(gpu_device), n, act_mode=act_mode, out_dtype=dt)
    torch.cuda.synchronize()
    y32 = ys[torch.float32].cpu().numpy()
    for dt in (torch.float16, torch.bfloat16):
        got = ys[dt].float().cpu().numpy()
        assert np.array_equal(got.view(np.uint32), _round_to(y32, dt).view(np.uint32)), f"{dt} is not RN(fp32 out)"
    ref = gemm.epilogue_group(gemm.partials(codes, wq, 64), sa, s16.astype(np.float64), bias.float().numpy())
    assert gemm.rel_l2(ref, y32) < 2e-3


def _w4a8_ref(xf, qd, s16, zp, bias, hb):
    qa, sa = quant.rotquant(xf, hb, 8)
    q = quant.unpack_u4(qd.cpu().numpy()).astype(np.float64)
    z = quant.unpack_u4(zp.cpu().numpy())[:, : s16.shape[1]].astype(np.float64)
    wdq = (q.reshape(q.shape[0], -1, 64) - z[..., None]) * s16.cpu().numpy().astype(np.float64)[..., None]
    return (qa.astype(np.float64) * sa.astype(np.float64)[:, None]) @ wdq.reshape(q.shape[0], -1).T + bias


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_w4a8_linear_f16_f32_config0(gpu_device, dtype):
    # C0 through the drop-in op with fp16 / fp32 activations and outputs (out_dtype = x.dtype, as
    # the loader passes it) and a bias in the same type
    m, k, n = 1024, 3072, 3072
    print(f"[dtypes] w4a8 linear C0 {dtype}", flush=True)
    w = torch.from_numpy(synth.weight(n, k, seed=1)).to(gpu_device)
    qd, s16, zp = ck.quantize_w4a8_asym_weight(w, 64, 256)
    xf = synth.bf16_bits_to_f32(synth.activations(m, k, seed=0))
    if dtype == torch.float16:
        xf = xf.astype(np.float16).astype(F32)
    rng = np.random.default_rng(2)
    bias = torch.from_numpy(rng.standard_normal(n).astype(F32) * 0.1).to(dtype)
    x = _t(xf, gpu_device).to(dtype)
    y = ck.w4a8_int8_linear(x, qd, s16, None, None, zp, bias.to(gpu_device), 64, 256, dtype)
    qa, sa = ops.quantize_int8_rowwise_convrot(x, 256)
    torch.cuda.synchronize()
    assert y.dtype == dtype and y.shape == (m, n)
    q0, s0 = quant.rotquant(xf, 256, 8)
    assert np.array_equal(qa.cpu().numpy(), q0) and np.array_equal(sa.cpu().numpy(), s0)
    ref = _w4a8_ref(xf, qd, s16, zp, bias.double().numpy(), 256)
    err = gemm.rel_l2(ref, y.double().cpu().numpy())
    print(f"[dtypes] rel L2 {err:.2e}", flush=True)
    assert err < 4e-3


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_convrot_w4a4_linear_writes_x_dtype(gpu_device, dtype):
    m, k, n = 300, 3072, 1024
    print(f"[dtypes] w4a4 linear {dtype}", flush=True)
    qw, s16 = ck.quantize_w4a4_group_weight(torch.from_numpy(synth.weight(n, k, seed=5)).to(gpu_device), 64, 64)
    xf = synth.bf16_bits_to_f32(synth.activations(m, k, seed=6, spike_frac=0.001))
    if dtype == torch.float16:
        xf = xf.astype(np.float16).astype(F32)
    y = ck.convrot_w4a4_linear(_t(xf, gpu_device).to(dtype), qw, s16, None, convrot_groupsize=64)
    torch.cuda.synchronize()
    assert y.dtype == dtype
    qa, sa = quant.rotquant(xf, 64, 4)
    q = quant.unpack_i4(qw.cpu().numpy()).astype(np.float64)
    wdq = (q.reshape(n, -1, 64) * s16.cpu().numpy().astype(np.float64)[..., None]).reshape(n, k)
    ref = (qa.astype(np.float64) * sa.astype(np.float64)[:, None]) @ wdq.T
    assert gemm.rel_l2(ref, y.double().cpu().numpy()) < 4e-3


def test_gelu_tanh_input_act(gpu_device):
    # input_act="gelu_tanh": applied eagerly in x's type (ComfyUI's INPUT_ACT_EAGER entry), then
    # the ordinary quantized linear; equal bit for bit to quantizing torch's gelu output
    m, k, n = 200, 3072, 512
    print("[dtypes] gelu_tanh input_act", flush=True)
    x = synth.to_bf16_tensor(synth.activations(m, k, seed=8), gpu_device)
    qw, s16 = ck.quantize_w4a4_group_weight(torch.from_numpy(synth.weight(n, k, seed=9)).to(gpu_device), 64, 256)
    g = torch.nn.functional.gelu(x, approximate="tanh")
    y = ck.convrot_w4a4_linear(x, qw, s16, input_act="gelu_tanh")
    y2 = ck.convrot_w4a4_linear(g, qw, s16)
    w8 = torch.from_numpy(np.random.default_rng(1).integers(-127, 128, (n, k)).astype(np.int8)).to(gpu_device)
    ws = torch.full((n, 1), 1e-3, device=gpu_device)
    y3 = ck.int8_linear(x, w8, ws, None, torch.bfloat16, True, 256, input_act="gelu_tanh")
    y4 = ck.int8_linear(g, w8, ws, None, torch.bfloat16, True, 256)
    torch.cuda.synchronize()
    assert torch.equal(y, y2) and torch.equal(y3, y4)
    q0, s0 = quant.rotquant(g.float().cpu().numpy(), 256, 4)
    qa, sa = ops.rotate_quantize(g, 256, 4, True)
    assert np.array_equal(qa.cpu().numpy(), quant.pack_i4(q0)) and np.array_equal(sa.cpu().numpy(), s0)
    with pytest.raises(ValueError, match="input_act"):
        ck.convrot_w4a4_linear(x, qw, s16, input_act="relu2")


def test_shipped_w4a8_is_decoded_once(gpu_device):
    # the shipped asym_w4a8_int8 layout: the op decodes a weight once and reuses it; a prepared
    # weight (what the loader builds) gives the same output without the op's cache
    n, k, gs = 512, 2048, 16
    print("[dtypes] shipped w4a8 decode once", flush=True)
    rng = np.random.default_rng(4)
    qdata = torch.from_numpy(rng.integers(-128, 128, (n, k // 2)).astype(np.int8)).to(gpu_device)
    s_rel = torch.from_numpy(rng.integers(0x60, 0x70, (n, k // gs)).astype(np.uint8)).to(gpu_device)
    s_ch = torch.from_numpy(rng.uniform(1e-3, 2e-3, n).astype(F32)).to(gpu_device)
    cb = torch.linspace(-1, 1, 16, device=gpu_device)
    x = synth.to_bf16_tensor(synth.activations(64, k, seed=2), gpu_device)
    ops._DECODED.clear()
    y1 = ck.w4a8_int8_linear(x, qdata, s_rel, s_ch, cb, None, None, gs, 256, torch.bfloat16)
    entry = ops._DECODED[id(qdata)][1]
    y2 = ck.w4a8_int8_linear(x, qdata, s_rel, s_ch, cb, None, None, gs, 256, torch.bfloat16)
    assert ops._DECODED[id(qdata)][1] is entry and len(ops._DECODED) == 1
    prepared = ops.PreparedW4A8(qdata, s_rel, s_ch, cb, gs, 256)
    y3 = prepared(x, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.equal(y1, y3)
    q8, rs = ops.decode_w4a8_codebook_weight(qdata, s_rel, s_ch, cb, gs)
    assert torch.equal(entry[0], q8) and torch.equal(entry[1], rs)
    # an in-place change of an operand invalidates the decoded copy
    s_ch.mul_(2)
    y4 = ck.w4a8_int8_linear(x, qdata, s_rel, s_ch, cb, None, None, gs, 256, torch.bfloat16)
    torch.cuda.synchronize()
    assert ops._DECODED[id(qdata)][1] is not entry
    assert not torch.equal(y4, y1)
    del qdata
    assert len(ops._DECODED) == 0
