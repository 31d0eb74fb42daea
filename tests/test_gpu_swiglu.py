"""GPU parity of the SwiGLU prologue fused into rotate + quantize (mq_swiglu_rotquant, both the
fused quantizer's single rounding and the eager path's two roundings) against the CPU oracle
(oracle/swiglu.py), and of the linears with input_act="swiglu" (each in the rounding the reference
takes for its arguments).

Bar: activation codes and scales bit-exact; linear outputs within 1e-2 rel-L2 of the oracle's
fp64 result (the tests require < 4e-3). Each case prints its name before the GPU step."""
import numpy as np
import pytest
import torch

from kitchen_amd import _lib, ops, synth, weights
from oracle import gemm, quant, swiglu

pytestmark = pytest.mark.gpu


def _h(m, k, seed, gate_scale=3.0):
    """gate | up rows as bf16 bits [m, 2k]: gate ~ N(0, gate_scale^2) covers silu's curved range,
    up carries the configs' outlier channels."""
    rng = np.random.default_rng(seed)
    g = rng.standard_normal((m, k)).astype(np.float32) * gate_scale
    u = synth.bf16_bits_to_f32(synth.activations(m, k, seed=seed + 1))
    return synth.f32_to_bf16_bits(np.concatenate([g, u], axis=1))


def _check(hb, hblock, bits, packed, dev, label, mode=_lib.SWIGLU_FUSED):
    m, k2 = hb.shape
    eager = mode == _lib.SWIGLU_EAGER
    print(f"[swiglu] {label} M={m} K={k2 // 2} hblock={hblock} bits={bits} packed={packed} eager={eager}", flush=True)
    h = synth.to_bf16_tensor(hb, dev)
    q, s = ops.rotate_quantize(h, hblock, bits, packed, swiglu=mode)
    torch.cuda.synchronize()
    q, s = q.cpu().numpy(), s.cpu().numpy()
    act = swiglu.swiglu_bf16_eager if eager else swiglu.swiglu_bf16
    q0, s0 = swiglu.swiglu_rotquant(synth.bf16_bits_to_f32(hb), hblock, bits, eager=eager) if hblock else \
        quant.quant_per_token(act(*np.split(synth.bf16_bits_to_f32(hb), 2, axis=1)), 127 if bits == 8 else 7)
    assert np.array_equal(s.view(np.uint32), s0.view(np.uint32)), "scales differ"
    if packed == _lib.Q_X16ALT:
        sign = np.where((np.arange(q0.shape[1]) // 64) % 2 == 1, -1, 1).astype(np.int16)
        assert np.array_equal(q.astype(np.int16), 16 * q0.astype(np.int16) * sign[None, :]), "x16alt codes differ"
    elif packed:
        assert np.array_equal(q, quant.pack_i4(q0)), "packed codes differ"
    else:
        diff = np.nonzero(q != q0)
        assert diff[0].size == 0, f"{diff[0].size} codes differ, first at {diff[0][0]},{diff[1][0]}"


def test_activation_bits_exact_on_a_dense_gate_sweep(gpu_device):
    # one nonzero column per row (hblock 0, K = 16): the row's scale max(|a| / 127, 1e-10) then
    # carries the bf16 activation a = swiglu(g, u) itself, so equal scales pin a bit for bit; every
    # finite bf16 gate value in [-200, 200] (the exp clamp sits at |g| = 80 / 88)
    g = synth.bf16_bits_to_f32(np.arange(0, 0x10000, dtype=np.uint16).astype(np.uint16))
    g = g[np.isfinite(g) & (np.abs(g) <= 200)]
    rng = np.random.default_rng(0)
    for up in (1.0, -0.3125, 7.5, None):
        u = rng.standard_normal(g.size).astype(np.float32) * 4 if up is None else np.full(g.size, up, np.float32)
        h = np.zeros((g.size, 32), np.float32)
        h[:, 0], h[:, 16] = g, u
        for mode in (_lib.SWIGLU_FUSED, _lib.SWIGLU_EAGER):
            _check(synth.f32_to_bf16_bits(h), 0, 8, False, gpu_device, f"sweep up={up}", mode)


@pytest.mark.parametrize("hblock", [0, 16, 64, 256])
@pytest.mark.parametrize("bits,packed", [(8, False), (4, False), (4, True), (4, _lib.Q_X16ALT)])
@pytest.mark.parametrize("mode", [_lib.SWIGLU_FUSED, _lib.SWIGLU_EAGER])
def test_mlp_down_input_bitexact(gpu_device, hblock, bits, packed, mode):
    # MLP-down input of C1: h = [gate | up] [512, 2 x 12288]
    _check(_h(512, 12288, seed=7), hblock, bits, packed, gpu_device, "C1-down", mode)


@pytest.mark.parametrize("k", [256, 1024, 1280, 3072, 16384])
def test_k_range_and_m_tails(gpu_device, k):
    for m in (1, 3, 65):
        _check(_h(m, k, seed=k + m), 256, 8, False, gpu_device, f"K{k}")
        _check(_h(m, k, seed=k + m), 256, 4, True, gpu_device, f"K{k}")


def test_strided_h_c_abi(gpu_device):
    print("[swiglu] strided ldh", flush=True)
    m, k = 17, 1024
    hb = _h(m, k, seed=3)
    wide = np.zeros((m, 2 * k + 256), np.uint16)
    wide[:, :2 * k] = hb
    hw = synth.to_bf16_tensor(wide, gpu_device)
    q = torch.full((m, 1040), 99, dtype=torch.int8, device=gpu_device)
    s = torch.empty(m, dtype=torch.float32, device=gpu_device)
    _lib.call("mq_swiglu_rotquant", hw.data_ptr(), _lib.DT_BF16, m, k, 2 * k + 256, 256, 8, 0, _lib.SWIGLU_FUSED,
              q.data_ptr(), 1040, s.data_ptr(), _lib.stream_of(hw))
    torch.cuda.synchronize()
    q0, s0 = swiglu.swiglu_rotquant(synth.bf16_bits_to_f32(hb), 256, 8)
    qn = q.cpu().numpy()
    assert np.array_equal(qn[:, :k], q0) and np.array_equal(s.cpu().numpy(), s0)
    assert (qn[:, k:] == 99).all(), "wrote past K"


def test_reference_entry_point_name(gpu_device):
    print("[swiglu] swiglu_quantize_int4_rowwise_convrot64", flush=True)
    hb = _h(64, 3072, seed=5)
    q, s = ops.swiglu_quantize_int4_rowwise_convrot64(synth.to_bf16_tensor(hb, gpu_device))
    q0, s0 = swiglu.swiglu_rotquant(synth.bf16_bits_to_f32(hb), 256, 4)
    assert q.shape == (64, 1536) and s.shape == (64,)
    assert np.array_equal(q.cpu().numpy(), quant.pack_i4(q0)) and np.array_equal(s.cpu().numpy(), s0)
    with pytest.raises(ValueError):
        ops.swiglu_quantize_int4_rowwise_convrot64(synth.to_bf16_tensor(_h(4, 320, seed=1), gpu_device))


@pytest.mark.parametrize("linear_dtype,hblock", [("int4", 64), ("int8", 64), ("int4", 256), ("int8", 256)])
def test_convrot_w4a4_linear_input_act_swiglu(gpu_device, linear_dtype, hblock):
    # MLP-down of C2 at reduced M: W4A4 group weights (K = 12288 -> N = 3072). comfy-kitchen fuses
    # input_act="swiglu" (one rounding) only for int4 activations under H256; H64 and int8
    # activations take its eager path, silu(gate).mul_(up) in bf16 (two roundings)
    m, k, n = 256, 12288, 3072
    eager = not (linear_dtype == "int4" and hblock == 256)
    print(f"[swiglu] convrot_w4a4_linear input_act=swiglu {linear_dtype} H{hblock} eager={eager} M={m} K={k} N={n}",
          flush=True)
    hb = _h(m, k, seed=11)
    w = synth.weight(n, k, seed=12)
    wt = torch.from_numpy(w).to(gpu_device)
    qw, s16 = weights.quantize_w4a4_group_weight(wt, 64, hblock)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(13)).to(torch.bfloat16)
    h = synth.to_bf16_tensor(hb, gpu_device)
    y = ops.convrot_w4a4_linear(h, qw, s16, bias.to(gpu_device), convrot_groupsize=hblock,
                                linear_dtype=linear_dtype, input_act="swiglu")
    torch.cuda.synchronize()
    act = swiglu.swiglu_bf16_eager if eager else swiglu.swiglu_bf16
    a = act(*np.split(synth.bf16_bits_to_f32(hb), 2, axis=1))
    y_plain = ops.convrot_w4a4_linear(synth.to_bf16_tensor(synth.f32_to_bf16_bits(a), gpu_device), qw, s16,
                                      bias.to(gpu_device), convrot_groupsize=hblock, linear_dtype=linear_dtype)
    torch.cuda.synchronize()
    # the prologue in the reference's rounding, then the plain linear, bit for bit
    assert torch.equal(y, y_plain)
    if eager:
        # the eager activation is what torch's own silu(gate).mul_(up) in bf16 gives (up to torch's
        # fp32 silu next to a rounding boundary): the linear of torch's activation agrees closely
        gate, up = h.chunk(2, dim=-1)
        y_torch = ops.convrot_w4a4_linear(torch.nn.functional.silu(gate).mul_(up), qw, s16, bias.to(gpu_device),
                                          convrot_groupsize=hblock, linear_dtype=linear_dtype)
        torch.cuda.synchronize()
        assert gemm.rel_l2(y_torch.float().cpu().numpy(), y.float().cpu().numpy()) < 1e-3
    # against the oracle on the first 32 rows: int4 or int8 per-token codes of the bf16 activation,
    # exact int32 group partials, fp64 epilogue
    rows = slice(0, 32)
    q0, s0 = swiglu.swiglu_rotquant(synth.bf16_bits_to_f32(hb[rows]), hblock, 4 if linear_dtype == "int4" else 8,
                                    eager=eager)
    qa, sa = quant.rotquant(a[rows], hblock, 4 if linear_dtype == "int4" else 8)
    assert np.array_equal(qa, q0) and np.array_equal(sa, s0)
    p = gemm.partials(qa, quant.unpack_i4(qw.cpu().numpy()), 64)
    ref = gemm.epilogue_group(p, sa, s16.cpu().numpy().astype(np.float64), bias.float().numpy())
    err = gemm.rel_l2(ref, y.float().cpu().numpy()[rows])
    print(f"[swiglu] rel L2 {err:.2e}", flush=True)
    assert err < 4e-3


def test_activation_codes_eager_h64_int4(gpu_device):
    # the eager activation's int4 codes under H64 straight from the C ABI, against the oracle
    m, k = 96, 3072
    print(f"[swiglu] C ABI eager H64 int4 M={m} K={k}", flush=True)
    hb = _h(m, k, seed=31)
    h = synth.to_bf16_tensor(hb, gpu_device)
    q = torch.empty((m, k // 2), dtype=torch.int8, device=gpu_device)
    s = torch.empty(m, dtype=torch.float32, device=gpu_device)
    _lib.call("mq_swiglu_rotquant", h.data_ptr(), _lib.DT_BF16, m, k, 2 * k, 64, 4, _lib.Q_PACKED,
              _lib.SWIGLU_EAGER, q.data_ptr(), k // 2, s.data_ptr(), _lib.stream_of(h))
    torch.cuda.synchronize()
    q0, s0 = swiglu.swiglu_rotquant(synth.bf16_bits_to_f32(hb), 64, 4, eager=True)
    assert np.array_equal(q.cpu().numpy(), quant.pack_i4(q0)) and np.array_equal(s.cpu().numpy(), s0)
    # and the fused codes of the same input differ somewhere (the mode is not ignored)
    q1, _ = swiglu.swiglu_rotquant(synth.bf16_bits_to_f32(hb), 64, 4, eager=False)
    assert not np.array_equal(q0, q1)
    with pytest.raises(ValueError, match="mode"):
        _lib.call("mq_swiglu_rotquant", h.data_ptr(), _lib.DT_BF16, m, k, 2 * k, 64, 4, _lib.Q_PACKED, 3,
                  q.data_ptr(), k // 2, s.data_ptr(), _lib.stream_of(h))


def test_int8_linear_input_act_swiglu(gpu_device):
    m, k, n = 128, 3072, 1024
    print(f"[swiglu] int8_linear input_act=swiglu M={m} K={k} N={n}", flush=True)
    hb = _h(m, k, seed=21)
    w = synth.weight(n, k, seed=22)
    qw, ws = weights.quantize_int8_convrot_weight(torch.from_numpy(w).to(gpu_device), 256)
    h = synth.to_bf16_tensor(hb, gpu_device)
    y = ops.int8_linear(h, qw, ws, None, convrot=True, convrot_groupsize=256, input_act="swiglu")
    a = swiglu.swiglu_bf16(*np.split(synth.bf16_bits_to_f32(hb), 2, axis=1))
    y_plain = ops.int8_linear(synth.to_bf16_tensor(synth.f32_to_bf16_bits(a), gpu_device), qw, ws, None,
                              convrot=True, convrot_groupsize=256)
    torch.cuda.synchronize()
    assert torch.equal(y, y_plain)
    # activations outside ComfyUI's INPUT_ACT_EAGER table are refused (gelu_tanh is covered in
    # tests/test_gpu_dtypes.py)
    with pytest.raises(ValueError, match="input_act"):
        ops.int8_linear(h, qw, ws, None, convrot=True, input_act="relu")
