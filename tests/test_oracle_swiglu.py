"""Pins oracle.swiglu: silu correctly rounded to fp32 over every bf16 gate (exact decimal
arithmetic), its closed-form regions and identities, the bf16 rounding of the product, and the
generated table libmq.so stages in LDS (CPU only)."""
import importlib.util
import os
import struct
from decimal import MAX_EMAX, MIN_EMIN, Decimal, localcontext

import numpy as np
import pytest

from conftest import PKG_ROOT
from oracle import quant, swiglu

F32 = np.float32


def _all_bf16():
    bits = np.arange(0x10000, dtype=np.uint32)
    g = (bits << np.uint32(16)).view(F32)
    keep = np.isfinite(g)
    return bits[keep].astype(np.uint16), g[keep]


def _rn32_decimal(d: Decimal) -> int:
    """Bits of the fp32 nearest to d (ties to even), searched around the nearest double."""
    if d == 0:
        return 0
    u = np.array([float(d)], np.float64).astype(F32).view(np.uint32)[0]
    best = None
    for c in (int(u) - 1, int(u), int(u) + 1):
        v = struct.unpack("<f", struct.pack("<I", c & 0xFFFFFFFF))[0]
        if not np.isfinite(v):
            continue
        key = (abs(Decimal(v) - d), c & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return best[1] & 0xFFFFFFFF


@pytest.fixture(scope="module")
def exact_silu():
    """Correctly rounded fp32 silu of every finite bf16 gate with |g| <= 1e4, by decimal arithmetic."""
    _, g = _all_bf16()
    sel = np.abs(g) <= 1e4
    out = np.zeros(g.shape, np.uint32)
    with localcontext() as ctx:
        ctx.prec, ctx.Emax, ctx.Emin = 60, MAX_EMAX, MIN_EMIN
        for i in np.nonzero(sel)[0]:
            d = Decimal(float(g[i]))
            s = d / (1 + (-d).exp())
            r = _rn32_decimal(s)
            out[i] = r | (0x80000000 if (r == 0 and np.signbit(g[i])) else 0)
    return sel, out


def test_silu32_is_correctly_rounded_for_every_bf16_gate(exact_silu):
    sel, want = exact_silu
    _, g = _all_bf16()
    got = swiglu.silu32(g).view(np.uint32)
    assert np.array_equal(got[sel], want[sel])


def test_exhaustive_check_catches_planted_mistakes(exact_silu):
    # an all-fp32 evaluation (exp and division rounded separately) is what a plausible shortcut
    # gives; the exhaustive comparison must reject it
    sel, want = exact_silu
    _, g = _all_bf16()

    def silu_fp32(x):
        x = np.asarray(x, F32)
        with np.errstate(over="ignore"):
            return (x / (F32(1) + np.exp(-x))).astype(F32)

    assert not np.array_equal(silu_fp32(g).view(np.uint32)[sel], want[sel])
    # and so must a sign slip in the exponent
    with np.errstate(over="ignore"):
        wrong = (g.astype(np.float64) / (1.0 + np.exp(g.astype(np.float64)))).astype(F32)
    assert not np.array_equal(wrong.view(np.uint32)[sel], want[sel])


def test_closed_form_regions():
    _, g = _all_bf16()
    s = swiglu.silu32(g)
    tiny = np.abs(g) < 2.0**-25
    assert np.array_equal(s[tiny].view(np.uint32), (g[tiny] * F32(0.5)).view(np.uint32))
    big = g >= 128
    assert np.array_equal(s[big], g[big])
    neg = g <= -128
    assert (s[neg] == 0).all() and np.signbit(s[neg]).all()


def test_silu_identities():
    _, g = _all_bf16()
    g = g[np.abs(g) < 60]
    s, sm = swiglu.silu32(g).astype(np.float64), swiglu.silu32(-g).astype(np.float64)
    # silu(g) - silu(-g) = g: each term within half an ulp of its exact value
    tol = np.spacing(np.abs(s).astype(F32)) + np.spacing(np.abs(sm).astype(F32))
    assert (np.abs(s - sm - g.astype(np.float64)) <= tol).all()
    # increasing above the minimum at g = -1.2785
    inc = np.sort(g[g > -1.27])
    assert (np.diff(swiglu.silu32(inc).astype(np.float64)) >= 0).all()
    assert np.sign(swiglu.silu32(g)).tolist() == np.sign(g).tolist()


def test_swiglu_bf16_product_rounding():
    rng = np.random.default_rng(2)
    g = quant.bf16_bits_to_f32(quant.f32_to_bf16_bits(rng.standard_normal(400_000).astype(F32) * 3))
    u = quant.bf16_bits_to_f32(quant.f32_to_bf16_bits(rng.standard_normal(400_000).astype(F32) * 2))
    got = swiglu.swiglu_bf16(g, u)
    # one fp32 rounding of silu * u, then bf16 round-to-nearest-even
    s = swiglu.silu32(g)
    assert np.array_equal(got, quant.bf16_bits_to_f32(quant.f32_to_bf16_bits((s * u).astype(F32))))
    # against the product rounded once from float64: equal except within fp32 error of a bf16
    # rounding midpoint, and then one bf16 step apart
    exact = s.astype(np.float64) * u.astype(np.float64)
    e = np.floor(np.log2(np.abs(np.where(exact == 0, 1.0, exact))))
    step = 2.0 ** (e - 7)
    want = np.where(exact == 0, 0.0, np.round(exact / step) * step)
    diff = got.astype(np.float64) != want
    frac = np.abs(exact / step - np.floor(exact / step) - 0.5)
    assert (frac[diff] < 2.0**-15).all()
    assert np.allclose(np.abs(got[diff] - want[diff]), step[diff])
    assert diff.mean() < 1e-3


def test_swiglu_special_values():
    g = np.array([0.0, -0.0, 50.0, 200.0, -200.0, 3.0], F32)
    u = np.array([5.0, 5.0, 2.0, 0.5, 7.0, 0.0], F32)
    got = swiglu.swiglu_bf16(g, u)
    assert got[0] == 0.0 and got[1] == 0.0
    assert got[2] == F32(100.0) and got[3] == F32(100.0)
    assert got[4] == 0.0 and got[5] == 0.0


def test_swiglu_rotquant_is_prologue_then_rotquant():
    rng = np.random.default_rng(5)
    h = quant.bf16_bits_to_f32(quant.f32_to_bf16_bits(rng.standard_normal((3, 1024)).astype(F32) * 2))
    q, s = swiglu.swiglu_rotquant(h, 256, 8)
    q2, s2 = quant.rotquant(swiglu.swiglu_bf16(h[:, :512], h[:, 512:]), 256, 8)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)
    q3, _ = quant.rotquant(swiglu.swiglu_bf16(h[:, 512:], h[:, :512]), 256, 8)
    assert not np.array_equal(q, q3)


def test_generated_device_table_matches_oracle():
    # the table libmq.so's build generates (comfy-quant-bench_amd/csrc/gen_silu_table.py) holds the
    # oracle's silu32 for its bf16 range, and the kernel's closed forms cover the rest
    path = os.path.join(PKG_ROOT, "csrc", "gen_silu_table.py")
    spec = importlib.util.spec_from_file_location("gen_silu_table", path)
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    tab = np.array(gen.table(), np.uint32)
    n = gen.ENTRIES
    assert tab.size == 2 * n
    for sign in (0, 1):
        b = (np.arange(gen.LO, gen.HI, dtype=np.uint32) | np.uint32(sign << 15))
        g = (b << np.uint32(16)).view(F32)
        assert np.array_equal(tab[sign * n:(sign + 1) * n], swiglu.silu32(g).view(np.uint32))
    _, g = _all_bf16()
    t = (g.view(np.uint32) >> 16) & 0x7FFF
    assert (np.abs(g[t < gen.LO]) < 2.0**-25).all() and (np.abs(g[t >= gen.HI]) >= 128).all()


def _all_f16():
    bits = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
    g = bits.view(np.float16).astype(F32)
    keep = np.isfinite(g)
    return bits[keep], g[keep]


def test_silu32_is_correctly_rounded_for_every_f16_gate():
    # fp16 gates (the fp16 SwiGLU prologue): every finite pattern against exact decimal arithmetic
    _, g = _all_f16()
    got = swiglu.silu32(g).view(np.uint32)
    with localcontext() as ctx:
        ctx.prec, ctx.Emax, ctx.Emin = 60, MAX_EMAX, MIN_EMIN
        for i in range(g.size):
            d = Decimal(float(g[i]))
            r = _rn32_decimal(d / (1 + (-d).exp()))
            r |= 0x80000000 if (r == 0 and np.signbit(g[i])) else 0
            assert got[i] == r, f"gate {g[i]!r}: {got[i]:#010x} != {r:#010x}"


def test_swiglu_f16_product_rounding():
    rng = np.random.default_rng(3)
    g = (rng.standard_normal(200_000) * 3).astype(np.float16).astype(F32)
    u = (rng.standard_normal(200_000) * 2).astype(np.float16).astype(F32)
    got = swiglu.swiglu_f16(g, u)
    # one fp32 rounding of silu * u, then fp16 round-to-nearest-even (numpy's float16 cast)
    assert np.array_equal(got, (swiglu.silu32(g) * u).astype(F32).astype(np.float16).astype(F32))
    # fp16 values, and within one fp16 step of the float64 product
    assert np.array_equal(got, got.astype(np.float16).astype(F32))
    exact = swiglu.silu32(g).astype(np.float64) * u.astype(np.float64)
    assert (np.abs(got - exact) <= np.spacing(np.abs(got).astype(np.float16)).astype(np.float64)).all()
    # the bf16 rounding is a different function on the same inputs
    assert not np.array_equal(got, swiglu.swiglu_bf16(g, u))


def test_generated_f16_device_table_matches_oracle():
    # the fp16 table (one entry per 16-bit pattern) holds the oracle's silu32 of every finite gate
    path = os.path.join(PKG_ROOT, "csrc", "gen_silu_table.py")
    spec = importlib.util.spec_from_file_location("gen_silu_table", path)
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    tab = np.array(gen.table_f16(), np.uint32)
    assert tab.size == 0x10000
    bits, g = _all_f16()
    assert np.array_equal(tab[bits.astype(np.int64)], swiglu.silu32(g).view(np.uint32))
    # non-finite gates follow the formula in IEEE arithmetic: +inf -> +inf, -inf and NaN -> NaN
    assert tab[0x7C00] == 0x7F800000 and np.isnan(tab[[0xFC00, 0x7E00]].view(F32)).all()


def test_eager_swiglu_rounds_twice_like_torch():
    """The eager activation is silu(gate).mul_(up) in the input's type: silu rounded to the type,
    then the product rounded again. Checked against torch's own rounding (silu taken in float64 and
    converted by torch), and against torch's silu itself on the CPU, which may differ only where
    its fp32 silu lies next to a rounding boundary."""
    import torch

    rng = np.random.default_rng(11)
    g = quant.bf16_bits_to_f32(quant.f32_to_bf16_bits(rng.standard_normal(200_000).astype(F32) * 3))
    u = quant.bf16_bits_to_f32(quant.f32_to_bf16_bits(rng.standard_normal(200_000).astype(F32) * 2))
    g64 = g.astype(np.float64)
    s64 = torch.from_numpy(g64 / (1 + np.exp(-g64)))
    for dt, ours in ((torch.bfloat16, swiglu.swiglu_bf16_eager), (torch.float16, swiglu.swiglu_f16_eager)):
        gt, ut = torch.from_numpy(g).to(dt), torch.from_numpy(u).to(dt)
        want = (s64.float().to(dt).float() * ut.float()).to(dt).float().numpy()
        got = ours(gt.float().numpy(), ut.float().numpy())
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        eager_torch = torch.nn.functional.silu(gt).mul_(ut).float().numpy()
        assert (got != eager_torch).mean() < 1e-3
    # the two roundings differ from the fused single rounding on some inputs, by one unit at most
    fused = swiglu.swiglu_bf16(g, u)
    eager = swiglu.swiglu_bf16_eager(g, u)
    diff = fused != eager
    assert 0.05 < diff.mean() < 0.5
    ulp = np.abs(fused.view(np.int32) - eager.view(np.int32)) >> 16
    assert ulp.max() == 1


def test_eager_swiglu_known_answers():
    # g = 1: silu32 = 0.731058597564697 -> bf16 0.73046875; times u = 1.0078125 (1 + 2^-7):
    # eager 0.73046875 * 1.0078125 = 0.736175537... -> bf16 0.734375 (1.46875 * 2^-1),
    # fused 0.731058... * 1.0078125 = 0.7367700... -> bf16 0.73828125
    g = np.array([1.0], F32)
    u = np.array([1.0078125], F32)
    assert swiglu.swiglu_bf16_eager(g, u)[0] == F32(0.734375)
    assert swiglu.swiglu_bf16(g, u)[0] == F32(0.73828125)
