"""Pins oracle.codebook: the fp8 e4m3fn decode against torch's float8_e4m3fn on all 256 bytes,
the nibble order, and the int8 decode's rounding bound and special rows (CPU only)."""
import numpy as np
import torch

from oracle import codebook as cbk

F32 = np.float32


def test_fp8_decode_matches_torch_on_every_byte():
    b = np.arange(256, dtype=np.uint8)
    ours = cbk.fp8_e4m3fn_to_f32(b)
    ref = torch.from_numpy(b).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_fp8_known_answers():
    got = cbk.fp8_e4m3fn_to_f32(np.array([0x38, 0x7E, 0x01, 0x80, 0x08, 0xB8, 0x3C], np.uint8))
    assert got[0] == 1.0 and got[1] == 448.0 and got[2] == 2.0**-9
    assert got[3] == 0.0 and np.signbit(got[3])
    assert got[4] == 2.0**-6 and got[5] == -1.0 and got[6] == 1.5


def test_nibble_order_low_is_even_k():
    q = np.array([[0x21, 0xF0]], np.uint8)
    assert cbk.unpack_codes(q).tolist() == [[1, 2, 0, 15]]
    lev = cbk.levels(q, None)
    assert lev.tolist() == [[1.0, 2.0, 0.0, -1.0]]        # signed without a codebook
    cb = np.linspace(-1, 1, 16).astype(F32)
    assert np.array_equal(cbk.levels(q, cb), cb[[[1, 2, 0, 15]]])


def _case(n, k, gs, seed, with_codebook=True):
    rng = np.random.default_rng(seed)
    qdata = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    s_rel = rng.integers(0x20, 0x7F, (n, k // gs), dtype=np.uint8)      # finite positive fp8
    s_ch = rng.uniform(0.001, 0.05, n).astype(F32)
    cb = np.sort(rng.uniform(-1, 1, 16)).astype(F32) if with_codebook else None
    return qdata, s_rel, s_ch, cb


def test_decode_rounding_bound_and_range():
    for gs in (4, 16, 64):
        for with_cb in (True, False):
            qdata, s_rel, s_ch, cb = _case(12, 256, gs, seed=gs, with_codebook=with_cb)
            q8, rs = cbk.decode_w4a8_codebook(qdata, s_rel, s_ch, cb, gs)
            t = (cbk.levels(qdata, cb) * np.repeat(cbk.fp8_e4m3fn_to_f32(s_rel), gs, axis=1)).astype(np.float64)
            s = np.abs(t).max(axis=1) / 127
            assert (np.abs(q8.astype(np.float64) * s[:, None] - t) <= 0.5 * s[:, None] * (1 + 1e-6)).all()
            assert (np.abs(q8.astype(np.int16)).max(axis=1) == 127).all()
            assert np.allclose(rs, s * s_ch, rtol=1e-6)
            # q8 * row_scale reproduces the described weight to half an int8 step per row
            w = cbk.dequant_rotated(qdata, s_rel, s_ch, cb, gs)
            err = np.abs(q8.astype(np.float64) * rs.astype(np.float64)[:, None] - w)
            assert (err <= 0.5 * rs.astype(np.float64)[:, None] * (1 + 1e-5)).all()


def test_decode_zero_row_and_ties():
    qdata, s_rel, s_ch, cb = _case(3, 64, 16, seed=1)
    cb = np.array([0.0] + [0.5] * 7 + [-1.0] + [0.25] * 7, F32)
    qdata[0] = 0                                   # every level 0 -> zero row
    s_rel[1] = 0x38                                # s_rel = 1
    qdata[1] = 0x18                                # codes 8 (-1.0) and 1 (0.5): t = -1, 0.5
    q8, rs = cbk.decode_w4a8_codebook(qdata, s_rel, s_ch, cb, 16)
    assert (q8[0] == 0).all() and rs[0] == 0.0
    # absmax 1 -> s = fp32(1 / 127); the codes are the IEEE quotients rounded half to even
    s = F32(1.0) / F32(127)
    assert q8[1, 0] == np.rint(F32(-1.0) / s) and q8[1, 1] == np.rint(F32(0.5) / s)
