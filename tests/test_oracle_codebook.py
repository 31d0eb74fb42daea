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
    """Random codes; s_rel in int8 units (|level * s_rel| <= 120: levels in [-1, 1] with s_rel in
    [32, 120], signed int4 levels with s_rel in [1, 15])."""
    rng = np.random.default_rng(seed)
    qdata = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    lo, hi = (0x60, 0x70) if with_codebook else (0x38, 0x58)              # fp8 32..120 / 1..15
    s_rel = rng.integers(lo, hi, (n, k // gs), dtype=np.uint8)
    s_ch = rng.uniform(0.001, 0.05, n).astype(F32)
    cb = np.sort(rng.uniform(-1, 1, 16)).astype(F32) if with_codebook else None
    return qdata, s_rel, s_ch, cb


def _fp8_byte(v: float) -> int:
    """The e4m3fn byte of an exactly representable value (looked up over all 256 bytes)."""
    table = cbk.fp8_e4m3fn_to_f32(np.arange(256, dtype=np.uint8))
    hits = np.flatnonzero(table == F32(v))
    assert hits.size, v
    return int(hits[0])


def test_decode_pairs_int8_weight_with_stored_s_channel():
    for gs in (4, 16, 64):
        for with_cb in (True, False):
            qdata, s_rel, s_ch, cb = _case(12, 256, gs, seed=gs, with_codebook=with_cb)
            q8, rs = cbk.decode_w4a8_codebook(qdata, s_rel, s_ch, cb, gs)
            # the row scale is s_channel itself, bit for bit
            assert np.array_equal(rs.view(np.uint32), s_ch.view(np.uint32))
            # q8 is level * s_rel rounded to an integer: within half a step of it, in int8 range
            t = cbk.levels(qdata, cb).astype(np.float64) * np.repeat(cbk.fp8_e4m3fn_to_f32(s_rel), gs, axis=1)
            assert (np.abs(q8 - t) <= 0.5).all()
            # q8 * s_channel reconstructs the weight the tensors describe to half an int8 step
            w = cbk.dequant_rotated(qdata, s_rel, s_ch, cb, gs)
            err = np.abs(q8.astype(np.float64) * s_ch.astype(np.float64)[:, None] - w)
            assert (err <= 0.5 * s_ch.astype(np.float64)[:, None] * (1 + 1e-6)).all()


def test_decode_hand_built_rows():
    # codebook levels chosen by hand; s_rel 64 -> level * 64 in int8 units
    cb = np.array([0.0, 0.5, -1.0, 0.25, 1.0, -0.5, 0.0390625, -0.0078125] + [0.0] * 8, F32)
    s64, s3, s5, s448 = _fp8_byte(64.0), _fp8_byte(3.0), _fp8_byte(5.0), _fp8_byte(448.0)
    # row 0: codes 1, 2, 3, 4, 5, 6, 7, 0 at s_rel 64 -> 32, -64, 16, 64, -32, 2.5 -> 2, -0.5 -> -0, 0
    # row 1: code 1 (0.5) at s_rel 3 (1.5 -> 2), later at s_rel 5 (2.5 -> 2): ties to even
    # row 2: codes 4 / 2 (+-1) at s_rel 448: saturate at +-127
    qdata = np.zeros((3, 8), np.uint8)
    qdata[0, :4] = [0x21, 0x43, 0x65, 0x07]
    qdata[1, :2] = [0x11, 0x11]
    qdata[2, :1] = [0x24]
    s_rel = np.array([[s64, s64], [s3, s5], [s448, s448]], np.uint8)   # group size 8
    s_ch = np.array([0.5, 0.25, 2.0], F32)
    q8, rs = cbk.decode_w4a8_codebook(qdata, s_rel, s_ch, cb, 8)
    assert q8[0, :8].tolist() == [32, -64, 16, 64, -32, 2, 0, 0]
    assert q8[1, :8].tolist() == [2, 2, 2, 2, 0, 0, 0, 0] and q8[1, 8:12].tolist() == [0, 0, 0, 0]
    s_rel[1, 1] = s5
    qdata[1, 4:6] = [0x11, 0x11]
    q8, _ = cbk.decode_w4a8_codebook(qdata, s_rel, s_ch, cb, 8)
    assert q8[1, 8:12].tolist() == [2, 2, 2, 2]                        # 0.5 * 5 = 2.5 -> 2
    assert q8[2, :2].tolist() == [127, -127]
    assert rs.tolist() == [0.5, 0.25, 2.0]
    # without a codebook the levels are the signed nibbles: 7 * 15 = 105, -8 * 15 = -120
    s15 = _fp8_byte(15.0)
    q8, _ = cbk.decode_w4a8_codebook(np.array([[0x87] + [0] * 7], np.uint8), np.array([[s15, s15]], np.uint8),
                                     np.array([1.0], F32), None, 8)
    assert q8[0, :2].tolist() == [105, -120]


def test_decode_nan_scale_gives_zero():
    qdata = np.full((1, 8), 0x11, np.uint8)
    s_rel = np.array([[0x7F, _fp8_byte(2.0)]], np.uint8)               # 0x7F is e4m3fn NaN
    q8, _ = cbk.decode_w4a8_codebook(qdata, s_rel, np.array([1.0], F32), None, 8)
    assert q8[0, :8].tolist() == [0] * 8 and q8[0, 8:].tolist() == [2] * 8
