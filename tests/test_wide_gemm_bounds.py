"""Host-side model of the wide GEMM's global loads (comfy-quant-bench_amd/csrc/mq_gemm_wide.hip,
every tile, 256 x 256, 256 x 192 and 128 x 128, each with 512 threads): for every workgroup, thread role and K group of a launch, the buffer resource
(base row, byte range), the per-lane vector offset and the wave-uniform scalar offset each load
uses, restated from the kernel's index arithmetic. Asserts that every load either fails the
hardware range check on its vector offset (rows past M / N: offset 0x80000000; groups past the
last: a zero-byte resource), so it returns zeros without touching memory, or reads bytes that lie
wholly inside its resource range, scalar offset included (the range check does not cover the
scalar offset). Ragged M and N, K / 64 mod 4 in {0, 1, 2, 3}, split-K slices. CPU only."""
import itertools

import numpy as np
import pytest

TK = 64
KOOB = 0x80000000


TILES = [(256, 256), (256, 192), (128, 128)]


def _loads(M, N, K, ldwz, ldws, kgroups=None, slices=1, T=(256, 256)):
    """Yield (what, range_bytes, voff, soff, width) for every load lane of a launch on TM x TN tiles
    of 512 threads (vectorised over lanes with numpy where the arithmetic is per lane)."""
    TM, TN = T
    NH = TM // 128           # 1 KB DMA blocks per wave and K group
    TPR = 512 // TM          # threads per packed weight row (the B stage has TM rows)
    BPT = 32 // TPR          # packed bytes each of them loads per K group
    G = K // TK
    G4 = (G + 3) // 4 * 4
    tiles_m, tiles_n = -(-M // TM), -(-N // TN)
    lda, ldw = K, K // 2
    tid = np.arange(512)
    wave, lane = tid >> 6, tid & 63
    for tm, tn, s in itertools.product(range(tiles_m), range(tiles_n), range(slices)):
        m0, n0 = tm * TM, tn * TN
        rows_m, rows_n = min(TM, M - m0), min(TN, N - n0)
        g0 = s * kgroups if slices > 1 else 0
        g1 = min(g0 + kgroups, G4) if slices > 1 else G4
        ra = (rows_m - 1) * lda + K
        rb = (rows_n - 1) * ldw + K // 2
        rz = (rows_n - 1) * ldwz + (G + 1) // 2
        rs = ((rows_n - 1) * ldws + G) * 2
        # A DMA: wave w copies rows 16 NH w + 16 h + lane / 4, chunk lane % 4 (swizzled)
        dma = []
        for h in range(NH):
            r = 16 * NH * wave + 16 * h + (lane >> 2)
            c = (lane & 3) ^ ((r >> 1) & 3)
            dma.append(np.where(r < rows_m, r * lda + c * 16, KOOB))
        brow, bpart = tid // TPR, tid % TPR
        bhalf = bpart & 1
        b_ok = brow < rows_n
        b_off = np.where(b_ok, brow * ldw + bpart * BPT, KOOB)
        z_off = np.where(b_ok, brow * ldwz, KOOB)
        s_off = np.where(b_ok & (bpart < 2), brow * ldws * 2 + 4 * bhalf, KOOB)
        last = brow == rows_n - 1
        for g in range(g0, g1):
            live = g < G
            for h in range(NH):
                yield "A", ra if live else 0, dma[h], g * TK if live else 0, 16
            yield "B", rb if live else 0, b_off, g * (TK // 2) if live else 0, BPT
            if g % 4 == 0:
                b4 = g
                # zero-points of groups b4 .. b4 + 3 (two bytes) and scales of b4 + 2 bhalf,
                # b4 + 2 bhalf + 1 (four bytes); the tile's last weight row ends at its last valid
                # byte, so in a block past G its loads move back and their bytes are shifted down
                zb = (G + 1) // 2
                z_back = np.where(last & (b4 // 2 + 2 > zb), 1, 0)
                ga = b4 + 2 * bhalf
                s_voff = np.where(last & (ga >= G), KOOB,
                                  np.where(last & (ga + 1 == G), s_off - 2, s_off))
                s_voff = np.where(s_off == KOOB, KOOB, s_voff)
                z_voff = np.where(z_off == KOOB, KOOB, z_off - z_back)
                yield "Z", rz if live else 0, z_voff, (b4 >> 1) if live else 0, 2
                yield "S", rs if live else 0, s_voff, 2 * b4 if live else 0, 4


def _check(M, N, K, ldwz=None, ldws=None, kgroups=None, slices=1, loads=None, T=(256, 256)):
    G = K // TK
    ldwz = ldwz if ldwz is not None else ((G + 1) // 2 + 1) // 2 * 2   # the wide kernel needs even strides
    ldws = ldws if ldws is not None else (G + 1) // 2 * 2
    for what, rng, voff, soff, width in (loads or _loads)(M, N, K, ldwz, ldws, kgroups, slices, T):
        voff = np.asarray(voff, dtype=np.int64)
        masked = voff >= rng                       # fails the range check: zeros, no memory access
        ok = masked | ((voff >= 0) & (voff + soff + width <= rng))
        assert ok.all(), (f"{what} load outside its {rng}-byte range: voff {voff[~ok][:4]}, soff {soff}, "
                          f"width {width} (M={M} N={N} K={K})")


@pytest.mark.parametrize("t", TILES)
@pytest.mark.parametrize("k", [192, 256, 320, 384, 448, 1472, 3072, 3136])
@pytest.mark.parametrize("m,n", [(257, 300), (300, 256), (513, 400)])
def test_every_load_stays_in_its_range(m, n, k, t):
    _check(m, n, k, T=t)


@pytest.mark.parametrize("t", TILES)
@pytest.mark.parametrize("k", [320, 1472, 3072, 3200])
def test_split_k_slices_stay_in_range(k, t):
    g = k // 64
    blocks = (g + 3) // 4
    per = max(2, blocks // 3)
    slices = -(-blocks // per)
    _check(256, 520, k, kgroups=per * 4, slices=slices, T=t)


@pytest.mark.parametrize("t", TILES)
@pytest.mark.parametrize("which", ["S", "Z"])
def test_model_catches_an_offset_past_the_range(which, t):
    # planted mistakes: the scale dword or the zero-point word of the last block loaded without
    # moving back on the tile's last weight row (the kernel's loads before that correction) must be
    # reported for K / 64 = 5 (the block 4..7 runs past G)
    def unshifted(M, N, K, ldwz, ldws, kgroups=None, slices=1, T=(256, 256)):
        tid = np.arange(512)
        brow, bpart = tid // (512 // T[0]), tid % (512 // T[0])
        rows_n = min(T[1], N)
        for what, rng, voff, soff, width in _loads(M, N, K, ldwz, ldws, kgroups, slices, T):
            if what == which == "S":
                voff = np.where((brow < rows_n) & (bpart < 2), brow * ldws * 2 + 4 * (bpart & 1), KOOB)
            if what == which == "Z":
                voff = np.where(brow < rows_n, brow * ldwz, KOOB)
            yield what, rng, voff, soff, width

    with pytest.raises(AssertionError, match=f"{which} load"):
        _check(300, 200, 320, loads=unshifted, T=t)


def _loads_i8(M, N, K, ldwz, ldws, kgroups=None, slices=1, T=(256, 256), tiled=True, atiled=False):
    """The int8-weight kinds' DMA loads (A, and B through the same DMA roles): B rows of K bytes or,
    tiled, 16-row tiles [ceil(N / 16)][K / 64][16][64] whose K group of 16 rows is one 1 KB block
    (mq_gemm_wide.hip, wt); atiled: the activation codes in the same tiles (at). Also checks that
    each tile's resources lie inside the tiled arrays."""
    TM, TN = T
    NH = TM // 128
    G = K // TK
    G4 = (G + 3) // 4 * 4
    tiles_m, tiles_n = -(-M // TM), -(-N // TN)
    tid = np.arange(512)
    wave, lane = tid >> 6, tid & 63
    for tm, tn, s in itertools.product(range(tiles_m), range(tiles_n), range(slices)):
        m0, n0 = tm * TM, tn * TN
        rows_m, rows_n = min(TM, M - m0), min(TN, N - n0)
        g0 = s * kgroups if slices > 1 else 0
        g1 = min(g0 + kgroups, G4) if slices > 1 else G4
        ra = (rows_m - 1) * K + K
        if atiled:
            ra = ((rows_m + 15) >> 4) * G * 1024
            assert (m0 >> 4) * G * 1024 + ra <= -(-M // 16) * G * 1024
        if tiled:
            rb = ((rows_n + 15) >> 4) * G * 1024
            assert (n0 >> 4) * G * 1024 + rb <= -(-N // 16) * G * 1024
        else:
            rb = (rows_n - 1) * K + K
        dma_a, dma_b = [], []
        for h in range(NH):
            r = 16 * NH * wave + 16 * h + (lane >> 2)
            c = (lane & 3) ^ ((r >> 1) & 3)
            ta = (r >> 4) * G * 1024 + (r & 15) * 64 + c * 16 if atiled else r * K + c * 16
            dma_a.append(np.where(r < rows_m, ta, KOOB))
            tb = (r >> 4) * G * 1024 + (r & 15) * 64 + c * 16 if tiled else r * K + c * 16
            dma_b.append(np.where(r < rows_n, tb, KOOB))
        for g in range(g0, g1):
            live = g < G
            for h in range(NH):
                yield "A", ra if live else 0, dma_a[h], (g * (1024 if atiled else TK)) if live else 0, 16
                yield "B8", rb if live else 0, dma_b[h], (g * (1024 if tiled else TK)) if live else 0, 16


@pytest.mark.parametrize("atiled", [True, False])
@pytest.mark.parametrize("tiled", [True, False])
@pytest.mark.parametrize("t", TILES)
@pytest.mark.parametrize("m,n,k", [(257, 300, 192), (300, 256, 320), (513, 400, 3136), (5, 3000, 1024),
                                   (64, 17, 448), (1, 16, 192)])
def test_int8_weight_dma_stays_in_range(m, n, k, t, tiled, atiled):
    _check(m, n, k, T=t, loads=lambda *a, **kw: _loads_i8(*a, **kw, tiled=tiled, atiled=atiled))


def test_int8_tiled_model_catches_a_wrong_band_stride():
    # a band stride of one K group (instead of G) runs past the tile's range for K > 64
    def wrong(M, N, K, ldwz, ldws, kgroups=None, slices=1, T=(256, 256)):
        for what, rng, voff, soff, width in _loads_i8(M, N, K, ldwz, ldws, kgroups, slices, T, tiled=True):
            if what == "B8":
                voff = np.where(voff == KOOB, KOOB, voff + (voff // (K // TK * 1024)) * 1024 * 3)
            yield what, rng, voff, soff, width

    with pytest.raises(AssertionError):
        _check(300, 256, 256, loads=wrong)
