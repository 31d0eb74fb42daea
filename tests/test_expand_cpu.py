"""Host logic of the int8 expansion of 4-bit weights (ops._expansion): which calls read it. The
expansion itself and the GEMMs on it are GPU tests (test_gpu_expand.py)."""
import torch

from kitchen_amd import _lib, ops


def _w(n=256, k=3072):
    return torch.zeros((n, k // 2), dtype=torch.uint8)


def test_expansion_only_where_the_wide_kernel_reads_it():
    w = _w()
    s = torch.zeros((256, 48), dtype=torch.float16)
    # group scales: the packed weights' few rows (<= 128) run on the 128 x 128 kernel, whose
    # epilogue rounds differently, so they keep the packed weights (the same bits either way)
    for m in (1, 4, 5, 128):
        assert ops._expansion(w, None, _lib.ACT_I8, m, 3072, s) is None
    # row scales: only the GEMV's rows (<= 4) keep the packed bytes
    for m in (1, 4):
        assert ops._expansion(w, None, _lib.W4X_ROW, m, 3072) is None
    # K below the wide kernel's minimum, K groups not in pairs for the scale loads, odd scale stride
    assert ops._expansion(_w(k=128), None, _lib.ACT_I8, 1000, 128) is None
    s3 = torch.zeros((256, 3), dtype=torch.float16)
    assert ops._expansion(_w(k=192), None, _lib.ACT_I8, 1000, 192, s3) is None
    # switched off
    old = ops.EXPAND_W4
    ops.EXPAND_W4 = False
    try:
        assert ops._expansion(w, None, _lib.ACT_I8, 4096, 3072, s) is None
    finally:
        ops.EXPAND_W4 = old


def test_release_expanded_weights_empties_the_cache():
    ops._EXPANDED[12345] = {("k",): ("sig", "ex")}
    assert ops.release_expanded_weights() >= 1
    assert not ops._EXPANDED
