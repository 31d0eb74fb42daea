"""The C ABI: libmq.so loads, exports every symbol include/mq.h declares, and rejects bad
arguments with MQ_EINVAL before touching the GPU (CPU only: no kernel is launched)."""
import ctypes
import os
import re

import pytest

from conftest import REPO

HEADER = os.path.join(REPO, "include", "mq.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(mq_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    from kitchen_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libmq.so is not built (run __graft_entry__.build())")
    return _lib.load()


def test_header_declares_expected_entry_points():
    syms = declared_symbols()
    assert "mq_rotquant" in syms and "mq_gemm_w4_group" in syms and "mq_last_error" in syms
    from kitchen_amd import _lib

    assert sorted(_lib.EXPORTED) == syms


def test_library_exports_every_declared_symbol(lib):
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_abi_version(lib):
    assert lib.mq_abi_version() == 11


def _err(lib):
    return lib.mq_last_error().decode()


def test_rotquant_validation_rejects_before_launch(lib):
    # null device pointers are never dereferenced: every case fails validation first
    assert lib.mq_rotquant(None, 0, 4, 256, 256, 256, 5, 0, None, 256, None, None) == -1
    assert "bits" in _err(lib)
    assert lib.mq_rotquant(None, 0, 4, 256, 256, 32, 8, 0, None, 256, None, None) == -1
    assert "group size" in _err(lib)
    assert lib.mq_rotquant(None, 0, 4, 200, 200, 0, 8, 0, None, 256, None, None) == -1
    assert "multiple of 16" in _err(lib)
    assert lib.mq_rotquant(None, 0, 4, 320, 320, 256, 8, 0, None, 320, None, None) == -1
    assert "not a multiple of the group size" in _err(lib)
    assert lib.mq_rotquant(None, 0, 4, 32768, 32768, 256, 8, 0, None, 32768, None, None) == -2
    assert lib.mq_rotquant(None, 0, 4, 256, 256, 256, 8, 1, None, 256, None, None) == -1
    assert "packed" in _err(lib)
    assert lib.mq_rotquant(None, 0, 4, 256, 256, 256, 8, 2, None, 256, None, None) == -1
    assert "packed" in _err(lib)
    assert lib.mq_rotquant(None, 0, 4, 256, 256, 256, 4, 3, None, 256, None, None) == -1
    assert "layout" in _err(lib)
    # M == 0 is a valid no-op
    assert lib.mq_rotquant(None, 0, 0, 256, 256, 256, 8, 0, None, 256, None, None) == 0
    # input types: bf16 (0), fp16 (1), fp32 (2); rows must be multiples of 16 bytes (fake aligned
    # addresses: every case below fails validation, nothing is dereferenced or launched)
    a = 1 << 20
    assert lib.mq_rotquant(None, 3, 4, 256, 256, 256, 8, 0, None, 256, None, None) == -1
    assert "input type" in _err(lib)
    assert lib.mq_rotquant(a, 1, 4, 256, 260, 256, 8, 0, a, 256, a, None) == -1
    assert "ldx % 8" in _err(lib)
    assert lib.mq_rotquant(a, 2, 4, 256, 258, 256, 8, 0, a, 256, a, None) == -1
    assert "ldx % 4" in _err(lib)
    assert lib.mq_rotquant(None, 2, 0, 256, 256, 256, 8, 0, None, 256, None, None) == 0


def test_swiglu_rotquant_validation_rejects_before_launch(lib):
    # h holds gate | up: its row stride must cover 2K columns
    assert lib.mq_swiglu_rotquant(None, 0, 4, 256, 256, 256, 8, 0, 1, None, 256, None, None) == -1
    assert "null" in _err(lib)
    assert lib.mq_swiglu_rotquant(None, 0, 4, 256, 384, 256, 8, 0, 1, None, 256, None, None) == -1
    assert "swiglu_rotquant" in _err(lib)
    assert lib.mq_swiglu_rotquant(None, 0, 4, 320, 640, 256, 8, 0, 1, None, 320, None, None) == -1
    assert "not a multiple of the group size" in _err(lib)
    assert lib.mq_swiglu_rotquant(None, 0, 4, 32768, 65536, 256, 8, 0, 1, None, 32768, None, None) == -2
    assert lib.mq_swiglu_rotquant(None, 0, 0, 256, 512, 256, 4, 1, 1, None, 128, None, None) == 0
    # the SwiGLU prologue takes bf16 or fp16 (as the reference's fused quantizer does)
    assert lib.mq_swiglu_rotquant(None, 2, 4, 256, 512, 256, 8, 0, 1, None, 256, None, None) == -1
    assert "input type" in _err(lib)
    assert lib.mq_swiglu_rotquant(None, 1, 0, 256, 512, 256, 8, 0, 1, None, 256, None, None) == 0
    # the mode is the fused quantizer's single rounding (1) or the eager path's two (2)
    assert lib.mq_swiglu_rotquant(None, 0, 0, 256, 512, 256, 8, 0, 2, None, 256, None, None) == 0
    assert lib.mq_swiglu_rotquant(None, 0, 4, 256, 512, 256, 8, 0, 0, None, 256, None, None) == -1
    assert "mode" in _err(lib)


def test_decode_codebook_validation_rejects_before_launch(lib):
    assert lib.mq_decode_w4a8_codebook(None, 128, None, 16, None, None, 12, 8, 192, None, 192, None, None) == -1
    assert "group_size" in _err(lib)
    assert lib.mq_decode_w4a8_codebook(None, 128, None, 16, None, None, 16, 8, 200, None, 200, None, None) == -1
    assert "multiple of 16" in _err(lib)
    assert lib.mq_decode_w4a8_codebook(None, 128, None, 16, None, None, 16, 8, 256, None, 256, None, None) == -1
    assert "null" in _err(lib)
    assert lib.mq_decode_w4a8_codebook(None, 128, None, 16, None, None, 16, 0, 256, None, 256, None, None) == 0


def test_gemm_validation_rejects_before_launch(lib):
    assert lib.mq_gemm_w4_group(None, 64, None, None, 32, None, 1, None, 1, 128, 0, None, 0, None, 0, 8, 8, 8, 64, None) == -1
    assert "group size must be 64" in _err(lib)
    assert lib.mq_gemm_w4_group(None, 96, None, None, 48, None, 1, None, 1, 64, 0, None, 0, None, 0, 8, 8, 8, 96, None) == -1
    assert "multiple of 64" in _err(lib)
    assert lib.mq_gemm_w4_group(None, 64, None, None, 32, None, 1, None, 1, 64, 3, None, 0, None, 0, 8, 8, 8, 64, None) == -1
    assert "act_mode" in _err(lib)
    assert lib.mq_gemm_w4_group_partials(None, 64, None, 32, None, 1, 64, 7, None, 8, 8, 64, None) == -1
    assert "act_mode" in _err(lib)
    assert lib.mq_gemm_rowscale(None, 64, None, None, 64, 3, None, None, 0, None, 0, 8, 8, 8, 64, None) == -1
    assert "wbits" in _err(lib)
    assert lib.mq_gemm_rowscale_acc(None, 64, None, 64, 8, None, 8, 8, 64, None) == -1
    assert "null" in _err(lib)


def test_tile16_weight_validation(lib):
    # the 16-row tile layout: int8 weights only, K >= 192, whole tiled array under 2 GiB
    a = 1 << 20
    assert lib.mq_gemm_rowscale(a, 64, a, a, 32, 4 | 0x100, a, None, 0, a, 0, 64, 8, 8, 64, None) == -1
    assert "int8 weights" in _err(lib)
    assert lib.mq_gemm_rowscale(a, 128, a, a, 128, 8 | 0x100, a, None, 0, a, 0, 64, 8, 8, 128, None) == -1
    assert "K >= 192" in _err(lib)
    assert lib.mq_gemm_rowscale_acc(a, 1 << 16, a, 0, 8 | 0x100, a, 8, 1 << 16, 1 << 16, None) == -1
    assert "2 GiB" in _err(lib)
    assert lib.mq_tile_weight_i8(a, 128, 8, 128, a, None) == -1
    assert "K >= 192" in _err(lib)
    assert lib.mq_tile_weight_i8(a, 200, 8, 192, a, None) == -1
    assert "ldw" in _err(lib)
    assert lib.mq_tile_weight_i8(None, 192, 0, 192, None, None) == 0


def test_gemm_output_types_are_checked(lib):
    # operand pointers must be non-null before the output checks run: fake 256-byte aligned addresses
    # that are never dereferenced (every case fails validation before any launch)
    a = 1 << 20
    assert lib.mq_gemm_w4_group(a, 64, a, a, 32, a, 1, None, 1, 64, 0, None, 0, a, 3, 8, 8, 8, 64, None) == -1
    assert "output type" in _err(lib)
    assert lib.mq_gemm_w4_group(a, 64, a, a, 32, a, 1, None, 1, 64, 0, a, 5, a, 0, 8, 8, 8, 64, None) == -1
    assert "bias type" in _err(lib)
    assert lib.mq_gemm_w4_group(a, 64, a, a, 32, a, 1, None, 1, 64, 0, None, 0, a + 2, 2, 8, 8, 8, 64, None) == -1
    assert "aligned" in _err(lib)
    assert lib.mq_gemm_rowscale(a, 64, a, a, 64, 8, a, None, 0, None, 1, 8, 8, 8, 64, None) == -1
    assert "non-null" in _err(lib)
    assert lib.mq_gemm_rowscale(a, 64, a, a, 64, 8, a, a + 2, 2, a, 1, 8, 8, 8, 64, None) == -1
    assert "bias must be aligned" in _err(lib)
    assert lib.mq_gemm_rowscale(a, 64, a, a, 64, 8, a, None, 0, a, 1, 4, 8, 8, 64, None) == -1
    assert "ldy" in _err(lib)


def test_quantize_weight_validation_rejects_before_launch(lib):
    # (w, dtype, N, K, ldw, hblock, format, q, ldq, scale, ld_scale, zero, ld_zero, stream)
    assert lib.mq_quantize_weight(None, 3, 4, 256, 256, 256, 0, None, 128, None, 4, None, 2, None) == -1
    assert "dtype" in _err(lib)
    assert lib.mq_quantize_weight(None, 0, 4, 256, 256, 256, 4, None, 128, None, 4, None, 2, None) == -1
    assert "format" in _err(lib)
    assert lib.mq_quantize_weight(None, 0, 4, 96, 96, 0, 0, None, 48, None, 2, None, 1, None) == -1
    assert "multiple of 64" in _err(lib)
    assert lib.mq_quantize_weight(None, 0, 4, 200, 200, 0, 3, None, 200, None, 1, None, 0, None) == -1
    assert "multiple of 16" in _err(lib)
    assert lib.mq_quantize_weight(None, 0, 4, 320, 320, 256, 2, None, 160, None, 1, None, 0, None) == -1
    assert "not a multiple of the group size" in _err(lib)
    assert lib.mq_quantize_weight(None, 0, 4, 256, 256, 32, 1, None, 128, None, 4, None, 0, None) == -1
    assert "convrot group size" in _err(lib)
    assert lib.mq_quantize_weight(None, 0, 4, 65536, 65536, 256, 1, None, 32768, None, 1024, None, 0, None) == -1
    assert "32768" in _err(lib)
    assert lib.mq_quantize_weight(None, 0, 4, 256, 256, 256, 0, None, 128, None, 4, None, 2, None) == -1
    assert "null" in _err(lib)
    # N == 0 is a valid no-op
    assert lib.mq_quantize_weight(None, 2, 0, 256, 256, 256, 3, None, 256, None, 1, None, 0, None) == 0


def test_gemm_empty_shapes_are_noops(lib):
    # M == 0 or N == 0 passes the shape checks and touches nothing (null pointers are fine)
    assert lib.mq_gemm_w4_group(None, 64, None, None, 32, None, 1, None, 1, 64, 0, None, 0, None, 0, 8, 0, 8, 64, None) == 0
    assert lib.mq_gemm_w4_group(None, 64, None, None, 32, None, 1, None, 1, 64, 0, None, 0, None, 0, 8, 8, 0, 64, None) == 0
    assert lib.mq_gemm_rowscale(None, 64, None, None, 64, 8, None, None, 0, None, 0, 8, 0, 8, 64, None) == 0
    assert lib.mq_gemm_rowscale_acc(None, 64, None, 64, 8, None, 0, 8, 64, None) == 0
    assert lib.mq_gemm_w4_group_partials(None, 64, None, 32, None, 1, 64, 0, None, 0, 8, 64, None) == 0
    # shape checks still apply to empty products
    assert lib.mq_gemm_w4_group(None, 96, None, None, 48, None, 1, None, 1, 64, 0, None, 0, None, 0, 8, 0, 8, 96, None) == -1


def test_linear_validation_rejects_before_launch(lib):
    # (x, x_dtype, ldx, hblock, act_bits, swiglu, qw, ldw, ws, ldws, wz, ldwz, bias, bias_dtype, y,
    #  y_dtype, ldy, M, N, K, workspace, workspace_bytes, stream); fake aligned addresses are never
    # dereferenced: every case fails validation first
    a = 1 << 20
    need = 64 * 3072 + 256          # codes [64, 3072] and scales [64] (rounded up to 256 bytes)
    assert lib.mq_linear_workspace_bytes(64, 1024, 3072) >= need
    assert lib.mq_linear_workspace_bytes(0, 1024, 3072) == 0
    args = [a, 0, 3072, 256, 8, 0, a, 1536, a, 48, None, 0, None, 0, a, 0, 1024, 64, 1024, 3072, a, need, None]

    def call(**kw):
        names = ["x", "x_dtype", "ldx", "hblock", "act_bits", "swiglu", "qw", "ldw", "ws", "ldws", "wz", "ldwz",
                 "bias", "bias_dtype", "y", "y_dtype", "ldy", "M", "N", "K", "workspace", "workspace_bytes", "stream"]
        v = dict(zip(names, args))
        v.update(kw)
        return lib.mq_linear_w4_group(*[v[n] for n in names])

    assert call(act_bits=6) == -1 and "act_bits" in _err(lib)
    assert call(swiglu=3) == -1 and "swiglu" in _err(lib)
    assert call(K=3000) == -1 and "K % 64" in _err(lib)
    assert call(workspace=None) == -1 and "workspace" in _err(lib)
    assert call(workspace=a + 16) == -1 and "256-byte" in _err(lib)
    assert call(workspace_bytes=need - 1) == -1 and "codes and scales" in _err(lib)
    assert call(M=0) == 0 and call(N=0) == 0            # valid no-ops
    assert lib.mq_linear_rowscale(a, 0, 3072, 256, 5, 0, a, 3072, 8, a, None, 0, a, 0, 1024, 64, 1024, 3072, a,
                                  need, None) == -1
    assert "act_bits" in _err(lib)


def test_one_row_linear_validation_rejects_before_launch(lib):
    # M = 1: the GEMV quantizes the row itself, and the rotate+quantize entry's checks still run first
    a = 1 << 20
    need = lib.mq_linear_workspace_bytes(1, 1024, 3072)
    assert need >= 16 * 3072 + 4
    args = [a, 0, 3072, 256, 8, 0, a, 1536, a, 48, None, 0, None, 0, a, 0, 1024, 1, 1024, 3072, a, need, None]
    names = ["x", "x_dtype", "ldx", "hblock", "act_bits", "swiglu", "qw", "ldw", "ws", "ldws", "wz", "ldwz",
             "bias", "bias_dtype", "y", "y_dtype", "ldy", "M", "N", "K", "workspace", "workspace_bytes", "stream"]

    def call(**kw):
        v = dict(zip(names, args))
        v.update(kw)
        return lib.mq_linear_w4_group(*[v[n] for n in names])

    assert call(hblock=128) == -1 and "group size" in _err(lib)
    assert call(x=a + 2) == -1 and "16-byte" in _err(lib)
    assert call(x_dtype=7) == -1 and "input type" in _err(lib)
    assert call(workspace=None) == -1 and "workspace" in _err(lib)
    assert lib.mq_linear_rowscale(a, 0, 3072, 128, 8, 0, a, 3072, 8, a, None, 0, a, 0, 1024, 1, 1024, 3072, a,
                                  need, None) == -1
    assert "group size" in _err(lib)


def test_expanded_w4_validation(lib):
    # 4-bit weights expanded to int8 tiles: layouts 0 (int8 codes), 2 (x16 int4 codes), 3 (row scale)
    a = 1 << 20
    assert lib.mq_expand_weight_w4(a, 96, None, 0, a, 3, 8, 192, 1, a, None) == -1
    assert "layout" in _err(lib)
    assert lib.mq_expand_weight_w4(a, 104, None, 0, a, 4, 8, 200, 0, a, None) == -1
    assert "K % 64" in _err(lib)
    assert lib.mq_expand_weight_w4(a, 100, None, 0, a, 3, 8, 192, 0, a, None) == -1
    assert "ldw" in _err(lib)
    assert lib.mq_expand_weight_w4(a, 96, a, 1, a, 3, 8, 192, 2, a, None) == -1
    assert "ldwz" in _err(lib)
    # the group layouts carry the fp16 group scales (K/64 per row at least)
    assert lib.mq_expand_weight_w4(a, 96, None, 0, None, 3, 8, 192, 0, a, None) == -1
    assert "scales" in _err(lib)
    assert lib.mq_expand_weight_w4(a, 96, None, 0, a, 2, 8, 192, 2, a, None) == -1
    assert "scales" in _err(lib)
    assert lib.mq_expand_weight_w4(None, 96, None, 0, None, 0, 0, 192, 3, None, None) == 0
    # sizes: the int8 tiles, then (group layouts) 4 * ceil(K/256) groups x 16 x MQ_SCALE_PAIR_LD(N) dwords
    for n, k in ((8, 192), (16, 3072), (100, 1024), (12288, 3072)):
        tiles = (n + 15) // 16 * 16 * k
        ld = ((n + 15) // 16 + 17) // 2
        assert lib.mq_expanded_w4_bytes(n, k, 3) == tiles
        for layout in (0, 2):
            assert lib.mq_expanded_w4_bytes(n, k, layout) == tiles + (k // 64 + 3) // 4 * 4 * 16 * ld * 4
    # the group GEMMs take them for the int8 and x16 int4 activation layouts, K >= 192
    assert lib.mq_gemm_w4_group(a, 256, a, a, 0, a, 4, None, 0, 64, 1 | 0x100, None, 0, a, 0, 64, 8, 64, 256,
                                None) == -1
    assert "MQ_ACT_I8 and MQ_ACT_X16ALT" in _err(lib)
    assert lib.mq_gemm_w4_group(a, 128, a, a, 0, a, 2, None, 0, 64, 0x100, None, 0, a, 0, 64, 8, 64, 128, None) == -1
    assert "K >= 192" in _err(lib)
    assert lib.mq_gemm_w4_group_partials(a, 256, a, 128, None, 0, 64, 0x100, a, 8, 64, 256, None) == -1
    assert "act_mode" in _err(lib)
    # a GEMV-sized product (M <= 4) takes the packed weights: refused before anything is launched
    assert lib.mq_linear_w4_group(a, 0, 256, 256, 8 | 0x100, 0, a, 0, a, 4, a, 2, None, 0, a, 0, 64, 2, 64, 256, a,
                                  1 << 20, None) == -2
    assert "wide kernel only" in _err(lib)
