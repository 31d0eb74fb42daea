"""ctypes binding of libmq.so (C ABI in include/mq.h).

The library is loaded after `import torch`, so its `libamdhip64.so.7` dependency resolves to the
HIP runtime torch already mapped: device pointers, streams and the kernels share one runtime.
There is no fallback: if the library is missing, every call raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be imported before the library is loaded)

ABI_VERSION = 11
_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmq.so")

_lib = None

c_i64 = ctypes.c_int64
c_int = ctypes.c_int
c_vp = ctypes.c_void_p

_SIGNATURES = {
    "mq_abi_version": ([], c_int),
    "mq_last_error": ([], ctypes.c_char_p),
    "mq_rotquant": ([c_vp, c_int, c_i64, c_i64, c_i64, c_int, c_int, c_int, c_vp, c_i64, c_vp, c_vp], c_int),
    "mq_swiglu_rotquant": ([c_vp, c_int, c_i64, c_i64, c_i64, c_int, c_int, c_int, c_int, c_vp, c_i64, c_vp, c_vp],
                           c_int),
    "mq_decode_w4a8_codebook": ([c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_int, c_i64, c_i64, c_vp, c_i64, c_vp, c_vp],
                                c_int),
    "mq_quantize_weight": ([c_vp, c_int, c_i64, c_i64, c_i64, c_int, c_int, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp],
                           c_int),
    "mq_gemm_w4_group": ([c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_int, c_int, c_vp, c_int, c_vp,
                          c_int, c_i64, c_i64, c_i64, c_i64, c_vp], c_int),
    "mq_gemm_w4_group_ws": ([c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_int, c_int, c_vp, c_int, c_vp,
                             c_int, c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp], c_int),
    "mq_gemm_workspace_bytes": ([c_i64, c_i64, c_i64], c_i64),
    "mq_gemm_w4_group_partials": ([c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_int, c_int, c_vp, c_i64, c_i64, c_i64,
                                   c_vp], c_int),
    "mq_gemm_rowscale": ([c_vp, c_i64, c_vp, c_vp, c_i64, c_int, c_vp, c_vp, c_int, c_vp, c_int, c_i64, c_i64, c_i64,
                          c_i64, c_vp], c_int),
    "mq_gemm_rowscale_ws": ([c_vp, c_i64, c_vp, c_vp, c_i64, c_int, c_vp, c_vp, c_int, c_vp, c_int, c_i64, c_i64,
                             c_i64, c_i64, c_vp, c_i64, c_vp], c_int),
    "mq_tile_weight_i8": ([c_vp, c_i64, c_i64, c_i64, c_vp, c_vp], c_int),
    "mq_expand_weight_w4": ([c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_i64, c_i64, c_int, c_vp, c_vp], c_int),
    "mq_expanded_w4_bytes": ([c_i64, c_i64, c_int], c_i64),
    "mq_gemm_rowscale_acc": ([c_vp, c_i64, c_vp, c_i64, c_int, c_vp, c_i64, c_i64, c_i64, c_vp], c_int),
    "mq_linear_workspace_bytes": ([c_i64, c_i64, c_i64], c_i64),
    "mq_linear_w4_group": ([c_vp, c_int, c_i64, c_int, c_int, c_int, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp,
                            c_int, c_vp, c_int, c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp], c_int),
    "mq_linear_rowscale": ([c_vp, c_int, c_i64, c_int, c_int, c_int, c_vp, c_i64, c_int, c_vp, c_vp, c_int, c_vp,
                            c_int, c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp], c_int),
    "mq_linear_w4_group_noalloc": ([c_vp, c_int, c_i64, c_int, c_int, c_int, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64,
                                    c_vp, c_int, c_vp, c_int, c_i64, c_i64, c_i64, c_i64, c_vp], c_int),
}

EXPORTED = tuple(_SIGNATURES)

# code layouts (include/mq.h)
Q_BYTES, Q_PACKED, Q_X16ALT = 0, 1, 2
SWIGLU_NONE, SWIGLU_FUSED, SWIGLU_EAGER = 0, 1, 2
W8_TILE16 = 0x100            # wbits flag: int8 weights in 16-row tiles (include/mq.h)
ACT_I8, ACT_I4, ACT_X16ALT = 0, 1, 2
W4_EXPANDED = 0x100          # act_mode / act_bits flag: 4-bit weights expanded to int8 tiles
W4X_ROW = 3                  # mq_expand_weight_w4 layout for the row-scale GEMMs
DT_BF16, DT_F16, DT_F32 = 0, 1, 2
NOALLOC_SCRATCH_BYTES = 64 << 20   # MQ_NOALLOC_SCRATCH_BYTES
DTYPE_CODE = {torch.bfloat16: DT_BF16, torch.float16: DT_F16, torch.float32: DT_F32}


def dtype_code(dt) -> int:
    """MQ_DT_* code of a torch floating-point dtype (bf16, fp16, fp32)."""
    try:
        return DTYPE_CODE[dt]
    except KeyError:
        raise ValueError(f"unsupported floating-point type {dt}: expected bfloat16, float16 or float32") from None
WFMT_U4_ASYM_G64, WFMT_I4_SYM_G64, WFMT_I4_ROW, WFMT_I8_ROW = 0, 1, 2, 3


class MQError(RuntimeError):
    """A libmq entry point returned a failure status."""


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built: run `python comfy-quant-bench_amd/build.py` "
                           "(or __graft_entry__.build()) first; there is no CPU fallback")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (argtypes, restype) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    ver = lib.mq_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"libmq ABI version {ver}, expected {ABI_VERSION}: rebuild the library")
    _lib = lib
    return lib


def call(name: str, *args) -> None:
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.mq_last_error().decode(errors="replace")
        if rc == -1:
            raise ValueError(f"{name}: {msg}")
        raise MQError(f"{name} failed ({rc}): {msg}")


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for a missing optional operand)."""
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of_device(device) -> int:
    """hipStream_t of torch's current stream on a CUDA device (the stream every op enqueues on)."""
    if _raw_stream is not None:
        return _raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def stream_of(t: torch.Tensor) -> int:
    """hipStream_t of torch's current stream on t's device."""
    return stream_of_device(t.device)
