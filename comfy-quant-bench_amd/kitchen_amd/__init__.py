"""kitchen_amd: MI355X-native (gfx950) backend of the ComfyUI quantized-linear path.

A drop-in for the comfy-kitchen ops the reference calls on its W4A8 / W4A4 path
(`ck.convrot_w4a4_linear`, `ck.w4a8_int8_linear`, `ck.int8_linear`,
`ck.quantize_int4_rowwise_convrot64`, `ck.quantize_convrot_w4a4_weight`, ...): the same names and
keyword arguments, executed by hand-written HIP kernels in `libmq.so` through its C ABI
(include/mq.h). Host code is plain Python on PyTorch-ROCm; there is no CPU fallback.

    import kitchen_amd as ck
    y = ck.w4a8_int8_linear(x, qdata, s_rel, None, None, zeros, bias, 64, 256, torch.bfloat16)
"""
from . import weights
from ._lib import LIB_PATH, MQError, load
from .ops import (
    ExpandedW4,
    PreparedW4A8,
    convrot_w4a4_linear,
    decode_w4a8_codebook_weight,
    expand_w4_weight,
    gemm_rowscale,
    gemm_rowscale_acc,
    gemm_w4_group,
    gemm_w4_group_partials,
    int8_linear,
    int8_rowscale_linear,
    is_tile16,
    quantize_int4_rowwise_convrot64,
    quantize_int8_rowwise_convrot,
    release_expanded_weights,
    rotate_quantize,
    swiglu_quantize_int4_rowwise_convrot64,
    tile_int8_weight,
    w4a8_int8_linear,
)
from .weights import (
    quantize_convrot_w4a4_weight,
    quantize_int8_convrot_weight,
    quantize_w4a4_group_weight,
    quantize_w4a8_asym_weight,
)

__all__ = [
    "LIB_PATH", "MQError", "load", "weights",
    "convrot_w4a4_linear", "w4a8_int8_linear", "int8_linear", "int8_rowscale_linear", "PreparedW4A8",
    "ExpandedW4", "expand_w4_weight", "release_expanded_weights", "tile_int8_weight", "is_tile16",
    "quantize_int4_rowwise_convrot64", "quantize_int8_rowwise_convrot", "rotate_quantize",
    "swiglu_quantize_int4_rowwise_convrot64", "decode_w4a8_codebook_weight",
    "gemm_w4_group", "gemm_w4_group_partials", "gemm_rowscale", "gemm_rowscale_acc",
    "quantize_w4a8_asym_weight", "quantize_w4a4_group_weight", "quantize_convrot_w4a4_weight",
    "quantize_int8_convrot_weight",
]
