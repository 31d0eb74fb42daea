"""Online ops with comfy-kitchen's call surface, executed by libmq.so on the current HIP stream.

Names, keyword arguments and error messages follow the reference's contract:
  convrot_w4a4_linear(x, qweight, wscales, bias=None, convrot_groupsize=256, quant_group_size=64,
                      linear_dtype="int4", input_act=None)
      compile_support.py:84-113; patches/comfy_kitchen_swiglu_w4a4_fused.patch:41-67
  w4a8_int8_linear(x, qdata, s_rel, s_channel, codebook, correction, bias, group_size,
                   convrot_groupsize, out_dtype)
      kwargs pinned at tools/test_verify_formats.py:375-383
  int8_linear(x, weight, weight_scale, bias, out_dtype, convrot, convrot_groupsize, input_act)
      tools/verify_w4a4.py:342-370
  quantize_int4_rowwise_convrot64(x, convrot_groupsize) -> (qact int8 [M, K/2], x_scale f32 [M])
      patches/comfy_kitchen_swiglu_w4a4_fused.patch:37
  swiglu_quantize_int4_rowwise_convrot64(h) -> (qact int8 [M, K/2], x_scale f32 [M])
      tools/ck_swiglu/swiglu_quant.cu:111-120 (h = gate | up [M, 2K])
input_act="swiglu" takes x as the [gate | up] pair and folds silu(gate) * up into the activation
quantizer (patches/comfy_kitchen_swiglu_w4a4_fused.patch:17-33,60-63;
patches/comfyui_swiglu_triton_env.patch:65-97). The activation is rounded to x's type as the
reference rounds it: once (the fused quantizer) where comfy-kitchen fuses, i.e. convrot_w4a4_linear
with linear_dtype="int4", convrot_groupsize=256 and bf16 / fp16 input
(patches/comfy_kitchen_swiglu_w4a4_fused.patch:25-31), and in int8_linear (ComfyUI folds the
activation into the INT8 quantizer, patches/comfyui_swiglu_triton_env.patch:24,97-99; that
kernel's rounding is not in the reference tree); twice (silu(gate).mul_(up) in x's type,
patches/comfyui_swiglu_triton_env.patch:16-20) everywhere else convrot_w4a4_linear would apply it
eagerly (patches/comfy_kitchen_swiglu_w4a4_fused.patch:60-64), still inside the quantizer kernel;
other activations of ComfyUI's INPUT_ACT_EAGER table ("gelu_tanh",
patches/comfyui_swiglu_triton_env.patch:54-56) are applied eagerly first, as comfy-kitchen's
fallback `x = _apply_input_act(x, input_act)` does (patches/comfy_kitchen_swiglu_w4a4_fused.patch:60-64).
Activations are taken in their own type (bf16, fp16 or fp32: the rotation runs in fp32 from the
exact value) and outputs are written by the GEMM epilogue directly in the requested type, with the
bias in its own type; the reference writes out_dtype=x.dtype from its GEMM
(patches/comfy_kitchen_swiglu_w4a4_fused.patch:37-38).
Every op is a thin host wrapper: the caller's tensors are validated, outputs are allocated with
torch on the input's device, and the HIP kernels run asynchronously on the current stream.
"""
from __future__ import annotations

import os
import weakref

import torch

from . import _lib

INT4_GROUP_SIZE = 64
CONVROT_GROUPSIZES = (16, 64, 256)
FLOAT_TYPES = (torch.bfloat16, torch.float16, torch.float32)


def _as_2d(x: torch.Tensor, k: int) -> torch.Tensor:
    if not x.is_cuda:
        raise ValueError("kitchen_amd ops run on the GPU: x must be a device tensor")
    if x.dtype not in FLOAT_TYPES:
        raise ValueError(f"x must be bfloat16, float16 or float32, got {x.dtype}")
    # a contiguous 2-D x is what the reshape would return: used as it is (no new view per call)
    if x.dim() == 2 and x.shape[1] == k and x.stride(1) == 1 and x.stride(0) == k:
        return x
    return x.reshape(-1, k).contiguous()


def _bias(bias, n: int, device):
    """The bias on the device in its own floating-point type (bf16, fp16 or fp32), or None."""
    if bias is None:
        return None
    # already a contiguous [N] device vector of a float type: used as it is (no new tensor per call)
    if bias.dim() == 1 and bias.shape[0] == n and bias.device == device and bias.dtype in FLOAT_TYPES \
            and bias.stride(0) == 1:
        return bias
    if bias.numel() != n:
        raise ValueError(f"bias has {bias.numel()} elements, expected {n}")
    if bias.dtype not in FLOAT_TYPES:
        bias = bias.float()
    return bias.reshape(-1).to(device=device).contiguous()


def _out_dtype(out_dtype, x: torch.Tensor):
    dt = x.dtype if out_dtype is None else out_dtype
    if dt not in FLOAT_TYPES:
        raise ValueError(f"out_dtype must be bfloat16, float16 or float32, got {dt}")
    return dt


def _finish(y: torch.Tensor, x: torch.Tensor, n: int) -> torch.Tensor:
    return y if x.dim() == 2 else y.reshape(*x.shape[:-1], n)


# --------------------------------------------------------------------------- activation quantizers

def _swiglu_eager(h: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up in h's own type (ComfyUI's _swiglu_eager, patches/comfyui_swiglu_triton_env.patch:16-19)."""
    gate, up = h.chunk(2, dim=-1)
    return torch.nn.functional.silu(gate).mul_(up)


def rotate_quantize(x: torch.Tensor, convrot_groupsize: int | None, bits: int, packed: bool | int = False,
                    swiglu: bool | int = False):
    """Rotate x [.., K] by H_cg per block and quantize per token to int8 (bits 8) or int4 (bits 4).

    x: bfloat16, float16 or float32 (rotated in fp32 from its exact value).
    packed: False / Q_BYTES one code per byte, True / Q_PACKED packed int4 [M, K/2], Q_X16ALT the
    group GEMM's int4 operand layout (16 * q, negated in odd 64-column groups).
    swiglu: x is [.., 2K] = gate | up and the quantized activation is silu(gate) * up in x's type,
    rounded once (True / SWIGLU_FUSED: the fused quantizer) or twice (SWIGLU_EAGER:
    silu(gate).mul_(up)); bf16 / fp16 pairs are formed inside the kernel, fp32 pairs eagerly in fp32
    first (the reference's quantizer takes bf16 or fp16 only).
    Returns (q, scale): q int8 [M, K] or [M, K/2], scale float32 [M]."""
    layout = int(packed)
    mode = int(swiglu)
    if mode not in (_lib.SWIGLU_NONE, _lib.SWIGLU_FUSED, _lib.SWIGLU_EAGER):
        raise ValueError(f"swiglu must be False, True / SWIGLU_FUSED or SWIGLU_EAGER, got {swiglu!r}")
    width = x.shape[-1]
    if mode and width % 2:
        raise ValueError("h must hold gate | up halves")
    if mode and x.dtype == torch.float32:
        x, mode, width = _swiglu_eager(x), _lib.SWIGLU_NONE, width // 2
    k = width // 2 if mode else width
    x2 = _as_2d(x, width)
    m = x2.shape[0]
    q = torch.empty((m, k // 2 if layout == _lib.Q_PACKED else k), dtype=torch.int8, device=x2.device)
    s = torch.empty((m,), dtype=torch.float32, device=x2.device)
    if mode:
        _lib.call("mq_swiglu_rotquant", x2.data_ptr(), _lib.dtype_code(x2.dtype), m, k, width,
                  int(convrot_groupsize or 0), int(bits), layout, mode, q.data_ptr(), q.stride(0), s.data_ptr(),
                  _lib.stream_of(x2))
    else:
        _lib.call("mq_rotquant", x2.data_ptr(), _lib.dtype_code(x2.dtype), m, k, width, int(convrot_groupsize or 0),
                  int(bits), layout, q.data_ptr(), q.stride(0), s.data_ptr(), _lib.stream_of(x2))
    return q, s


INPUT_ACTS = ("swiglu", "gelu_tanh")


def _input_act(x: torch.Tensor, input_act: str | None):
    """(x for the quantizer, SwiGLU mode): "swiglu" folds into the quantizer (SWIGLU_FUSED; callers
    outside the reference's fused domain switch it to SWIGLU_EAGER); "gelu_tanh" is applied eagerly
    in x's type (ComfyUI's INPUT_ACT_EAGER entry, patches/comfyui_swiglu_triton_env.patch:54-56)
    before quantizing, the way comfy-kitchen falls back for activations it does not fuse."""
    if input_act is None:
        return x, _lib.SWIGLU_NONE
    if input_act == "swiglu":
        return x, _lib.SWIGLU_FUSED
    if input_act == "gelu_tanh":
        return torch.nn.functional.gelu(x, approximate="tanh"), _lib.SWIGLU_NONE
    raise ValueError(f"unknown input_act {input_act!r}: expected one of {INPUT_ACTS} or None")


def _swiglu_fused_domain(x: torch.Tensor, convrot_groupsize, linear_dtype: str) -> bool:
    """Whether comfy-kitchen's convrot_w4a4_linear fuses input_act="swiglu" into its quantizer
    (one rounding): int4 activations, convrot group 256, bf16 / fp16 input, K % 256 == 0 and
    K <= 16384 (patches/comfy_kitchen_swiglu_w4a4_fused.patch:25-31)."""
    k = x.shape[-1] // 2
    return (linear_dtype == "int4" and convrot_groupsize == 256 and x.dtype in (torch.bfloat16, torch.float16)
            and k % 256 == 0 and k <= 16384)


def quantize_int4_rowwise_convrot64(x: torch.Tensor, convrot_groupsize: int = 256):
    """comfy-kitchen's activation quantizer: (qact int8 [M, K/2] packed int4, x_scale f32 [M])."""
    return rotate_quantize(x, convrot_groupsize, 4, packed=True)


def swiglu_quantize_int4_rowwise_convrot64(h: torch.Tensor, convrot_groupsize: int = 256):
    """The fused SwiGLU quantizer of tools/ck_swiglu/swiglu_quant.cu:111-120: h [M, 2K] = gate | up,
    returns (qact int8 [M, K/2] packed int4, x_scale f32 [M]) of bf16(silu(gate) * up)."""
    k = h.shape[-1] // 2
    if k % 256 != 0 or k > 16384:
        raise ValueError("K must be a multiple of 256 and <= 16384")
    return rotate_quantize(h, convrot_groupsize, 4, packed=True, swiglu=True)


def quantize_int8_rowwise_convrot(x: torch.Tensor, convrot_groupsize: int | None = 256):
    """int8 sibling used inside w4a8_int8_linear / int8_linear: (q int8 [M, K], scale f32 [M])."""
    return rotate_quantize(x, convrot_groupsize, 8)


# --------------------------------------------------------------------------- shipped W4A8 decode

def _u8(t: torch.Tensor) -> torch.Tensor:
    """Raw bytes of an 8-bit tensor (int8, uint8 or float8_e4m3fn)."""
    if t.element_size() != 1:
        raise ValueError(f"expected an 8-bit tensor, got {t.dtype}")
    return t.contiguous().view(torch.uint8)


def decode_w4a8_codebook_weight(qdata: torch.Tensor, s_rel: torch.Tensor, s_channel: torch.Tensor,
                                codebook=None, group_size: int = 16):
    """Decode comfy-kitchen's shipped asym_w4a8_int8 weight (qdata I8 [N, K/2], s_rel fp8 e4m3fn
    or its U8 bytes [N, K/gs], s_channel F32 [N], codebook F32 [16] or None) to
    (q8 int8 [N, K], row_scale float32 [N]) for the int8 row-scale GEMM; the rule is in
    include/mq.h (mq_decode_w4a8_codebook)."""
    if not qdata.is_cuda:
        raise ValueError("kitchen_amd ops run on the GPU: qdata must be a device tensor")
    q = _u8(qdata)
    n, k = q.shape[0], q.shape[1] * 2
    sr = _u8(s_rel)
    if sr.shape != (n, k // group_size):
        raise ValueError(f"s_rel must be [{n}, {k // group_size}] for group_size {group_size}, got {list(sr.shape)}")
    sc = s_channel.reshape(-1).to(torch.float32).contiguous()
    if sc.numel() != n:
        raise ValueError(f"s_channel must have {n} elements, got {sc.numel()}")
    cb = None
    if codebook is not None:
        cb = codebook.reshape(-1).to(device=q.device, dtype=torch.float32).contiguous()
        if cb.numel() != 16:
            raise ValueError(f"codebook must have 16 levels, got {cb.numel()}")
    q8 = torch.empty((n, k), dtype=torch.int8, device=q.device)
    rs = torch.empty((n,), dtype=torch.float32, device=q.device)
    _lib.call("mq_decode_w4a8_codebook", q.data_ptr(), q.stride(0), sr.data_ptr(), sr.stride(0), sc.data_ptr(),
              _lib.ptr(cb), int(group_size), n, k, q8.data_ptr(), q8.stride(0), rs.data_ptr(), _lib.stream_of(q))
    return q8, rs


# --------------------------------------------------------------------------- GEMMs

def _check_w4_group(qa, qweight, wscales, wzeros, n, group_size):
    """Buffer-size checks the C ABI cannot do (it sees raw pointers)."""
    m, k = qa.shape
    if qa.dtype != torch.int8:
        raise ValueError("qa must be int8 [M, K]")
    _check_w4_group_weights(qweight, wscales, wzeros, n, k, group_size)


def _check_w4_group_weights(qweight, wscales, wzeros, n, k, group_size):
    if qweight is not None and (qweight.shape != (n, k // 2) or qweight.element_size() != 1):
        raise ValueError(f"qweight must be 8-bit [{n}, {k // 2}]")
    groups = k // group_size
    if wscales is not None and (wscales.dtype != torch.float16 or wscales.shape[0] != n
                                or wscales.shape[1] < groups or wscales.stride(1) != 1):
        raise ValueError(f"wscales must be float16 [{n}, {groups}] with unit column stride")
    if wzeros is not None and (wzeros.element_size() != 1 or wzeros.shape[0] != n
                               or wzeros.shape[1] < (groups + 1) // 2 or wzeros.stride(1) != 1):
        raise ValueError(f"zero-points must be packed uint4 [{n}, {(groups + 1) // 2}]")


_WS_BYTES: dict = {}

# Workspaces up to this size are kept per (device, stream) and reused by the next call on that
# stream (calls on one stream run in order, so they never overlap); larger ones, and every
# workspace taken while a HIP graph is being captured (the graph's own pool then holds it), are
# allocated per call.
WORKSPACE_CACHE_BYTES = 64 << 20
_WS_CACHE: dict = {}


def _scratch(nbytes: int, device) -> torch.Tensor:
    if nbytes > WORKSPACE_CACHE_BYTES or torch.cuda.is_current_stream_capturing():
        return torch.empty(nbytes, dtype=torch.uint8, device=device)
    key = (device.index, _lib.stream_of_device(device))
    buf = _WS_CACHE.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = _WS_CACHE[key] = torch.empty(nbytes, dtype=torch.uint8, device=device)
    return buf


def _workspace(m: int, n: int, k: int, device):
    """Split-K workspace for an M x N x K product when the library wants one (small M), else None.
    The size is asked of the library once per shape and device."""
    key = (device.index, m, n, k)
    nbytes = _WS_BYTES.get(key)
    if nbytes is None:
        with torch.cuda.device(device):
            nbytes = _WS_BYTES[key] = int(_lib.load().mq_gemm_workspace_bytes(m, n, k))
    return _scratch(nbytes, device) if nbytes > 0 else None


def _linear_workspace(m: int, n: int, k: int, device) -> torch.Tensor:
    """Workspace of the whole-linear entry points (activation codes, scales and split-K partials),
    its size asked of the library once per shape and device."""
    key = ("linear", device.index, m, n, k)
    nbytes = _WS_BYTES.get(key)
    if nbytes is None:
        with torch.cuda.device(device):
            nbytes = _WS_BYTES[key] = int(_lib.load().mq_linear_workspace_bytes(m, n, k))
    return _scratch(nbytes, device)


def _bias_args(bias):
    return (_lib.ptr(bias), _lib.DT_BF16 if bias is None else _lib.dtype_code(bias.dtype))


def gemm_w4_group(qa, sa, qweight, wscales, wzeros, bias, n: int, group_size: int = INT4_GROUP_SIZE,
                  act_mode: int = _lib.ACT_I8, out_dtype=torch.bfloat16):
    """y [M, N] = sa * sum_g wscales[:, g] * P_g + bias with P_g exact int32 group partials, written
    in out_dtype (bf16, fp16 or fp32); bias in its own floating-point type or None.

    act_mode: ACT_I8 int8 codes, ACT_I4 int4 codes one per byte, ACT_X16ALT the layout written by
    rotate_quantize(..., packed=Q_X16ALT). Small M splits K over a torch-allocated workspace.
    qweight may be the ExpandedW4 of the weights for act_mode (M > 4 rows; wzeros is then not read)."""
    m, k = qa.shape
    y = torch.empty((m, n), dtype=out_dtype, device=qa.device)
    work = _workspace(m, n, k, qa.device)
    if isinstance(qweight, ExpandedW4):
        if qweight.layout != act_mode or (qweight.n, qweight.k) != (n, k):
            raise ValueError(f"expanded weights for layout {qweight.layout} [{qweight.n}, {qweight.k}] "
                             f"do not serve act_mode {act_mode} [{n}, {k}]")
        _check_w4_group(qa, None, wscales, None, n, group_size)
        if qweight.scales != _scales_id(wscales):
            raise ValueError("expanded weights carry the group scales they were made with: pass the same wscales")
        qptr, ldw, mode = qweight.tiles.data_ptr(), k, int(act_mode) | _lib.W4_EXPANDED
        zptr, ldwz = (qweight.tiles.data_ptr() if qweight.asym else None), 0   # non-null: uint4 (not read)
    else:
        _check_w4_group(qa, qweight, wscales, wzeros, n, group_size)
        qptr, ldw, mode = qweight.data_ptr(), qweight.stride(0), int(act_mode)
        zptr, ldwz = _lib.ptr(wzeros), (wzeros.stride(0) if wzeros is not None else 0)
    _lib.call("mq_gemm_w4_group_ws", qa.data_ptr(), qa.stride(0), sa.data_ptr(), qptr, ldw, wscales.data_ptr(),
              wscales.stride(0), zptr, ldwz, int(group_size), mode, *_bias_args(bias), y.data_ptr(),
              _lib.dtype_code(out_dtype), y.stride(0), m, n, k, _lib.ptr(work), 0 if work is None else work.numel(),
              _lib.stream_of(qa))
    return y


def gemm_w4_group_partials(qa, qweight, wzeros, n: int, group_size: int = INT4_GROUP_SIZE,
                           act_mode: int = _lib.ACT_I8):
    """Parity entry: exact int32 partials P [K/G, M, N] of gemm_w4_group (of the codes themselves,
    whatever act_mode's scaling)."""
    m, k = qa.shape
    _check_w4_group(qa, qweight, None, wzeros, n, group_size)
    part = torch.empty((k // group_size, m, n), dtype=torch.int32, device=qa.device)
    ldwz = wzeros.stride(0) if wzeros is not None else 0
    _lib.call("mq_gemm_w4_group_partials", qa.data_ptr(), qa.stride(0), qweight.data_ptr(), qweight.stride(0),
              _lib.ptr(wzeros), ldwz, int(group_size), int(act_mode), part.data_ptr(), m, n, k, _lib.stream_of(qa))
    return part


def is_tile16(weight) -> bool:
    """True for int8 weights in the 16-row tile layout of tile_int8_weight."""
    return weight.dim() == 4 and tuple(weight.shape[2:]) == (16, 64)


def tile_int8_weight(weight: torch.Tensor) -> torch.Tensor:
    """int8 weights [N, K] -> the 16-row tile layout [ceil(N / 16), K / 64, 16, 64]
    (mq_tile_weight_i8): block [b, g] holds bytes 64 g .. 64 g + 63 of rows 16 b .. 16 b + 15, rows
    past N zero. The int8 row-scale linears and GEMMs take it in place of [N, K] (N is then the
    length of the row scale) with the same results bit for bit; every K group of the GEMM's weight
    loads is then whole cache lines. Prepare it once per weight. Needs K % 64 == 0 and K >= 192."""
    if weight.dim() != 2 or weight.element_size() != 1:
        raise ValueError(f"expected 8-bit weights [N, K], got {weight.dtype} {list(weight.shape)}")
    n, k = weight.shape
    w = weight if weight.stride(1) == 1 and weight.stride(0) % 16 == 0 else weight.contiguous()
    out = torch.empty(((n + 15) // 16, k // 64, 16, 64), dtype=torch.int8, device=weight.device)
    _lib.call("mq_tile_weight_i8", w.data_ptr(), w.stride(0), n, k, out.data_ptr(), _lib.stream_of(w))
    return out


# --------------------------------------------------------------------------- expanded 4-bit weights

class ExpandedW4:
    """Packed 4-bit weights expanded once to int8 in 16-row tiles (mq_expand_weight_w4).

    tiles   int8 [ceil(N / 16), K / 64, 16, 64], the front of the expansion's buffer
    layout  _lib.ACT_I8 / _lib.ACT_X16ALT: for the group GEMMs with that activation layout (the
            bytes their in-kernel unpack would store, zero-point and sign included), with the
            weight's fp16 group scales carried after the tiles in the layout the GEMM's lanes read;
            _lib.W4X_ROW: an int8 weight for the row-scale GEMMs (the signed codes)
    asym    uint4 weights with zero-points (folded into the bytes) rather than signed int4
    scales  (data_ptr, shape, stride) of the group scales the expansion carries (None for W4X_ROW):
            the group GEMMs take the same tensor as wscales, for their epilogue's correction term
The GEMMs give the packed weights' results bit for bit from it, without the per-use unpack, at
twice the packed weight's memory."""

    __slots__ = ("tiles", "buf", "layout", "asym", "n", "k", "scales")

    def __init__(self, buf: torch.Tensor, layout: int, asym: bool, n: int, k: int, scales=None):
        self.buf = buf
        self.tiles = buf[: (n + 15) // 16 * 16 * k].view(torch.int8).view((n + 15) // 16, k // 64, 16, 64)
        self.layout, self.asym, self.n, self.k, self.scales = int(layout), bool(asym), int(n), int(k), scales


def _scales_id(wscales):
    return (wscales.data_ptr(), tuple(wscales.shape), tuple(wscales.stride()))


def expand_w4_weight(qweight: torch.Tensor, wzeros=None, layout: int = _lib.ACT_I8, wscales=None) -> ExpandedW4:
    """qweight 8-bit [N, K/2] packed 4-bit codes (uint4 with wzeros packed uint4 [N, ceil(K/128)],
    or signed int4 when wzeros is None) -> ExpandedW4 for `layout` (see ExpandedW4); the group
    layouts take the weight's fp16 group scales wscales [N, K/64]."""
    if qweight.dim() != 2 or qweight.element_size() != 1:
        raise ValueError(f"qweight must be 8-bit [N, K/2], got {qweight.dtype} {list(qweight.shape)}")
    if layout not in (_lib.ACT_I8, _lib.ACT_X16ALT, _lib.W4X_ROW):
        raise ValueError(f"layout must be ACT_I8, ACT_X16ALT or W4X_ROW, got {layout}")
    n, k = qweight.shape[0], qweight.shape[1] * 2
    qw = qweight if qweight.stride(1) == 1 and qweight.stride(0) % 8 == 0 else qweight.contiguous()
    zz = None
    if wzeros is not None:
        if wzeros.element_size() != 1 or wzeros.shape[0] != n or wzeros.shape[1] < (k // 64 + 1) // 2:
            raise ValueError(f"zero-points must be packed uint4 [{n}, {(k // 64 + 1) // 2}]")
        zz = wzeros if wzeros.stride(1) == 1 else wzeros.contiguous()
    ws = None
    if layout != _lib.W4X_ROW:
        if wscales is None or wscales.dtype != torch.float16 or wscales.dim() != 2 or wscales.shape[0] != n \
                or wscales.shape[1] < k // 64 or wscales.stride(1) != 1:
            raise ValueError(f"the group layouts need the fp16 group scales [{n}, {k // 64}] (unit column stride)")
        ws = wscales
    nbytes = _lib.load().mq_expanded_w4_bytes(n, k, int(layout))
    buf = torch.empty(nbytes, dtype=torch.uint8, device=qweight.device)
    _lib.call("mq_expand_weight_w4", qw.data_ptr(), qw.stride(0), _lib.ptr(zz), 0 if zz is None else zz.stride(0),
              _lib.ptr(ws), 0 if ws is None else ws.stride(0), n, k, int(layout), buf.data_ptr(), _lib.stream_of(qw))
    return ExpandedW4(buf, layout, zz is not None, n, k, None if ws is None else _scales_id(ws))


# The linears run their 4-bit weights from an int8 expansion wherever the packed weights would run
# on the wide kernel too, so that the results are the same bits either way: group scales above 128
# rows (fewer rows run on the 128 x 128 few-row kernel, whose group epilogue rounds differently),
# row scales above the GEMV's 4 rows (exact int32 sums on every kernel). The GEMV reads the packed
# bytes: it is bound by their HBM traffic. The expansion is made on a weight's first such call and
# kept until the tensor it was made from (its base tensor, for a view) is freed, for as long as that
# weight's storage and version are unchanged; it costs 1 byte per weight element beside the packed
# 0.5 (release_expanded_weights() drops them all). A HIP graph that captured a linear keeps the
# expansion it captured: re-capture after changing a weight in place. KITCHEN_AMD_EXPAND_W4=0 (or
# EXPAND_W4 = False) keeps every call on the packed weights.
EXPAND_W4 = os.environ.get("KITCHEN_AMD_EXPAND_W4", "1") != "0"
GEMV_ROWS = 4
FEW_ROWS = 128
_EXPANDED: dict = {}


def _expansion(qweight, wzeros, layout: int, m: int, k: int, wscales=None):
    """The cached ExpandedW4 of qweight for `layout` when a product of m rows reads one (the wide
    kernel's conditions: K >= 192, K groups in pairs for the group scales' loads, under 2 GiB;
    the group layouts also carry wscales, fp16 with unit column stride), else None."""
    n = qweight.shape[0]
    if not EXPAND_W4 or m <= (GEMV_ROWS if layout == _lib.W4X_ROW else FEW_ROWS) or k < 192 or k % 64 \
            or _lib.load().mq_expanded_w4_bytes(n, k, int(layout)) >= 1 << 31 or (m + 15) // 16 * 16 * k >= 1 << 31:
        return None
    if wscales is not None and (wscales.stride(0) % 2 or wscales.data_ptr() % 4 or wscales.stride(1) != 1
                                or wscales.dtype != torch.float16):
        return None
    root = qweight._base if qweight._base is not None else qweight
    zroot = None if wzeros is None else (wzeros._base if wzeros._base is not None else wzeros)
    if layout != _lib.W4X_ROW and wscales is None:
        return None
    key = (qweight.data_ptr(), tuple(qweight.shape), tuple(qweight.stride()),
           0 if wzeros is None else wzeros.data_ptr(), int(layout),
           None if layout == _lib.W4X_ROW else _scales_id(wscales))
    sig = (qweight._version, 0 if wzeros is None else wzeros._version, id(zroot),
           0 if layout == _lib.W4X_ROW else wscales._version)
    per = _EXPANDED.get(id(root))
    hit = None if per is None else per.get(key)
    if hit is not None and hit[0] == sig:
        return hit[1]
    if torch.cuda.is_current_stream_capturing():
        return None   # nothing is allocated under capture: the packed weights, unless expanded before
    if per is None:
        per = _EXPANDED[id(root)] = {}
        weakref.finalize(root, _EXPANDED.pop, id(root), None)
    ex = expand_w4_weight(qweight, wzeros, layout, None if layout == _lib.W4X_ROW else wscales)
    per[key] = (sig, ex)
    return ex


def release_expanded_weights() -> int:
    """Drop every cached int8 expansion of 4-bit weights (they are made again on their weights'
    next large-M calls); returns how many were held."""
    held = sum(len(per) for per in _EXPANDED.values())
    _EXPANDED.clear()
    return held


def _weight_args(qweight, n: int, k: int, wbits: int):
    """(ldw, wbits) of the row-scale entries for [N, K'] rows or the 16-row tile layout."""
    if isinstance(qweight, ExpandedW4):
        if qweight.layout != _lib.W4X_ROW or (qweight.n, qweight.k) != (n, k):
            raise ValueError("the row-scale GEMMs take the W4X_ROW expansion of an [N, K/2] weight")
        return k, 8 | _lib.W8_TILE16
    if is_tile16(qweight):
        if wbits != 8 or qweight.element_size() != 1:
            raise ValueError("the 16-row tile layout holds int8 weights (wbits 8)")
        if tuple(qweight.shape) != ((n + 15) // 16, k // 64, 16, 64) or not qweight.is_contiguous():
            raise ValueError(f"16-row tile weights for N={n} K={k} must be contiguous "
                             f"[{(n + 15) // 16}, {k // 64}, 16, 64], got {list(qweight.shape)}")
        return k, wbits | _lib.W8_TILE16
    return qweight.stride(0), wbits


def gemm_rowscale(qa, sa, qweight, wscales, bias, n: int, wbits: int, out_dtype=torch.bfloat16):
    """y [M, N] = (qa . w^T) * sa[m] * wscales[n] + bias in out_dtype, full-K int32 accumulator (split
    over K into int32 partial sums for small M, summed exactly)."""
    m, k = qa.shape
    y = torch.empty((m, n), dtype=out_dtype, device=qa.device)
    work = _workspace(m, n, k, qa.device)
    ldw, wb = _weight_args(qweight, n, k, int(wbits))
    _lib.call("mq_gemm_rowscale_ws", qa.data_ptr(), qa.stride(0), sa.data_ptr(), qweight.data_ptr(),
              ldw, wb, wscales.data_ptr(), *_bias_args(bias), y.data_ptr(),
              _lib.dtype_code(out_dtype), y.stride(0), m, n, k, _lib.ptr(work), 0 if work is None else work.numel(),
              _lib.stream_of(qa))
    return y


def gemm_rowscale_acc(qa, qweight, n: int, wbits: int):
    """Parity entry: the full-K int32 accumulator [M, N] of gemm_rowscale."""
    m, k = qa.shape
    acc = torch.empty((m, n), dtype=torch.int32, device=qa.device)
    ldw, wb = _weight_args(qweight, n, k, int(wbits))
    _lib.call("mq_gemm_rowscale_acc", qa.data_ptr(), qa.stride(0), qweight.data_ptr(), ldw, wb, acc.data_ptr(),
              m, n, k, _lib.stream_of(qa))
    return acc


# --------------------------------------------------------------------------- linears

def convrot_w4a4_linear(x: torch.Tensor, qweight: torch.Tensor, wscales: torch.Tensor, bias=None,
                        convrot_groupsize: int = 256, quant_group_size: int = INT4_GROUP_SIZE,
                        linear_dtype: str = "int4", input_act: str | None = None) -> torch.Tensor:
    """``act(x) @ W.T + bias`` with ConvRot W4A4 weights, written in x's type.

    qweight int8 [N, K/2] holds signed int4 (low nibble = even k). wscales is either the shipped
    per-row F32 [N] scale (full-K int32 accumulation) or the configs' per-group fp16 [N, K/64]
    scale. linear_dtype "int4" quantizes activations to int4, "int8" to int8."""
    if linear_dtype not in {"int4", "int8"}:
        raise ValueError(f"ConvRot W4A4 linear_dtype must be 'int4' or 'int8', got {linear_dtype!r}")
    if quant_group_size != INT4_GROUP_SIZE:
        raise ValueError(f"int4 MMA kernel requires quant_group_size {INT4_GROUP_SIZE}")
    x_out = x
    x, swiglu = _input_act(x, input_act)
    if swiglu and not _swiglu_fused_domain(x, convrot_groupsize, linear_dtype):
        swiglu = _lib.SWIGLU_EAGER           # comfy-kitchen's eager fallback: two roundings
    k = x.shape[-1] // 2 if swiglu else x.shape[-1]
    if k != qweight.shape[-1] * 2:
        raise ValueError(f"Input K={k} does not match qweight K={qweight.shape[-1] * 2}")
    if k % convrot_groupsize != 0:
        raise ValueError(f"Input K={k} is not divisible by convrot_groupsize={convrot_groupsize}")
    n = qweight.shape[0]
    bits = 4 if linear_dtype == "int4" else 8
    out_dtype = _out_dtype(None, x_out)
    if wscales.dim() == 2 and wscales.shape[1] > 1:
        if wscales.shape != (n, k // quant_group_size):
            raise ValueError(f"per-group wscales must be [{n}, {k // quant_group_size}], got {list(wscales.shape)}")
        ws = wscales.to(torch.float16).contiguous()
        y = _linear_w4_group(x, swiglu, convrot_groupsize, bits, qweight, ws, None, bias, n, k, out_dtype)
    else:
        ws = wscales.reshape(-1).to(torch.float32).contiguous()
        if ws.numel() != n:
            raise ValueError(f"per-row wscales must have {n} elements, got {ws.numel()}")
        y = _linear_rowscale(x, swiglu, convrot_groupsize, bits, qweight, 4, ws, bias, n, k, out_dtype)
    return _finish(y, x_out, n)


def _linear_input(x: torch.Tensor, swiglu: int, k: int):
    """(x as [M, width] for the whole-linear entry points, SwiGLU mode): fp32 gate | up pairs are
    formed eagerly (the SwiGLU prologue takes bf16 / fp16, as the reference's does)."""
    if swiglu and x.dtype == torch.float32:
        x, swiglu = _swiglu_eager(x), _lib.SWIGLU_NONE
    x2 = _as_2d(x, 2 * k if swiglu else k)
    return x2, swiglu


def _linear_w4_group(x, swiglu, cg, act_bits, qweight, wscales, wzeros, bias, n, k, out_dtype):
    """rotate + quantize + group GEMM in one library call (mq_linear_w4_group)."""
    x2, swiglu = _linear_input(x, swiglu, k)
    m = x2.shape[0]
    _check_w4_group_weights(qweight, wscales, wzeros, n, k, INT4_GROUP_SIZE)
    b = _bias(bias, n, x2.device)
    y = torch.empty((m, n), dtype=out_dtype, device=x2.device)
    if m == 0:
        return y
    work = _linear_workspace(m, n, k, x2.device)
    xw = _expansion(qweight, wzeros, _lib.ACT_X16ALT if act_bits == 4 else _lib.ACT_I8, m, k, wscales)
    if xw is not None:
        qptr, ldw, ab = xw.tiles.data_ptr(), k, int(act_bits) | _lib.W4_EXPANDED
        zptr, ldwz = (xw.tiles.data_ptr() if xw.asym else None), 0   # non-null: uint4 (not read)
    else:
        qw = qweight.contiguous()
        zz = None if wzeros is None else wzeros.contiguous()
        qptr, ldw, ab = qw.data_ptr(), qw.stride(0), int(act_bits)
        zptr, ldwz = _lib.ptr(zz), (0 if zz is None else zz.stride(0))
    _lib.call("mq_linear_w4_group", x2.data_ptr(), _lib.dtype_code(x2.dtype), x2.stride(0), int(cg or 0), ab,
              int(swiglu), qptr, ldw, wscales.data_ptr(), wscales.stride(0), zptr, ldwz, *_bias_args(b),
              y.data_ptr(), _lib.dtype_code(out_dtype), y.stride(0), m, n, k, work.data_ptr(), work.numel(),
              _lib.stream_of(x2))
    return y


def _linear_rowscale(x, swiglu, cg, act_bits, qweight, wbits, wscales, bias, n, k, out_dtype):
    """rotate + quantize + row-scale GEMM in one library call (mq_linear_rowscale)."""
    x2, swiglu = _linear_input(x, swiglu, k)
    m = x2.shape[0]
    qw = qweight if is_tile16(qweight) else qweight.contiguous()
    wbytes = k // 2 if wbits == 4 else k
    if not is_tile16(qw) and (qw.shape != (n, wbytes) or qw.element_size() != 1):
        raise ValueError(f"weight must be 8-bit [{n}, {wbytes}]")
    if wbits == 4:
        # signed int4 rows: their int8 expansion where the wide kernel reads it (same int32 sums)
        xw = _expansion(qweight, None, _lib.W4X_ROW, m, k)
        if xw is not None:
            qw, wbits = xw.tiles, 8
    ldw, wbits = _weight_args(qw, n, k, int(wbits))
    b = _bias(bias, n, x2.device)
    y = torch.empty((m, n), dtype=out_dtype, device=x2.device)
    if m == 0:
        return y
    work = _linear_workspace(m, n, k, x2.device)
    _lib.call("mq_linear_rowscale", x2.data_ptr(), _lib.dtype_code(x2.dtype), x2.stride(0), int(cg or 0),
              int(act_bits), int(swiglu), qw.data_ptr(), ldw, wbits, wscales.data_ptr(), *_bias_args(b),
              y.data_ptr(), _lib.dtype_code(out_dtype), y.stride(0), m, n, k, work.data_ptr(), work.numel(),
              _lib.stream_of(x2))
    return y


# Shipped asym_w4a8_int8 weights decoded to (int8 [N, K], row scale [N]) once per weight: one entry
# per packed-weight tensor object, valid while the operands' storage and versions are unchanged,
# dropped when that tensor is freed.
_DECODED: dict = {}


def _decoded_w4a8(qdata, s_rel, s_channel, codebook, group_size):
    sig = (qdata.data_ptr(), qdata._version, s_rel.data_ptr(), s_rel._version, s_channel.data_ptr(),
           s_channel._version, 0 if codebook is None else codebook.data_ptr(),
           0 if codebook is None else codebook._version, int(group_size))
    qid = id(qdata)
    hit = _DECODED.get(qid)
    if hit is not None and hit[0] == sig:
        return hit[1]
    dec = decode_w4a8_codebook_weight(qdata, s_rel, s_channel, codebook, group_size)
    if hit is None:
        weakref.finalize(qdata, _DECODED.pop, qid, None)
    _DECODED[qid] = (sig, dec)
    return dec


class PreparedW4A8:
    """A shipped asym_w4a8_int8 weight decoded once (at load) to the int8 weight and per-row scale
    the row-scale GEMM takes; calling it runs only rotate + quantize and the int8 GEMM."""

    def __init__(self, qdata, s_rel, s_channel, codebook=None, group_size: int = 16, convrot_groupsize: int = 256):
        q8, self.row_scale = decode_w4a8_codebook_weight(qdata, s_rel, s_channel, codebook, group_size)
        self.n, self.k = q8.shape
        # held in 16-row tiles where the GEMM takes them (same results, whole-line weight loads)
        self.q8 = tile_int8_weight(q8) if self.k >= 192 and self.k % 64 == 0 else q8
        self.convrot_groupsize = convrot_groupsize

    def __call__(self, x, bias=None, out_dtype=None):
        return int8_rowscale_linear(x, self.q8, self.row_scale, bias, out_dtype, self.convrot_groupsize)


def int8_rowscale_linear(x, q8, row_scale, bias=None, out_dtype=None, convrot_groupsize: int | None = 256,
                         input_act: str | None = None):
    """The W8A8 linear the decoded W4A8 weights and int8_tensorwise share: rotate + int8 per-token
    quantize, then the int8 row-scale GEMM."""
    x_out = x
    x, swiglu = _input_act(x, input_act)
    k = x.shape[-1] // 2 if swiglu else x.shape[-1]
    # [N, K] rows, or the 16-row tile layout of tile_int8_weight (N = the row scale's length)
    n = row_scale.numel() if is_tile16(q8) else q8.shape[0]
    kw = q8.shape[1] * 64 if is_tile16(q8) else q8.shape[1]
    if kw != k:
        raise ValueError(f"Input K={k} does not match weight K={kw}")
    if convrot_groupsize and k % convrot_groupsize:
        raise ValueError(f"Input K={k} is not divisible by convrot_groupsize={convrot_groupsize}")
    ws = row_scale.reshape(-1).to(torch.float32).contiguous()
    if ws.numel() != n:
        raise ValueError(f"row scale must have {n} elements, got {ws.numel()}")
    y = _linear_rowscale(x, swiglu, convrot_groupsize, 8, q8, 8, ws, bias, n, k, _out_dtype(out_dtype, x_out))
    return _finish(y, x_out, n)


def w4a8_int8_linear(x: torch.Tensor, qdata: torch.Tensor, s_rel: torch.Tensor, s_channel=None, codebook=None,
                     correction=None, bias=None, group_size: int = INT4_GROUP_SIZE, convrot_groupsize: int = 256,
                     out_dtype=torch.bfloat16) -> torch.Tensor:
    """W4A8 linear: H_cg rotation + int8 per-token activations + 4-bit weights. Two layouts:

    * configs' scheme (uint4 asymmetric per group): qdata uint8 [N, K/2] packed codes, s_rel fp16
      [N, K/group] per-group scales, correction uint8 [N, ceil(K/group/2)] packed uint4
      zero-points (None = signed int4 weights), s_channel and codebook None; group GEMM.
    * comfy-kitchen's shipped asym_w4a8_int8 (tools/_formats.py:79-125): qdata I8 [N, K/2] codes,
      s_rel fp8 e4m3fn (or its U8 bytes) [N, K/group], s_channel F32 [N], codebook F32 [16] or
      None, no correction; the weight is decoded to int8 with a per-row scale once (cached per
      weight tensor; PreparedW4A8 holds it explicitly) and runs on the int8 row-scale GEMM."""
    k = x.shape[-1]
    if k != qdata.shape[-1] * 2:
        raise ValueError(f"Input K={k} does not match qdata K={qdata.shape[-1] * 2}")
    if convrot_groupsize and k % convrot_groupsize:
        raise ValueError(f"Input K={k} is not divisible by convrot_groupsize={convrot_groupsize}")
    n = qdata.shape[0]
    if s_channel is not None or codebook is not None or s_rel.element_size() == 1:
        if correction is not None:
            raise NotImplementedError("asym_w4a8_int8 with a correction tensor (asymmetric) is not supported; "
                                      "the reference's loader drops it as well")
        if s_channel is None:
            raise ValueError("the shipped asym_w4a8_int8 layout needs s_channel")
        q8, rs = _decoded_w4a8(qdata, s_rel, s_channel, codebook, group_size)
        return int8_rowscale_linear(x, q8, rs, bias, out_dtype, convrot_groupsize)
    if s_rel.dtype != torch.float16:
        raise ValueError(f"per-group s_rel must be float16 (configs' scheme) or fp8 bytes, got {s_rel.dtype}")
    if group_size != INT4_GROUP_SIZE:
        raise ValueError(f"W4A8 kernel requires group_size {INT4_GROUP_SIZE}, got {group_size}")
    if s_rel.shape != (n, k // group_size):
        raise ValueError(f"s_rel must be [{n}, {k // group_size}], got {list(s_rel.shape)}")
    if correction is not None and correction.shape != (n, (k // group_size + 1) // 2):
        raise ValueError(f"correction (zero-points) must be [{n}, {(k // group_size + 1) // 2}]")
    qw = qdata if qdata.dtype == torch.uint8 else qdata.view(torch.uint8)
    zz = correction
    if zz is not None and zz.dtype != torch.uint8:
        zz = zz.view(torch.uint8)
    y = _linear_w4_group(x, False, convrot_groupsize, 8, qw, s_rel.contiguous(), zz, bias, n, k,
                         _out_dtype(out_dtype, x))
    return _finish(y, x, n)


def int8_linear(x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor, bias=None,
                out_dtype=torch.bfloat16, convrot: bool = False, convrot_groupsize: int = 256,
                input_act: str | None = None) -> torch.Tensor:
    """int8_tensorwise linear: int8 per-row weights [N, K] + F32 scale [N, 1], int8 per-token
    activations (after H_cg when convrot), full-K int32 accumulation."""
    return int8_rowscale_linear(x, weight, weight_scale, bias, out_dtype, convrot_groupsize if convrot else None,
                                input_act)
