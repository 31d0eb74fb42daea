/*
 * mq.h - C ABI of libmq.so, the MI355X (gfx950) quantized-linear library.
 *
 * Every entry point takes raw device pointers, sizes and a hipStream_t (passed as void*),
 * enqueues its kernels on that stream and returns immediately. The caller allocates every
 * buffer; no entry point allocates device memory. Global state: a per-device cache of the compute
 * unit count and of kernel occupancies (filled once, read-only afterwards, guarded for concurrent
 * first use), the thread-local error message, and the fixed per-device scratch array behind
 * mq_linear_w4_group_noalloc (with the cached device address of each GPU's copy). Concurrent calls
 * from several threads are safe, except mq_linear_w4_group_noalloc calls that overlap on one GPU:
 * they share its scratch array and race. Return value: MQ_OK (0) or a negative MQ_E* code; the
 * message of the last failure on the calling thread is returned by mq_last_error().
 *
 * Layout conventions (all row-major, strides in elements of the stated type):
 *   floating-point operands whose type the caller chooses (activations, bias, outputs, weights to
 *   quantize) are passed as void pointers with an MQ_DT_* type code; bf16 / fp16 are their bit
 *   patterns. Scales keep fixed types (fp32 per token / per row, fp16 per weight group).
 *   int4 packing: byte j of a row holds k = 2j in bits 0-3 and k = 2j + 1 in bits 4-7
 *   (experiments/qwen21-kernel/node/__init__.py:82-86; custom_nodes/comfy-lowbit-loader/
 *   kernel.py:75-81 for the unsigned form). Signed nibbles decode as v >= 8 -> v - 16.
 *   Hadamard blocks: 0 (no rotation), 16, 64 or 256; H_b = (H4/2)^(x log4 b) applied to each
 *   block of b consecutive columns with the fp32 radix-4 FWHT of
 *   experiments/qwen21-kernel/kernels/g64_quant.cu:68-86 (strides 1, 4, 16, 64 in that order).
 */
#ifndef MQ_H
#define MQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MQ_ABI_VERSION 11

enum {
    MQ_OK = 0,
    MQ_EINVAL = -1,       /* bad shape, stride, alignment or argument */
    MQ_EUNSUPPORTED = -2, /* valid request outside what this build implements */
    MQ_ELAUNCH = -3,      /* the HIP runtime refused a launch */
};

/* Element types of the floating-point operands (the *_dtype arguments). */
#define MQ_DT_BF16 0
#define MQ_DT_F16 1
#define MQ_DT_F32 2

/* Layouts of the activation codes written by mq_rotquant (its `packed` argument). */
enum {
    MQ_Q_BYTES = 0,    /* one code per byte: int8 codes (bits 8) or int4 codes in [-7, 7] (bits 4) */
    MQ_Q_PACKED = 1,   /* int4 codes packed two per byte, low nibble = even k (bits 4) */
    MQ_Q_X16ALT = 2,   /* int4 codes one per byte as 16 * q, negated in odd 64-column groups (bits 4):
                          the operand layout of the group GEMMs for int4 activations (MQ_ACT_X16ALT) */
};

/* SwiGLU prologue modes (the `mode` of mq_swiglu_rotquant, the `swiglu` of the whole linears). */
#define MQ_SWIGLU_NONE 0    /* whole linears: x is the activation itself                            */
#define MQ_SWIGLU_FUSED 1   /* T(silu(g) * u): fp32 product rounded once to the input type T, as the */
                            /* fused quantizer (tools/ck_swiglu/swiglu_quant.cu:56-70)               */
#define MQ_SWIGLU_EAGER 2   /* T(T(silu(g)) * u): silu rounded to T, then the product rounded again, */
                            /* as the eager silu(gate).mul_(up) in T                                 */
                            /* (patches/comfyui_swiglu_triton_env.patch:16-20)                      */

/* Layouts of the activation codes qa taken by the group-scale GEMMs (their `act_mode`). */
enum {
    MQ_ACT_I8 = 0,       /* int8 per-token codes (int8 range) */
    MQ_ACT_I4 = 1,       /* int4 codes in [-8, 7], one per byte (scaled by 16 inside the kernel) */
    MQ_ACT_X16ALT = 2,   /* layout MQ_Q_X16ALT of mq_rotquant */
};

/* ABI version this library was built with (MQ_ABI_VERSION). */
int mq_abi_version(void);

/* Message of the last failure on the calling thread ("" if none). */
const char* mq_last_error(void);

/*
 * Rotate + per-token dynamic quantize the activations of one linear.
 *
 * Replaces comfy-kitchen's quantize_int4_rowwise_convrot64(x, cg) as called at
 * patches/comfy_kitchen_swiglu_w4a4_fused.patch:37 and its int8 sibling inside
 * w4a8_int8_linear (tools/quant_mixed.py:315-317); arithmetic per tools/activation_balance.py:65-71:
 *   xr = x rotated by H_hblock per block of hblock columns (fp32, pinned FWHT order),
 *   s[m] = max(max_k |xr[m,k]| / L, 1e-10f), q[m,k] = clamp(rne(xr[m,k] / s[m]), -L, L),
 * with L = 127 for bits = 8 and L = 7 for bits = 4. The division is IEEE fp32.
 *
 *   x      [M, K] of type x_dtype (MQ_DT_BF16, MQ_DT_F16 or MQ_DT_F32; the 16-bit types convert
 *          exactly to fp32, the type the rotation runs in), row stride ldx elements (a multiple of
 *          16 bytes, 16-byte aligned base)
 *   bits   8 or 4
 *   packed MQ_Q_BYTES: q is int8 [M, K] (one code per byte, stride ldq bytes)
 *          MQ_Q_PACKED: q is int8 [M, K/2] packed int4 (bits must be 4, stride ldq bytes)
 *          MQ_Q_X16ALT: q is int8 [M, K], 16 * code, negated where (k / 64) is odd (bits 4)
 *   scale  fp32 [M]
 * Requires K % 16 == 0, K <= 16384, K % hblock == 0.
 */
int mq_rotquant(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, int hblock, int bits, int packed,
                void* q, int64_t ldq, float* scale, void* stream);

/*
 * SwiGLU prologue fused into rotate + quantize: the activation is, by mode,
 *   MQ_SWIGLU_FUSED  a[m,k] = T( silu(h[m,k]) * h[m,K+k] )        (fp32 product, one rounding)
 *   MQ_SWIGLU_EAGER  a[m,k] = T( T(silu(h[m,k])) * h[m,K+k] )     (two roundings)
 * with T = h_dtype, formed while loading the gate | up row, then rotated and quantized exactly as
 * mq_rotquant does with x = a. The intermediate never touches memory.
 *
 * FUSED replaces swiglu_quantize_int4_rowwise_convrot64(h) (tools/ck_swiglu/swiglu_quant.cu:23-97
 * and :111-120), which rounds the fp32 product once to the input type (:63-70,124-132);
 * comfy-kitchen takes it for convrot_w4a4_linear(..., input_act="swiglu") only with
 * linear_dtype="int4", convrot_groupsize=256 and bf16 / fp16 input
 * (patches/comfy_kitchen_swiglu_w4a4_fused.patch:25-31). Outside that domain it applies the
 * activation eagerly first (:60-64), silu(gate).mul_(up) in the input's type
 * (patches/comfyui_swiglu_triton_env.patch:16-20): EAGER reproduces those two roundings. Both modes
 * take every Hadamard block, int8 codes and the group GEMM's code layouts. silu(g) =
 * g / (1 + exp(-g)) is taken correctly rounded to fp32 (the reference's kernel uses a hardware exp
 * approximation and an fp32 division; torch's silu is its own fp32 evaluation): tables of the exact
 * results, for every bf16 gate outside the closed forms |g| < 2^-25 -> g / 2, g >= 128 -> g,
 * g <= -128 -> -0, and for every fp16 gate.
 *
 *   h      [M, 2K] of type h_dtype (MQ_DT_BF16 or MQ_DT_F16): gate in columns [0, K), up in
 *          [K, 2K); row stride ldh >= 2K elements (ldh % 8 == 0, 16-byte aligned base)
 *   mode   MQ_SWIGLU_FUSED or MQ_SWIGLU_EAGER
 *   other arguments as mq_rotquant (K is the width of the activation, half of h's).
 * Requires K % 16 == 0, K <= 16384, K % hblock == 0.
 */
int mq_swiglu_rotquant(const void* h, int h_dtype, int64_t M, int64_t K, int64_t ldh, int hblock, int bits,
                       int packed, int mode, void* q, int64_t ldq, float* scale, void* stream);

/* Weight formats written by mq_quantize_weight. */
#define MQ_WFMT_U4_ASYM_G64 0   /* configs' W4A8: uint4 asymmetric per 64, fp16 scale, uint4 zero   */
#define MQ_WFMT_I4_SYM_G64 1    /* configs' W4A4: int4 symmetric per 64, fp16 scale                  */
#define MQ_WFMT_I4_ROW 2        /* shipped ConvRot W4A4: int4 per row, fp32 scale [N]                */
#define MQ_WFMT_I8_ROW 3        /* int8_tensorwise: int8 per row, fp32 scale [N]                     */

/*
 * Offline weight quantizer (the converter side of the path): rotate each weight row by H_hblock
 * (hblock 0 = no rotation; the pinned fp32 radix-4 order of mq_rotquant, folded into the weight
 * as W_rot = W H, experiments/qwen21-kernel/node/__init__.py:69-71) and quantize it. Replaces the
 * quantizers the converters call: quantize_convrot_w4a4_weight (tools/_formats.py:53-76,
 * MQ_WFMT_I4_ROW), the int8_tensorwise quantizer (tools/_formats.py:128-167, MQ_WFMT_I8_ROW) and,
 * for the configs' group schemes, the packed-uint4 writer behind tools/quant_w4a8.py:91-168.
 * Arithmetic (fp32, IEEE division, round half to even):
 *   U4_ASYM_G64  per group of 64: lo = min(min w, 0), hi = max(max w, 0), s = fp16((hi - lo) / 15),
 *                z = clamp(rne(-lo / s), 0, 15), q = clamp(rne(w / s) + z, 0, 15); s = 0 -> q = z = 0
 *   I4_SYM_G64   per group of 64: s = fp16(max |w| / 7), q = clamp(rne(w / s), -7, 7); s = 0 -> q = 0
 *   I4_ROW       s = max(max |w|, 1e-10) / 7,   q = clamp(rne(w / s), -7, 7)
 *   I8_ROW       s = max(max |w|, 1e-10) / 127, q = clamp(rne(w / s), -127, 127)
 * A group whose range overflows fp16 stores an infinite scale (callers check the scales).
 *
 *   w      [N, K] of dtype MQ_DT_*, row stride ldw elements (>= K)
 *   q      packed 4-bit codes [N, K/2] (low nibble = even k; unsigned for U4_ASYM, signed
 *          otherwise) or int8 [N, K] for I8_ROW; row stride ldq bytes
 *   scale  fp16 [N, K/64] (stride ld_scale elements) for the group formats, fp32 [N] otherwise
 *   zero   U4_ASYM_G64 only: packed uint4 [N, ceil(K/128)] (group 2j low nibble), stride ld_zero
 * Requires K % 64 == 0 (group formats) or K % 16 == 0, K % hblock == 0, K <= 32768. Output rows
 * are written by plain stores; no alignment beyond the element size is needed.
 */
int mq_quantize_weight(const void* w, int dtype, int64_t N, int64_t K, int64_t ldw, int hblock, int format,
                       void* q, int64_t ldq, void* scale, int64_t ld_scale, void* zero, int64_t ld_zero,
                       void* stream);

/*
 * Load-time decode of comfy-kitchen's shipped asym_w4a8_int8 weight (tools/_formats.py:79-125:
 * qdata I8 [N, K/2] 4-bit codes, s_rel fp8 e4m3fn stored as U8 [N, K/gs], s_channel F32 [N],
 * codebook F32 [16] or none) to an int8 weight with a per-row scale, which the int8 row-scale GEMM
 * (mq_gemm_rowscale, wbits 8) then takes. comfy-kitchen finishes a decoded W4A8 weight the same way,
 * as dequantize_int8_convrot_weight_dtype(int8_weight, s_channel, ...)
 * (patches/comfy_kitchen_w4a8_dequant_fused.patch:15-18): the int8 weight's row scale is the stored
 * s_channel, unchanged, so level * s_rel is in int8 units:
 *   level = codebook[code] (unsigned nibble, low nibble = even k), or the signed nibble if
 *           codebook is NULL
 *   t[n,k]  = fp32(level * fp8(s_rel[n, k / group_size]))
 *   q8[n,k] = clamp(rne(t[n,k]), -127, 127)   (0 where t is NaN: an fp8 NaN scale byte)
 *   row_scale[n] = s_channel[n]
 * q8 * row_scale is then level * s_rel * s_channel to within half an int8 step wherever
 * |t| <= 127.5. comfy-kitchen's rounding of t is not in the reference tree (round half to even is
 * this library's choice).
 *
 *   qdata  [N, K/2] bytes, stride ldq (ldq % 4 == 0, 4-byte aligned)
 *   s_rel  [N, K/group_size] fp8 bytes, stride lds
 *   q8     int8 [N, K], stride ldq8 (ldq8 % 8 == 0, 8-byte aligned); row_scale fp32 [N]
 * Requires K % 16 == 0, K % group_size == 0, group_size >= 4 dividing or a multiple of 16
 * (the accepts() rule of tools/_formats.py:86-97).
 */
int mq_decode_w4a8_codebook(const void* qdata, int64_t ldq, const void* s_rel, int64_t lds, const float* s_channel,
                            const float* codebook, int group_size, int64_t N, int64_t K, int8_t* q8, int64_t ldq8,
                            float* row_scale, void* stream);

/*
 * Load-time expansion of packed 4-bit weights [N, K/2] (uint4 with zero-points wz, or signed int4
 * when wz is NULL) to int8 in the 16-row tiles of MQ_W8_TILE16, [ceil(N/16)][K/64][16][64] bytes
 * (rows past N zero). Byte (n, k) is v = q - z[n, k/64] (uint4) or the signed nibble, then by
 * layout:
 *   MQ_ACT_I8      v, negated where (k / 64) is odd: for the group GEMMs with act_mode MQ_ACT_I8
 *   MQ_ACT_X16ALT  v for uint4, 16 * v for signed int4: for act_mode MQ_ACT_X16ALT
 *   MQ_W4X_ROW     v: an int8 weight for the row-scale GEMMs (wbits 8 | MQ_W8_TILE16), the
 *                  shipped ConvRot W4A4 weight with the same int32 sums as its packed form
 * These are the bytes the group GEMM's in-kernel unpack stores to LDS for that activation layout,
 * so a GEMM on them gives the packed GEMM's results bit for bit; the GEMM then reads them by the
 * same DMA as the activation codes and does no unpack (half the weight bytes per K group more,
 * none of the unpack's VALU work). No counterpart in the reference (whose kernel unpacks per use,
 * experiments/qwen21-kernel/kernels/g64_gemm6.cu:93-343): it trades twice the packed weight's
 * memory for that work. Run once per weight.
 * The group-GEMM layouts (MQ_ACT_I8, MQ_ACT_X16ALT) also carry the weight's fp16 group scales, after
 * the tiles, as the GEMM's lanes read them straight into registers: uint32 [G4][16][ld] with
 * G4 = 4 * ceil(K/256) and ld = MQ_SCALE_PAIR_LD(N), dword [g][c][u] = ws[32u + c, g] |
 * ws[32u + 16 + c, g] << 16, zero where the column is >= N or g >= K/64. MQ_W4X_ROW carries none.
 *   qw   packed 4-bit [N, K/2], stride ldw bytes (ldw % 8 == 0, 8-byte aligned)
 *   wz   packed uint4 zero-points [N, ceil(K/128)], stride ldwz, or NULL (signed int4)
 *   ws   fp16 group scales [N, K/64], stride ldws elements (MQ_ACT_I8 / MQ_ACT_X16ALT; NULL for
 *        MQ_W4X_ROW)
 *   out  mq_expanded_w4_bytes(N, K, layout) bytes, 16-byte aligned, under 2 GiB
 * Requires K % 64 == 0.
 */
#define MQ_W4X_ROW 3
#define MQ_SCALE_PAIR_LD(N) ((((N) + 15) / 16 + 17) / 2)
int mq_expand_weight_w4(const uint8_t* qw, int64_t ldw, const uint8_t* wz, int64_t ldwz, const uint16_t* ws,
                        int64_t ldws, int64_t N, int64_t K, int layout, int8_t* out, void* stream);
int64_t mq_expanded_w4_bytes(int64_t N, int64_t K, int layout);

/* act_mode flag of the group GEMMs (act_bits flag of the whole group linears): qw holds the
 * expansion of mq_expand_weight_w4 for that activation layout (ldw ignored; the GEMM reads the
 * scales the expansion carries, and ws / ldws for the correction term of its epilogue, so they must
 * be the scales it was made with). wz is then not read;
 * non-NULL marks weights that were uint4 asymmetric (their MQ_ACT_X16ALT scaling differs from signed
 * int4). Read by the wide kernel only: M > 4 rows (fewer rows take the packed weights), K >= 192,
 * the expanded array under 2 GiB; the group-scale epilogue only (not the partials entry). */
#define MQ_W4_EXPANDED 0x100

/*
 * Quantized GEMM with per-group weight scales (W4A8 asym / W4A4 sym, configs' scheme):
 *   P[g,m,n] = sum_{k in group g} qa[m,k] * (w[n,k] - z[n,g])            (exact int32)
 *   y[m,n]   = T( sa[m] * sum_g ws[n,g] * P[g,m,n] + bias[n] )      (fp32, one rounding to T)
 *
 * Replaces the GEMM half of w4a8_int8_linear / convrot_w4a4_linear (the int4_linear call at
 * patches/comfy_kitchen_swiglu_w4a4_fused.patch:37-38) for per-group fp16 weight scales; the
 * reference's own per-group policy kernel is experiments/qwen21-kernel/kernels/g64_gemm6.cu:93-343
 * with its torch reference g64_bench6.py:50-68.
 *
 *   qa    activation codes [M, K] in layout act_mode (MQ_ACT_*), stride lda bytes (lda % 16 == 0)
 *   sa    fp32 [M]
 *   qw    packed 4-bit weights [N, K/2], stride ldw bytes (ldw % 16 == 0), or with
 *         act_mode | MQ_W4_EXPANDED their int8 expansion (mq_expand_weight_w4)
 *   ws    fp16 [N, K/group], stride ldws elements
 *   wz    packed uint4 zero-points [N, ceil(K/group/2)], stride ldwz bytes; NULL = signed
 *         symmetric int4 weights (no zero-point)
 *   group 64
 *   bias  [N] of type bias_dtype (MQ_DT_BF16, MQ_DT_F16 or MQ_DT_F32), or NULL
 *   y     [M, N] of type y_dtype (MQ_DT_BF16, MQ_DT_F16 or MQ_DT_F32: the caller's out_dtype,
 *         written directly), stride ldy elements
 * Requires K % 64 == 0. The partials are exact; the sum over groups is accumulated in fp32.
 */
int mq_gemm_w4_group(const int8_t* qa, int64_t lda, const float* sa, const uint8_t* qw, int64_t ldw,
                     const uint16_t* ws, int64_t ldws, const uint8_t* wz, int64_t ldwz, int group, int act_mode,
                     const void* bias, int bias_dtype, void* y, int y_dtype, int64_t ldy, int64_t M, int64_t N,
                     int64_t K, void* stream);

/*
 * mq_gemm_w4_group with a caller-provided workspace. Products whose 256 x 256 output tiles would
 * occupy at most half of the compute units run on 128 x 128 tiles (with or without a
 * workspace; the same bits either way). When those tiles still leave most compute units idle
 * (small M: the text-token linears) the K groups are split into slices, each slice's workgroups
 * write fp32 partial outputs [slices][M][N] into the workspace, and a reduction kernel sums them
 * in slice order (deterministic) and applies sa, bias and the bf16 rounding. For large M whose
 * 256 tiles would leave a last wave of whole tile rows occupying at most a quarter of the compute
 * units (M = 4352 against N = 12288 on 256 units), those trailing rows run as their own product
 * after the others, with the tile and split that their own shape gets.
 * mq_gemm_workspace_bytes(M, N, K) gives the size that enables the split on the current device
 * (0: no split for this shape); a smaller or NULL workspace runs without it. No reference
 * counterpart: comfy-kitchen's GEMMs allocate internally.
 *   workspace  device memory, 16-byte aligned, workspace_bytes long (or NULL)
 */
int mq_gemm_w4_group_ws(const int8_t* qa, int64_t lda, const float* sa, const uint8_t* qw, int64_t ldw,
                        const uint16_t* ws, int64_t ldws, const uint8_t* wz, int64_t ldwz, int group, int act_mode,
                        const void* bias, int bias_dtype, void* y, int y_dtype, int64_t ldy, int64_t M, int64_t N,
                        int64_t K, void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes mq_gemm_w4_group_ws / mq_gemm_rowscale_ws use for an M x N x K product on the
 * current device (0 when the shape fills the device without splitting K, whole or in part). */
int64_t mq_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K);

/*
 * Debug / parity entry: the exact per-group int32 partials P[g,m,n] of mq_gemm_w4_group
 * (same tile loaders, unpack and MFMA code), written to part int32 [K/group, M, N] (dense).
 * P is the partial of the codes themselves: the x16 / sign of layout MQ_ACT_X16ALT is undone.
 */
int mq_gemm_w4_group_partials(const int8_t* qa, int64_t lda, const uint8_t* qw, int64_t ldw,
                              const uint8_t* wz, int64_t ldwz, int group, int act_mode, int32_t* part,
                              int64_t M, int64_t N, int64_t K, void* stream);

/*
 * Quantized GEMM with per-row weight scales and a full-K int32 accumulator (policy 0 of
 * experiments/qwen21-kernel/kernels/g64_gemm6.cu:5):
 *   y[m,n] = T( (sum_k qa[m,k] * w[n,k]) * sa[m] * ws[n] + bias[n] )
 * Replaces int4_linear(qact, qweight, x_scale, wscales, bias, out_dtype) of the shipped ConvRot
 * W4A4 format (patches/comfy_kitchen_swiglu_w4a4_fused.patch:37-38) when wbits = 4, and the
 * int8 x int8 GEMM of int8_linear (tools/verify_w4a4.py:342-370) when wbits = 8.
 *
 *   qa    int8 activation codes [M, K], stride lda bytes
 *   qw    wbits 4: signed int4 packed [N, K/2]; wbits 8: int8 [N, K]; stride ldw bytes;
 *         wbits 8 | MQ_W8_TILE16: int8 in the 16-row tile layout below (ldw ignored)
 *   ws    fp32 [N]
 *   bias, y as mq_gemm_w4_group
 * Requires K % 64 == 0.
 */

/* wbits flag of the int8 row-scale entries (mq_gemm_rowscale*, mq_linear_rowscale): the int8
 * weights are in 16-row tiles, [ceil(N/16)][K/64][16][64] bytes, block (b, g) holding bytes
 * [64 g, 64 g + 64) of rows 16 b .. 16 b + 15 (rows past N zero). No counterpart in the reference,
 * whose int8 weights are [N, K] rows (tools/verify_w4a4.py:342-370): it is the same weight in a
 * layout whose K groups are whole cache lines for the GEMM's loads, written once per weight by
 * mq_tile_weight_i8, and gives the same results bit for bit. Needs K >= 192 and a tiled array
 * under 2 GiB. */
#define MQ_W8_TILE16 0x100

/* int8 weights [N, K] (stride ldw bytes, ldw % 16 == 0, 16-byte aligned) into the MQ_W8_TILE16
 * layout at out (ceil(N/16) * 16 * K bytes, 16-byte aligned). */
int mq_tile_weight_i8(const int8_t* w, int64_t ldw, int64_t N, int64_t K, int8_t* out, void* stream);
int mq_gemm_rowscale(const int8_t* qa, int64_t lda, const float* sa, const void* qw, int64_t ldw,
                     int wbits, const float* ws, const void* bias, int bias_dtype, void* y, int y_dtype,
                     int64_t ldy, int64_t M, int64_t N, int64_t K, void* stream);

/* mq_gemm_rowscale with a caller-provided workspace (int32 partial sums per K slice, summed
 * exactly before the epilogue: the same result as without the split). */
int mq_gemm_rowscale_ws(const int8_t* qa, int64_t lda, const float* sa, const void* qw, int64_t ldw, int wbits,
                        const float* ws, const void* bias, int bias_dtype, void* y, int y_dtype, int64_t ldy,
                        int64_t M, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, void* stream);

/* Debug / parity entry: the full-K int32 accumulator of mq_gemm_rowscale, acc int32 [M, N]. */
int mq_gemm_rowscale_acc(const int8_t* qa, int64_t lda, const void* qw, int64_t ldw, int wbits,
                         int32_t* acc, int64_t M, int64_t N, int64_t K, void* stream);

/*
 * Whole linears: rotate + quantize x (or the SwiGLU pair h), then the GEMM, in one call. The
 * activation codes and scales live in the caller's workspace; the kernels, arithmetic and results
 * are those of mq_rotquant / mq_swiglu_rotquant followed by mq_gemm_w4_group_ws / mq_gemm_rowscale_ws.
 * One row (M = 1, K <= 4096, swiglu = MQ_SWIGLU_NONE) runs as one launch: the GEMV rotates and
 * quantizes the row itself with the same arithmetic (same codes, scale and output bits) and leaves
 * the workspace unwritten; it is still required and checked.
 *
 * mq_linear_w4_group replaces w4a8_int8_linear (configs' uint4 asymmetric scheme, act_bits 8,
 * tools/test_verify_formats.py:375-383) and convrot_w4a4_linear with per-group fp16 weight scales
 * (act_bits 4 or 8, patches/comfy_kitchen_swiglu_w4a4_fused.patch:41-67); mq_linear_rowscale
 * replaces int8_linear (tools/verify_w4a4.py:342-370, wbits 8) and convrot_w4a4_linear with the
 * shipped per-row F32 scale (wbits 4).
 *
 *   x       [M, K] (swiglu = MQ_SWIGLU_NONE) or gate | up [M, 2K] (MQ_SWIGLU_FUSED / MQ_SWIGLU_EAGER,
 *           the activation of mq_swiglu_rotquant in that mode) of type x_dtype, stride ldx
 *   hblock  Hadamard block (0, 16, 64, 256); act_bits 8 or 4 (per-token int8 / int4 activations),
 *           for mq_linear_w4_group | MQ_W4_EXPANDED with expanded weights
 *   weights, scales, bias, y as mq_gemm_w4_group / mq_gemm_rowscale
 *   workspace  device memory, 256-byte aligned: the codes (M rounded up to 16 rows, K bytes
 *           each, in rows or in the 16-row tiles of MQ_W8_TILE16 wherever the product runs on the
 *           kernel that reads those) and scales [M] first (both required), then the split-K
 *           partials when the shape wants them and they fit;
 *           mq_linear_workspace_bytes(M, N, K) gives the size that holds all of it.
 */
int64_t mq_linear_workspace_bytes(int64_t M, int64_t N, int64_t K);

int mq_linear_w4_group(const void* x, int x_dtype, int64_t ldx, int hblock, int act_bits, int swiglu,
                       const uint8_t* qw, int64_t ldw, const uint16_t* ws, int64_t ldws, const uint8_t* wz,
                       int64_t ldwz, const void* bias, int bias_dtype, void* y, int y_dtype, int64_t ldy, int64_t M,
                       int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, void* stream);

int mq_linear_rowscale(const void* x, int x_dtype, int64_t ldx, int hblock, int act_bits, int swiglu, const void* qw,
                       int64_t ldw, int wbits, const float* ws, const void* bias, int bias_dtype, void* y,
                       int y_dtype, int64_t ldy, int64_t M, int64_t N, int64_t K, void* workspace,
                       int64_t workspace_bytes, void* stream);

/* Size of the fixed per-device scratch array behind mq_linear_w4_group_noalloc. */
#define MQ_NOALLOC_SCRATCH_BYTES (64ll << 20)

/*
 * mq_linear_w4_group without a workspace argument: it allocates nothing (no hipMalloc, no
 * allocating library call). No counterpart in the reference; it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * it). The activation codes, scales and split-K partials go to a fixed array of
 * MQ_NOALLOC_SCRATCH_BYTES in device memory that each GPU the library runs on holds until the
 * process ends; a call whose codes and scales (about M * K + 4 * M bytes) do not fit returns
 * MQ_EINVAL, and split-K partials are used only where they fit beside them. Results equal
 * mq_linear_w4_group's bit for bit whenever mq_linear_workspace_bytes(M, N, K) <=
 * MQ_NOALLOC_SCRATCH_BYTES (both entries then take the same split-K decision); when only the codes
 * and scales fit, the product runs without split-K: the same codes and int32 group partials, with
 * the fp32 group sums associated in another order (outputs within the linear's tolerance of the
 * exact result, not bit-identical to the split product's). Every call
 * on one GPU shares that GPU's array: calls that overlap on one GPU (several streams or threads)
 * race and must be serialized by the caller. Nothing in the array needs to start at zero: each call
 * writes every byte it reads.
 */
int mq_linear_w4_group_noalloc(const void* x, int x_dtype, int64_t ldx, int hblock, int act_bits, int swiglu,
                               const uint8_t* qw, int64_t ldw, const uint16_t* ws, int64_t ldws, const uint8_t* wz,
                               int64_t ldwz, const void* bias, int bias_dtype, void* y, int y_dtype, int64_t ldy,
                               int64_t M, int64_t N, int64_t K, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MQ_H */
