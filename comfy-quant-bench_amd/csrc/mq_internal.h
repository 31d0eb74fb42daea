// Internal declarations shared by the libmq translation units (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

namespace mq {

// Thread-local error message behind mq_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// Translates the HIP launch status into the ABI status and message.
int launch_status(const char* what);

// Compute units of the current device (0 if the runtime cannot say). The attribute query runs
// once per device; later calls read the cached value, so the launchers can size their grids on
// every call without a runtime query.
int device_cu_count();

// --- rotate + quantize (mq_rotquant*.hip), one launcher per input type
int launch_rotquant_bf16(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int hblock, int bits,
                         int packed, void* q, int64_t ldq, float* scale, hipStream_t stream);
int launch_rotquant_f16(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int hblock, int bits,
                        int packed, void* q, int64_t ldq, float* scale, hipStream_t stream);
int launch_rotquant_f32(const float* x, int64_t M, int64_t K, int64_t ldx, int hblock, int bits,
                        int packed, void* q, int64_t ldq, float* scale, hipStream_t stream);

// --- SwiGLU prologue + rotate + quantize (mq_swiglu*.hip); h holds gate | up, K columns each.
// The fused activation T(silu(g) * u) rounds once; the eager one T(T(silu(g)) * u) twice.
int launch_swiglu_rotquant_bf16(const uint16_t* h, int64_t M, int64_t K, int64_t ldh, int hblock, int bits,
                                int packed, void* q, int64_t ldq, float* scale, hipStream_t stream);
int launch_swiglu_rotquant_f16(const uint16_t* h, int64_t M, int64_t K, int64_t ldh, int hblock, int bits,
                               int packed, void* q, int64_t ldq, float* scale, hipStream_t stream);
int launch_swiglu_eager_rotquant_bf16(const uint16_t* h, int64_t M, int64_t K, int64_t ldh, int hblock, int bits,
                                      int packed, void* q, int64_t ldq, float* scale, hipStream_t stream);
int launch_swiglu_eager_rotquant_f16(const uint16_t* h, int64_t M, int64_t K, int64_t ldh, int hblock, int bits,
                                     int packed, void* q, int64_t ldq, float* scale, hipStream_t stream);

// --- load-time decode of the shipped asym_w4a8_int8 codebook weights (mq_codebook.hip)
int launch_decode_w4a8_codebook(const uint8_t* qdata, int64_t ldq, const uint8_t* s_rel, int64_t lds,
                                const float* s_channel, const float* codebook, int group_size, int64_t N,
                                int64_t K, int8_t* q8, int64_t ldq8, float* row_scale, hipStream_t stream);

// --- offline weight quantizer (mq_wquant.hip); dtype / format are MQ_DT_* / MQ_WFMT_*
int launch_quantize_weight(const void* w, int dtype, int64_t N, int64_t K, int64_t ldw, int hblock, int format,
                           void* q, int64_t ldq, void* scale, int64_t ld_scale, void* zero, int64_t ld_zero,
                           hipStream_t stream);

// int8 weights [N, K] into the 16-row tile layout of GemmArgs::wtile (mq_wquant.hip)
int launch_tile_weight_i8(const uint8_t* w, int64_t ldw, int64_t N, int64_t K, uint8_t* out, hipStream_t stream);

// packed 4-bit weights into int8 16-row tiles (mq_expand_weight_w4's layouts; mq_wquant.hip)
// dwords per [g][c] row of the scale pairs that expanded 4-bit weights carry (MQ_SCALE_PAIR_LD)
__host__ __device__ inline int64_t scale_pair_ld(int64_t N) { return ((N + 15) / 16 + 17) / 2; }
int launch_expand_scales_w4(const uint16_t* ws, int64_t ldws, int64_t N, int64_t K, uint32_t* out,
                            hipStream_t stream);
int launch_expand_weight_w4(const uint8_t* qw, int64_t ldw, const uint8_t* wz, int64_t ldwz, int64_t N, int64_t K,
                            int layout, uint8_t* out, hipStream_t stream);

// --- GEMMs (mq_gemm.hip)
enum class WKind : int { U4Asym = 0, I4Sym = 1, I8 = 2 };
enum class Epi : int { GroupScale = 0, GroupPartials = 1, RowScale = 2, RowAcc = 3 };

struct GemmArgs {
    const int8_t* qa;
    int64_t lda;
    const float* sa;
    const uint8_t* qw;
    int64_t ldw;
    const uint16_t* ws16;   // per-group fp16 scales [N, ldws]
    int64_t ldws;
    const float* ws32;      // per-row fp32 scales [N]
    const uint8_t* wz;      // packed u4 zero-points [N, ldwz]
    int64_t ldwz;
    const void* bias;       // [N] of type bias_dtype, or null
    void* y;                // [M, ldy] of type y_dtype
    int64_t ldy;
    int bias_dtype;         // MQ_DT_BF16 / MQ_DT_F16 / MQ_DT_F32
    int y_dtype;
    int32_t* part;          // int32 partials / accumulators
    int64_t M, N, K;
    int act_mode;           // group-scale GEMMs: MQ_ACT_* layout of qa (include/mq.h)
    // split-K (wide kernel, GroupScale / RowScale only): ksplit slices of kgroups K groups each
    // (a multiple of 4) write fp32 (GroupScale) or int32 (RowScale) partial outputs [ksplit][M][N]
    // to work, which a reduction kernel sums and finishes; ksplit 1 = no split
    int ksplit = 1;
    int kgroups = 0;
    void* work = nullptr;
    int64_t work_bytes = 0;   // capacity of work offered by the caller
    // output tile of the wide kernel: 256 (256 x 256), 192 (256 x 192) or 128 (128 x 128); 0:
    // choose_tile decides
    int tile = 0;
    // int8 weights (WKind::I8) in 16-row tiles: [ceil(N / 16)][K / 64][16][64] bytes, so that a
    // 1 KB block holds one K group of 16 consecutive rows (ldw = K); 0: rows of ldw bytes. With a
    // 4-bit kind (group scales): the weights expanded to int8 in those tiles (mq_expand_weight_w4),
    // read by the wide kernel only; wz then only tells uint4 asymmetric (non-null) from signed
    int wtile = 0;
    // activation codes (qa) in the same 16-row tiles, [ceil(M / 16)][K / 64][16][64] (lda = K):
    // written so by the whole-linear entries when the wide kernel runs their product
    int atile = 0;
    // One-row whole linears (gemv_quantizes_row): the GEMV rotates and quantizes the activation
    // row x (x_dtype, Hadamard block hblock, x_bits-bit codes) itself instead of reading qa / sa
    const void* x = nullptr;
    int x_dtype = 0;
    int hblock = 0;
    int x_bits = 8;
};

// Output tile of the wide kernel for an M x N product (a tile code as above): 128 when 256 x 256
// tiles would occupy at most half of the compute units; else 192 when its rounds of resident
// workgroups take less time than 256 x 256 tiles (with their trailing rows, tail_rows) would
// (N = 3072 at M = 4096: 256 tiles in one round instead of 192); else 256.
int choose_tile(int64_t M, int64_t N);

// K slices for a GEMM of this shape with a workspace of work_bytes (1 = no split): used when the
// tiles of choose_tile leave most compute units idle (small M). int_sums: the row-scale epilogue
// (int32 sums), which splits only over a long K.
int choose_ksplit(int64_t M, int64_t N, int64_t K, int64_t work_bytes, int* kgroups, bool int_sums);

// Rows at the end of an M x N product that run as a separate GEMM (0: none): when the 256 x 256
// tiles leave a last wave of whole tile rows that would occupy at most a quarter of the compute
// units (M = 4352 = 4096 + 256 tokens against N = 12288: 816 tiles on 256 units), those rows run
// on their own, on the tile and K split that choose_tile and choose_ksplit give them, so they take
// a fraction of a 256 tile's time.
int64_t tail_rows(int64_t M, int64_t N, int64_t K);

// Workspace bytes the split-K of an M x N x K product uses with the group-scale (int_sums false)
// or row-scale epilogue (0: none).
int64_t workspace_bytes(int64_t M, int64_t N, int64_t K, bool int_sums);

// Power-of-two factor by which a group GEMM's MFMA result exceeds the true partial, per
// activation layout and weight kind (see mq_gemm_wide.hip).
__host__ __device__ inline int group_shift(int act_mode, WKind wk) {
    if (act_mode == 1) return 4;
    if (act_mode == 2) return wk == WKind::I4Sym ? 8 : 4;
    return 0;
}

int launch_gemm(const GemmArgs& a, WKind wk, Epi epi, hipStream_t stream);
// whether launch_gemm runs these arguments' product on the wide kernel (the one that reads atile)
bool gemm_runs_wide(const GemmArgs& a, WKind wk, Epi epi);

// M <= 4 rows, GroupScale / RowScale only (mq_gemv.hip).
int launch_gemv(const GemmArgs& a, WKind wk, Epi epi, hipStream_t stream);
// Whether a whole linear of these operands can hand its activation row to the GEMV (one row,
// K <= 4096, a scaled epilogue): the GEMV then rotates and quantizes the row in its prologue with
// the rotate+quantize kernel's arithmetic, in the same launch.
bool gemv_quantizes_row(const GemmArgs& a, WKind wk, Epi epi);

// 256 x 256-tile kernel for large M (mq_gemm_wide.hip).
int launch_gemm_wide(const GemmArgs& a, WKind wk, Epi epi, hipStream_t stream);

}  // namespace mq
