// extern "C" entry points of libmq.so (declared in include/mq.h): argument validation, error
// reporting and dispatch to the kernel launchers. Nothing here allocates device memory.
#include "../../include/mq.h"

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstring>
#include <mutex>

#include "mq_internal.h"

namespace mq {

namespace {
thread_local char g_err[512] = "";

bool aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }
}  // namespace

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

int device_cu_count() {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> cache[kMaxDevices];   // 0 = not queried yet
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    const bool cached = dev >= 0 && dev < kMaxDevices;
    if (cached) {
        const int v = cache[dev].load(std::memory_order_relaxed);
        if (v > 0) return v;
    }
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
    if (cached) cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

int launch_status(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
        return MQ_ELAUNCH;
    }
    return MQ_OK;
}

namespace {

#define MQ_REQUIRE(cond, ...)        \
    do {                             \
        if (!(cond)) {               \
            set_error(__VA_ARGS__);  \
            return MQ_EINVAL;        \
        }                            \
    } while (0)

constexpr int kEmpty = 1;   // check_gemm_common: valid shape with nothing to compute

int dtype_bytes(int dt) { return dt == MQ_DT_F32 ? 4 : 2; }

// Output and bias checks shared by the GEMM entry points: types, alignment and the row stride.
int check_gemm_out(const char* what, const void* bias, int bias_dtype, const void* y, int y_dtype, int64_t ldy,
                   int64_t N) {
    MQ_REQUIRE(y_dtype >= MQ_DT_BF16 && y_dtype <= MQ_DT_F32, "%s: unknown output type %d", what, y_dtype);
    MQ_REQUIRE(!bias || (bias_dtype >= MQ_DT_BF16 && bias_dtype <= MQ_DT_F32), "%s: unknown bias type %d", what,
               bias_dtype);
    MQ_REQUIRE(y && aligned(y, dtype_bytes(y_dtype)), "%s: y must be non-null and aligned to its element size", what);
    MQ_REQUIRE(!bias || aligned(bias, dtype_bytes(bias_dtype)), "%s: bias must be aligned to its element size", what);
    MQ_REQUIRE(ldy >= N, "%s: ldy < N", what);
    return MQ_OK;
}

// Weights in 16-row tiles (MQ_W8_TILE16): int8 only, K >= 192 (the wide kernel's minimum), the
// whole tiled array under 2 GiB (32-bit buffer offsets); the row stride becomes K.
int check_tile16(const char* what, bool tile16, int wbits, int64_t N, int64_t K, int64_t* ldw) {
    if (!tile16) return MQ_OK;
    MQ_REQUIRE(wbits == 8, "%s: the 16-row tile layout is for int8 weights (wbits 8)", what);
    MQ_REQUIRE(K >= 192 && K % 64 == 0, "%s: 16-row tile weights need K %% 64 == 0 and K >= 192 (got %lld)", what,
               (long long)K);
    MQ_REQUIRE(N >= 0 && (N + 15) / 16 * 16 * K < (int64_t(1) << 31), "%s: 16-row tile weights must be under 2 GiB",
               what);
    *ldw = K;
    return MQ_OK;
}

int check_gemm_common(const int8_t* qa, int64_t lda, const void* qw, int64_t ldw, int64_t M, int64_t N,
                      int64_t K, int64_t wbytes_per_row) {
    MQ_REQUIRE(M >= 0 && N >= 0 && K > 0, "gemm: bad shape M=%lld N=%lld K=%lld", (long long)M,
               (long long)N, (long long)K);
    MQ_REQUIRE(K % 64 == 0, "gemm: K=%lld must be a multiple of 64", (long long)K);
    MQ_REQUIRE(M <= (int64_t(1) << 31) - 256 && N <= (int64_t(1) << 31) - 256, "gemm: M or N too large");
    if (M == 0 || N == 0) return kEmpty;   // a valid no-op: no operand is read or written
    MQ_REQUIRE(qa && qw, "gemm: null operand");
    MQ_REQUIRE(lda >= K && lda % 16 == 0 && aligned(qa, 16), "gemm: qa needs lda >= K, lda %% 16 == 0 and a 16-byte aligned base");
    MQ_REQUIRE(ldw >= wbytes_per_row && ldw % 16 == 0 && aligned(qw, 16),
               "gemm: qw needs ldw >= %lld bytes, ldw %% 16 == 0 and a 16-byte aligned base", (long long)wbytes_per_row);
    return MQ_OK;
}

}  // namespace
}  // namespace mq

using namespace mq;

extern "C" {

int mq_abi_version(void) { return MQ_ABI_VERSION; }

const char* mq_last_error(void) { return g_err; }

}  // extern "C"

namespace {

// Argument checks shared by mq_rotquant and mq_swiglu_rotquant; x holds `cols` 16-bit values per
// row (K, or 2K for gate | up).
int check_rotquant(const char* what, const void* x, int x_dtype, bool f32_ok, int64_t M, int64_t K, int64_t cols,
                   int64_t ldx, int hblock, int bits, int packed, const void* q, int64_t ldq, const float* scale) {
    MQ_REQUIRE(x_dtype == MQ_DT_BF16 || x_dtype == MQ_DT_F16 || (f32_ok && x_dtype == MQ_DT_F32),
               "%s: input type must be bf16 (%d), fp16 (%d)%s, got %d", what, MQ_DT_BF16, MQ_DT_F16,
               f32_ok ? " or fp32 (2)" : "", x_dtype);
    MQ_REQUIRE(M >= 0 && K > 0, "%s: bad shape M=%lld K=%lld", what, (long long)M, (long long)K);
    MQ_REQUIRE(M < (int64_t(1) << 31), "%s: M too large", what);
    MQ_REQUIRE(bits == 8 || bits == 4, "%s: bits must be 8 or 4 (got %d)", what, bits);
    MQ_REQUIRE(packed >= MQ_Q_BYTES && packed <= MQ_Q_X16ALT, "%s: unknown code layout %d", what, packed);
    MQ_REQUIRE(packed == MQ_Q_BYTES || bits == 4, "%s: packed output needs bits = 4", what);
    MQ_REQUIRE(hblock == 0 || hblock == 16 || hblock == 64 || hblock == 256,
               "%s: convrot group size must be 16, 64 or 256 (got %d)", what, hblock);
    MQ_REQUIRE(K % 16 == 0, "%s: K=%lld must be a multiple of 16", what, (long long)K);
    MQ_REQUIRE(hblock == 0 || K % hblock == 0, "%s: K=%lld is not a multiple of the group size %d", what,
               (long long)K, hblock);
    if (K > 16384) {
        set_error("%s: K=%lld exceeds 16384", what, (long long)K);
        return MQ_EUNSUPPORTED;
    }
    if (M == 0) return MQ_OK;
    MQ_REQUIRE(x && q && scale, "%s: null pointer", what);
    const int64_t per16 = x_dtype == MQ_DT_F32 ? 4 : 8;   // elements per 16 bytes
    MQ_REQUIRE(ldx >= cols && ldx % per16 == 0 && aligned(x, 16),
               "%s: x needs ldx >= %lld, ldx %% %lld == 0, 16-byte aligned base", what, (long long)cols,
               (long long)per16);
    const int64_t row_bytes = packed == MQ_Q_PACKED ? K / 2 : K;
    const int64_t qalign = packed == MQ_Q_PACKED ? 8 : 16;
    MQ_REQUIRE(ldq >= row_bytes && ldq % qalign == 0 && aligned(q, qalign),
               "%s: q needs ldq >= %lld bytes, ldq %% %lld == 0 and an aligned base", what, (long long)row_bytes,
               (long long)qalign);
    MQ_REQUIRE(aligned(scale, 4), "%s: scale must be 4-byte aligned", what);
    return MQ_OK;
}

// The SwiGLU prologue kernels of a mode (MQ_SWIGLU_FUSED / MQ_SWIGLU_EAGER) and input type.
int launch_swiglu(int mode, int h_dtype, const uint16_t* h, int64_t M, int64_t K, int64_t ldh, int hblock, int bits,
                  int packed, void* q, int64_t ldq, float* scale, hipStream_t st) {
    const bool f16 = h_dtype == MQ_DT_F16;
    if (mode == MQ_SWIGLU_EAGER)
        return f16 ? launch_swiglu_eager_rotquant_f16(h, M, K, ldh, hblock, bits, packed, q, ldq, scale, st)
                   : launch_swiglu_eager_rotquant_bf16(h, M, K, ldh, hblock, bits, packed, q, ldq, scale, st);
    return f16 ? launch_swiglu_rotquant_f16(h, M, K, ldh, hblock, bits, packed, q, ldq, scale, st)
               : launch_swiglu_rotquant_bf16(h, M, K, ldh, hblock, bits, packed, q, ldq, scale, st);
}

}  // namespace

extern "C" {

int mq_rotquant(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, int hblock, int bits, int packed,
                void* q, int64_t ldq, float* scale, void* stream) {
    clear_error();
    const int rc = check_rotquant("rotquant", x, x_dtype, true, M, K, K, ldx, hblock, bits, packed, q, ldq, scale);
    if (rc != MQ_OK || M == 0) return rc;
    auto* xs = static_cast<const uint16_t*>(x);
    auto* st = static_cast<hipStream_t>(stream);
    if (x_dtype == MQ_DT_F32)
        return launch_rotquant_f32(static_cast<const float*>(x), M, K, ldx, hblock, bits, packed, q, ldq, scale, st);
    return x_dtype == MQ_DT_F16 ? launch_rotquant_f16(xs, M, K, ldx, hblock, bits, packed, q, ldq, scale, st)
                                : launch_rotquant_bf16(xs, M, K, ldx, hblock, bits, packed, q, ldq, scale, st);
}

int mq_swiglu_rotquant(const void* h, int h_dtype, int64_t M, int64_t K, int64_t ldh, int hblock, int bits,
                       int packed, int mode, void* q, int64_t ldq, float* scale, void* stream) {
    clear_error();
    MQ_REQUIRE(mode == MQ_SWIGLU_FUSED || mode == MQ_SWIGLU_EAGER,
               "swiglu_rotquant: mode must be MQ_SWIGLU_FUSED (1) or MQ_SWIGLU_EAGER (2), got %d", mode);
    const int rc =
        check_rotquant("swiglu_rotquant", h, h_dtype, false, M, K, 2 * K, ldh, hblock, bits, packed, q, ldq, scale);
    if (rc != MQ_OK || M == 0) return rc;
    return launch_swiglu(mode, h_dtype, static_cast<const uint16_t*>(h), M, K, ldh, hblock, bits, packed, q, ldq,
                         scale, static_cast<hipStream_t>(stream));
}

int mq_decode_w4a8_codebook(const void* qdata, int64_t ldq, const void* s_rel, int64_t lds, const float* s_channel,
                            const float* codebook, int group_size, int64_t N, int64_t K, int8_t* q8, int64_t ldq8,
                            float* row_scale, void* stream) {
    clear_error();
    MQ_REQUIRE(N >= 0 && K > 0, "decode_w4a8_codebook: bad shape N=%lld K=%lld", (long long)N, (long long)K);
    MQ_REQUIRE(N < (int64_t(1) << 31) && K < (int64_t(1) << 30), "decode_w4a8_codebook: shape too large");
    MQ_REQUIRE(group_size >= 4 && (16 % group_size == 0 || group_size % 16 == 0),
               "decode_w4a8_codebook: group_size must be >= 4 and divide or be a multiple of 16 (got %d)", group_size);
    MQ_REQUIRE(K % 16 == 0 && K % group_size == 0,
               "decode_w4a8_codebook: K=%lld must be a multiple of 16 and of group_size %d", (long long)K, group_size);
    if (N == 0) return MQ_OK;
    MQ_REQUIRE(qdata && s_rel && s_channel && q8 && row_scale, "decode_w4a8_codebook: null pointer");
    MQ_REQUIRE(ldq >= K / 2 && ldq % 4 == 0 && aligned(qdata, 4),
               "decode_w4a8_codebook: qdata needs ldq >= K/2 bytes, ldq %% 4 == 0 and a 4-byte aligned base");
    MQ_REQUIRE(lds >= K / group_size, "decode_w4a8_codebook: s_rel needs lds >= K / group_size bytes");
    MQ_REQUIRE(ldq8 >= K && ldq8 % 8 == 0 && aligned(q8, 8),
               "decode_w4a8_codebook: q8 needs ldq8 >= K bytes, ldq8 %% 8 == 0 and an 8-byte aligned base");
    MQ_REQUIRE(aligned(s_channel, 4) && aligned(row_scale, 4) && (!codebook || aligned(codebook, 4)),
               "decode_w4a8_codebook: fp32 operands must be 4-byte aligned");
    return launch_decode_w4a8_codebook(static_cast<const uint8_t*>(qdata), ldq, static_cast<const uint8_t*>(s_rel),
                                       lds, s_channel, codebook, group_size, N, K, q8, ldq8, row_scale,
                                       static_cast<hipStream_t>(stream));
}

int mq_quantize_weight(const void* w, int dtype, int64_t N, int64_t K, int64_t ldw, int hblock, int format,
                       void* q, int64_t ldq, void* scale, int64_t ld_scale, void* zero, int64_t ld_zero,
                       void* stream) {
    clear_error();
    MQ_REQUIRE(dtype >= MQ_DT_BF16 && dtype <= MQ_DT_F32, "quantize_weight: unknown dtype %d", dtype);
    MQ_REQUIRE(format >= MQ_WFMT_U4_ASYM_G64 && format <= MQ_WFMT_I8_ROW, "quantize_weight: unknown format %d", format);
    MQ_REQUIRE(N >= 0 && K > 0, "quantize_weight: bad shape N=%lld K=%lld", (long long)N, (long long)K);
    MQ_REQUIRE(N < (int64_t(1) << 31), "quantize_weight: N too large");
    MQ_REQUIRE(K <= 32768, "quantize_weight: K=%lld exceeds 32768", (long long)K);
    const bool group = format == MQ_WFMT_U4_ASYM_G64 || format == MQ_WFMT_I4_SYM_G64;
    MQ_REQUIRE(group ? K % 64 == 0 : K % 16 == 0, "quantize_weight: K=%lld must be a multiple of %d", (long long)K,
               group ? 64 : 16);
    MQ_REQUIRE(hblock == 0 || hblock == 16 || hblock == 64 || hblock == 256,
               "quantize_weight: convrot group size must be 0, 16, 64 or 256 (got %d)", hblock);
    MQ_REQUIRE(hblock == 0 || K % hblock == 0, "quantize_weight: K=%lld is not a multiple of the group size %d",
               (long long)K, hblock);
    if (N == 0) return MQ_OK;
    const int64_t esz = dtype == MQ_DT_F32 ? 4 : 2;
    MQ_REQUIRE(w && q && scale, "quantize_weight: null pointer");
    MQ_REQUIRE(ldw >= K && aligned(w, esz), "quantize_weight: w needs ldw >= K and an element-aligned base");
    const bool i8 = format == MQ_WFMT_I8_ROW;
    const int64_t qalign = i8 ? 8 : 4;
    MQ_REQUIRE(ldq >= (i8 ? K : K / 2) && ldq % qalign == 0 && aligned(q, qalign),
               "quantize_weight: q needs ldq >= %lld bytes, ldq %% %lld == 0 and an aligned base",
               (long long)(i8 ? K : K / 2), (long long)qalign);
    if (group) {
        MQ_REQUIRE(ld_scale >= K / 64 && aligned(scale, 2), "quantize_weight: scale needs ld_scale >= K/64 (fp16)");
    } else {
        MQ_REQUIRE(aligned(scale, 4), "quantize_weight: scale must be 4-byte aligned (fp32 [N])");
    }
    if (format == MQ_WFMT_U4_ASYM_G64)
        MQ_REQUIRE(zero && ld_zero >= (K / 64 + 1) / 2, "quantize_weight: zero needs ld_zero >= ceil(K/128)");
    return launch_quantize_weight(w, dtype, N, K, ldw, hblock, format, q, ldq, scale, ld_scale, zero, ld_zero,
                                  static_cast<hipStream_t>(stream));
}

int mq_tile_weight_i8(const int8_t* w, int64_t ldw, int64_t N, int64_t K, int8_t* out, void* stream) {
    clear_error();
    MQ_REQUIRE(N >= 0 && K >= 192 && K % 64 == 0, "tile_weight_i8: bad shape N=%lld K=%lld (K %% 64 == 0, K >= 192)",
               (long long)N, (long long)K);
    MQ_REQUIRE((N + 15) / 16 * 16 * K < (int64_t(1) << 31), "tile_weight_i8: the tiled weight must be under 2 GiB");
    if (N == 0) return MQ_OK;
    MQ_REQUIRE(w && out, "tile_weight_i8: null pointer");
    MQ_REQUIRE(ldw >= K && ldw % 16 == 0 && aligned(w, 16) && aligned(out, 16),
               "tile_weight_i8: needs ldw >= K, ldw %% 16 == 0 and 16-byte aligned w and out");
    return launch_tile_weight_i8(reinterpret_cast<const uint8_t*>(w), ldw, N, K, reinterpret_cast<uint8_t*>(out),
                                 static_cast<hipStream_t>(stream));
}

int mq_expand_weight_w4(const uint8_t* qw, int64_t ldw, const uint8_t* wz, int64_t ldwz, const uint16_t* ws,
                        int64_t ldws, int64_t N, int64_t K, int layout, int8_t* out, void* stream) {
    clear_error();
    MQ_REQUIRE(layout == MQ_ACT_I8 || layout == MQ_ACT_X16ALT || layout == MQ_W4X_ROW,
               "expand_weight_w4: layout must be MQ_ACT_I8 (0), MQ_ACT_X16ALT (2) or MQ_W4X_ROW (3), got %d", layout);
    MQ_REQUIRE(N >= 0 && K > 0 && K % 64 == 0, "expand_weight_w4: bad shape N=%lld K=%lld (K %% 64 == 0)",
               (long long)N, (long long)K);
    MQ_REQUIRE(mq_expanded_w4_bytes(N, K, layout) < (int64_t(1) << 31),
               "expand_weight_w4: the expanded weight must be under 2 GiB");
    if (N == 0) return MQ_OK;
    MQ_REQUIRE(qw && out, "expand_weight_w4: null pointer");
    MQ_REQUIRE(ldw >= K / 2 && ldw % 8 == 0 && aligned(qw, 8) && aligned(out, 16),
               "expand_weight_w4: needs ldw >= K/2, ldw %% 8 == 0, an 8-byte aligned qw and a 16-byte aligned out");
    MQ_REQUIRE(!wz || ldwz >= (K / 64 + 1) / 2, "expand_weight_w4: ldwz < ceil(K/64/2)");
    const bool scaled = layout != MQ_W4X_ROW;
    MQ_REQUIRE(!scaled || (ws && ldws >= K / 64), "expand_weight_w4: the group layouts need the fp16 scales (ldws >= K/64)");
    hipStream_t st = static_cast<hipStream_t>(stream);
    int rc = launch_expand_weight_w4(qw, ldw, wz, ldwz, N, K, layout, reinterpret_cast<uint8_t*>(out), st);
    if (rc || !scaled) return rc;
    return launch_expand_scales_w4(ws, ldws, N, K,
                                   reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(out) + (N + 15) / 16 * 16 * K),
                                   st);
}

int64_t mq_expanded_w4_bytes(int64_t N, int64_t K, int layout) {
    if (N < 0 || K <= 0) return 0;
    const int64_t tiles = (N + 15) / 16 * 16 * K;
    if (layout == MQ_W4X_ROW) return tiles;
    return tiles + (K / 64 + 3) / 4 * 4 * 16 * MQ_SCALE_PAIR_LD(N) * 4;
}

}  // extern "C"

namespace {

// Validated arguments of the group-scale GEMM (mq_gemm_w4_group_ws); kEmpty for an empty product.
int w4_group_args(const int8_t* qa, int64_t lda, const float* sa, const uint8_t* qw, int64_t ldw, const uint16_t* ws,
                  int64_t ldws, const uint8_t* wz, int64_t ldwz, int group, int act_mode, const void* bias,
                  int bias_dtype, void* y, int y_dtype, int64_t ldy, int64_t M, int64_t N, int64_t K, void* workspace,
                  int64_t workspace_bytes, GemmArgs* out) {
    MQ_REQUIRE(group == 64, "gemm_w4_group: quant group size must be 64 (got %d)", group);
    const bool expanded = (act_mode & MQ_W4_EXPANDED) != 0;
    act_mode &= ~MQ_W4_EXPANDED;
    MQ_REQUIRE(act_mode >= MQ_ACT_I8 && act_mode <= MQ_ACT_X16ALT, "gemm_w4_group: unknown act_mode %d", act_mode);
    if (expanded) {
        MQ_REQUIRE(act_mode != MQ_ACT_I4, "gemm_w4_group: expanded weights serve MQ_ACT_I8 and MQ_ACT_X16ALT");
        MQ_REQUIRE(K >= 192 && K % 64 == 0, "gemm_w4_group: expanded weights need K %% 64 == 0 and K >= 192 (got %lld)",
                   (long long)K);
        MQ_REQUIRE(N >= 0 && mq_expanded_w4_bytes(N, K, act_mode) < (int64_t(1) << 31),
                   "gemm_w4_group: expanded weights must be under 2 GiB");
        ldw = K;
    }
    int rc = check_gemm_common(qa, lda, qw, ldw, M, N, K, expanded ? K : K / 2);
    if (rc) return rc;
    MQ_REQUIRE(sa && ws, "gemm_w4_group: null pointer");
    rc = check_gemm_out("gemm_w4_group", bias, bias_dtype, y, y_dtype, ldy, N);
    if (rc) return rc;
    MQ_REQUIRE(ldws >= K / group, "gemm_w4_group: ldws < K/group");
    MQ_REQUIRE(expanded || !wz || ldwz >= (K / group + 1) / 2, "gemm_w4_group: ldwz < ceil(K/group/2)");
    MQ_REQUIRE(workspace_bytes >= 0 && (!workspace || aligned(workspace, 16)),
               "gemm_w4_group: workspace must be 16-byte aligned");
    GemmArgs a{};
    a.qa = qa; a.lda = lda; a.sa = sa; a.qw = qw; a.ldw = ldw; a.ws16 = ws; a.ldws = ldws;
    a.wz = wz; a.ldwz = ldwz; a.bias = bias; a.bias_dtype = bias_dtype; a.y = y; a.y_dtype = y_dtype; a.ldy = ldy;
    a.M = M; a.N = N; a.K = K;
    a.act_mode = act_mode;
    a.work = workspace; a.work_bytes = workspace ? workspace_bytes : 0;
    a.wtile = expanded;
    *out = a;
    return MQ_OK;
}

// Validated arguments of the row-scale GEMM (mq_gemm_rowscale_ws), wbits with its layout flag.
int rowscale_args(const int8_t* qa, int64_t lda, const float* sa, const void* qw, int64_t ldw, int wbits,
                  const float* ws, const void* bias, int bias_dtype, void* y, int y_dtype, int64_t ldy, int64_t M,
                  int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, GemmArgs* out, WKind* wk) {
    const bool tile16 = (wbits & MQ_W8_TILE16) != 0;
    wbits &= ~MQ_W8_TILE16;
    MQ_REQUIRE(wbits == 4 || wbits == 8, "gemm_rowscale: wbits must be 4 or 8 (got %d)", wbits);
    int rc = check_tile16("gemm_rowscale", tile16, wbits, N, K, &ldw);
    if (rc) return rc;
    rc = check_gemm_common(qa, lda, qw, ldw, M, N, K, wbits == 4 ? K / 2 : K);
    if (rc) return rc;
    MQ_REQUIRE(sa && ws, "gemm_rowscale: null pointer");
    rc = check_gemm_out("gemm_rowscale", bias, bias_dtype, y, y_dtype, ldy, N);
    if (rc) return rc;
    MQ_REQUIRE(workspace_bytes >= 0 && (!workspace || aligned(workspace, 16)),
               "gemm_rowscale: workspace must be 16-byte aligned");
    GemmArgs a{};
    a.qa = qa; a.lda = lda; a.sa = sa; a.qw = static_cast<const uint8_t*>(qw); a.ldw = ldw; a.ws32 = ws;
    a.bias = bias; a.bias_dtype = bias_dtype; a.y = y; a.y_dtype = y_dtype; a.ldy = ldy; a.M = M; a.N = N; a.K = K;
    a.work = workspace; a.work_bytes = workspace ? workspace_bytes : 0;
    a.wtile = tile16;
    *out = a;
    *wk = wbits == 4 ? WKind::I4Sym : WKind::I8;
    return MQ_OK;
}

}  // namespace

extern "C" {

int mq_gemm_w4_group_ws(const int8_t* qa, int64_t lda, const float* sa, const uint8_t* qw, int64_t ldw,
                        const uint16_t* ws, int64_t ldws, const uint8_t* wz, int64_t ldwz, int group, int act_mode,
                        const void* bias, int bias_dtype, void* y, int y_dtype, int64_t ldy, int64_t M, int64_t N,
                        int64_t K, void* workspace, int64_t workspace_bytes, void* stream) {
    clear_error();
    GemmArgs a;
    const int rc = w4_group_args(qa, lda, sa, qw, ldw, ws, ldws, wz, ldwz, group, act_mode, bias, bias_dtype, y,
                                 y_dtype, ldy, M, N, K, workspace, workspace_bytes, &a);
    if (rc) return rc == kEmpty ? MQ_OK : rc;
    return launch_gemm(a, wz ? WKind::U4Asym : WKind::I4Sym, Epi::GroupScale, static_cast<hipStream_t>(stream));
}

int mq_gemm_w4_group(const int8_t* qa, int64_t lda, const float* sa, const uint8_t* qw, int64_t ldw,
                     const uint16_t* ws, int64_t ldws, const uint8_t* wz, int64_t ldwz, int group, int act_mode,
                     const void* bias, int bias_dtype, void* y, int y_dtype, int64_t ldy, int64_t M, int64_t N,
                     int64_t K, void* stream) {
    return mq_gemm_w4_group_ws(qa, lda, sa, qw, ldw, ws, ldws, wz, ldwz, group, act_mode, bias, bias_dtype, y,
                               y_dtype, ldy, M, N, K, nullptr, 0, stream);
}

int mq_gemm_w4_group_partials(const int8_t* qa, int64_t lda, const uint8_t* qw, int64_t ldw, const uint8_t* wz,
                              int64_t ldwz, int group, int act_mode, int32_t* part, int64_t M, int64_t N, int64_t K,
                              void* stream) {
    clear_error();
    MQ_REQUIRE(group == 64, "gemm_w4_group_partials: quant group size must be 64 (got %d)", group);
    MQ_REQUIRE(act_mode >= MQ_ACT_I8 && act_mode <= MQ_ACT_X16ALT, "gemm_w4_group_partials: unknown act_mode %d",
               act_mode);
    int rc = check_gemm_common(qa, lda, qw, ldw, M, N, K, K / 2);
    if (rc) return rc == kEmpty ? MQ_OK : rc;
    MQ_REQUIRE(part, "gemm_w4_group_partials: null pointer");
    MQ_REQUIRE(!wz || ldwz >= (K / group + 1) / 2, "gemm_w4_group_partials: ldwz < ceil(K/group/2)");
    GemmArgs a{};
    a.qa = qa; a.lda = lda; a.qw = qw; a.ldw = ldw; a.wz = wz; a.ldwz = ldwz; a.part = part;
    a.M = M; a.N = N; a.K = K; a.act_mode = act_mode;
    return launch_gemm(a, wz ? WKind::U4Asym : WKind::I4Sym, Epi::GroupPartials, static_cast<hipStream_t>(stream));
}

int mq_gemm_rowscale_ws(const int8_t* qa, int64_t lda, const float* sa, const void* qw, int64_t ldw, int wbits,
                        const float* ws, const void* bias, int bias_dtype, void* y, int y_dtype, int64_t ldy,
                        int64_t M, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, void* stream) {
    clear_error();
    GemmArgs a;
    WKind wk;
    const int rc = rowscale_args(qa, lda, sa, qw, ldw, wbits, ws, bias, bias_dtype, y, y_dtype, ldy, M, N, K, workspace,
                                 workspace_bytes, &a, &wk);
    if (rc) return rc == kEmpty ? MQ_OK : rc;
    return launch_gemm(a, wk, Epi::RowScale, static_cast<hipStream_t>(stream));
}

int mq_gemm_rowscale(const int8_t* qa, int64_t lda, const float* sa, const void* qw, int64_t ldw, int wbits,
                     const float* ws, const void* bias, int bias_dtype, void* y, int y_dtype, int64_t ldy,
                     int64_t M, int64_t N, int64_t K, void* stream) {
    return mq_gemm_rowscale_ws(qa, lda, sa, qw, ldw, wbits, ws, bias, bias_dtype, y, y_dtype, ldy, M, N, K, nullptr,
                               0, stream);
}

int64_t mq_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    // the larger of what the group-scale and the row-scale GEMM would use
    return std::max(workspace_bytes(M, N, K, false), workspace_bytes(M, N, K, true));
}

int mq_gemm_rowscale_acc(const int8_t* qa, int64_t lda, const void* qw, int64_t ldw, int wbits, int32_t* acc,
                         int64_t M, int64_t N, int64_t K, void* stream) {
    clear_error();
    const bool tile16 = (wbits & MQ_W8_TILE16) != 0;
    wbits &= ~MQ_W8_TILE16;
    MQ_REQUIRE(wbits == 4 || wbits == 8, "gemm_rowscale_acc: wbits must be 4 or 8 (got %d)", wbits);
    int rc = check_tile16("gemm_rowscale_acc", tile16, wbits, N, K, &ldw);
    if (rc) return rc;
    rc = check_gemm_common(qa, lda, qw, ldw, M, N, K, wbits == 4 ? K / 2 : K);
    if (rc) return rc == kEmpty ? MQ_OK : rc;
    MQ_REQUIRE(acc, "gemm_rowscale_acc: null pointer");
    GemmArgs a{};
    a.qa = qa; a.lda = lda; a.qw = static_cast<const uint8_t*>(qw); a.ldw = ldw; a.part = acc;
    a.M = M; a.N = N; a.K = K;
    a.wtile = tile16;
    return launch_gemm(a, wbits == 4 ? WKind::I4Sym : WKind::I8, Epi::RowAcc, static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace {

constexpr int64_t kWsAlign = 256;
int64_t align_up(int64_t v) { return (v + kWsAlign - 1) / kWsAlign * kWsAlign; }

// Workspace layout of the whole-linear entry points: codes [M, K] int8, scales [M] fp32, then the
// GEMM's split-K partials. `need` is what the linear cannot run without.
struct LinearWs {
    int64_t codes = 0, scales = 0, split = 0, need = 0, total = 0;
};

LinearWs linear_ws(int64_t M, int64_t N, int64_t K) {
    LinearWs w;
    w.codes = 0;
    // codes for M rows rounded up to 16: in the 16-row tile layout the last band spans 16 rows
    // whatever M is (its rows past M are never written or read)
    w.scales = align_up((M + 15) / 16 * 16 * K);
    w.split = w.scales + align_up(M * 4);
    w.need = w.split;
    w.total = w.split + align_up(mq_gemm_workspace_bytes(M, N, K));
    return w;
}

// Shared argument checks of the whole-linear entry points (the GEMM and quantizer entry points
// check the rest); returns MQ_OK, an error, or kEmpty for a valid call with nothing to compute.
int check_linear(const char* what, int act_bits, int swiglu, int64_t M, int64_t N, int64_t K, const void* workspace,
                 int64_t workspace_bytes) {
    MQ_REQUIRE(act_bits == 8 || act_bits == 4, "%s: act_bits must be 8 or 4 (got %d)", what, act_bits);
    MQ_REQUIRE(swiglu == MQ_SWIGLU_NONE || swiglu == MQ_SWIGLU_FUSED || swiglu == MQ_SWIGLU_EAGER,
               "%s: swiglu must be 0 (none), 1 (fused) or 2 (eager), got %d", what, swiglu);
    MQ_REQUIRE(M >= 0 && N >= 0 && K > 0 && K % 64 == 0, "%s: bad shape M=%lld N=%lld K=%lld (K %% 64 == 0)", what,
               (long long)M, (long long)N, (long long)K);
    MQ_REQUIRE(M < (int64_t(1) << 31), "%s: M too large", what);
    if (M == 0 || N == 0) return kEmpty;
    const LinearWs w = linear_ws(M, N, K);
    MQ_REQUIRE(workspace && aligned(workspace, kWsAlign),
               "%s: workspace must be non-null and 256-byte aligned", what);
    MQ_REQUIRE(workspace_bytes >= w.need, "%s: workspace of %lld bytes is below the %lld the codes and scales need",
               what, (long long)workspace_bytes, (long long)w.need);
    return MQ_OK;
}

// tiled: the codes in 16-row tiles [ceil(M / 16)][K / 64][16][64] (GemmArgs::atile) instead of rows
// of K bytes; the kernels take that layout from a row stride of 0
int quantize_into(const void* x, int x_dtype, int64_t ldx, int hblock, int act_bits, int swiglu, int layout,
                  bool tiled, int64_t M, int64_t K, uint8_t* ws_base, void* stream) {
    const LinearWs w = linear_ws(M, 1, K);
    void* q = ws_base + w.codes;
    float* s = reinterpret_cast<float*>(ws_base + w.scales);
    if (!tiled)
        return swiglu ? mq_swiglu_rotquant(x, x_dtype, M, K, ldx, hblock, act_bits, layout, swiglu, q, K, s, stream)
                      : mq_rotquant(x, x_dtype, M, K, ldx, hblock, act_bits, layout, q, K, s, stream);
    const int rc = swiglu ? check_rotquant("swiglu_rotquant", x, x_dtype, false, M, K, 2 * K, ldx, hblock, act_bits,
                                           layout, q, K, s)
                          : check_rotquant("rotquant", x, x_dtype, true, M, K, K, ldx, hblock, act_bits, layout, q, K,
                                           s);
    if (rc != MQ_OK) return rc;
    auto* xs = static_cast<const uint16_t*>(x);
    auto* st = static_cast<hipStream_t>(stream);
    if (swiglu) return launch_swiglu(swiglu, x_dtype, xs, M, K, ldx, hblock, act_bits, layout, q, 0, s, st);
    if (x_dtype == MQ_DT_F32)
        return launch_rotquant_f32(static_cast<const float*>(x), M, K, ldx, hblock, act_bits, layout, q, 0, s, st);
    return x_dtype == MQ_DT_F16 ? launch_rotquant_f16(xs, M, K, ldx, hblock, act_bits, layout, q, 0, s, st)
                                : launch_rotquant_bf16(xs, M, K, ldx, hblock, act_bits, layout, q, 0, s, st);
}

// A one-row linear whose product runs on the GEMV (gemv_quantizes_row): the GEMV rotates and
// quantizes the row in its prologue, one launch, with the rotate+quantize entry's argument checks
// and its codes and scale (the workspace is then not written).
int launch_fused_row(GemmArgs& a, WKind wk, Epi epi, const void* x, int x_dtype, int64_t ldx, int hblock,
                     int act_bits, int layout, uint8_t* ws_base, void* stream) {
    const LinearWs w = linear_ws(1, 1, a.K);
    const int rc = check_rotquant("rotquant", x, x_dtype, true, 1, a.K, a.K, ldx, hblock, act_bits, layout,
                                  ws_base + w.codes, a.K, reinterpret_cast<const float*>(ws_base + w.scales));
    if (rc != MQ_OK) return rc;
    a.x = x;
    a.x_dtype = x_dtype;
    a.hblock = hblock;
    a.x_bits = act_bits;
    return launch_gemm(a, wk, epi, static_cast<hipStream_t>(stream));
}

}  // namespace

extern "C" {

int64_t mq_linear_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    return linear_ws(M, N, K).total;
}

int mq_linear_w4_group(const void* x, int x_dtype, int64_t ldx, int hblock, int act_bits, int swiglu,
                       const uint8_t* qw, int64_t ldw, const uint16_t* ws, int64_t ldws, const uint8_t* wz,
                       int64_t ldwz, const void* bias, int bias_dtype, void* y, int y_dtype, int64_t ldy, int64_t M,
                       int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, void* stream) {
    clear_error();
    const int expanded = act_bits & MQ_W4_EXPANDED;
    act_bits &= ~MQ_W4_EXPANDED;
    int rc = check_linear("linear_w4_group", act_bits, swiglu, M, N, K, workspace, workspace_bytes);
    if (rc) return rc == kEmpty ? MQ_OK : rc;
    // int4 activations enter the group GEMM in its x16 operand layout
    const int layout = act_bits == 4 ? MQ_Q_X16ALT : MQ_Q_BYTES;
    const int act_mode = (act_bits == 4 ? MQ_ACT_X16ALT : MQ_ACT_I8) | expanded;
    auto* base = static_cast<uint8_t*>(workspace);
    const LinearWs w = linear_ws(M, N, K);
    GemmArgs a;
    rc = w4_group_args(reinterpret_cast<const int8_t*>(base + w.codes), K,
                       reinterpret_cast<const float*>(base + w.scales), qw, ldw, ws, ldws, wz, ldwz, 64, act_mode, bias,
                       bias_dtype, y, y_dtype, ldy, M, N, K, base + w.split, workspace_bytes - w.split, &a);
    if (rc) return rc == kEmpty ? MQ_OK : rc;
    const WKind wk = wz ? WKind::U4Asym : WKind::I4Sym;
    a.atile = 1;   // the codes in 16-row tiles wherever the wide kernel reads them
    a.atile = gemm_runs_wide(a, wk, Epi::GroupScale);
    if (a.wtile && !a.atile) {
        set_error("linear_w4_group: expanded 4-bit weights are read by the wide kernel only (M > 4, operands under "
                  "2 GiB); pass the packed weights");
        return MQ_EUNSUPPORTED;
    }
    if (swiglu == MQ_SWIGLU_NONE && gemv_quantizes_row(a, wk, Epi::GroupScale))
        return launch_fused_row(a, wk, Epi::GroupScale, x, x_dtype, ldx, hblock, act_bits, layout, base, stream);
    rc = quantize_into(x, x_dtype, ldx, hblock, act_bits, swiglu, layout, a.atile, M, K, base, stream);
    if (rc) return rc;
    return launch_gemm(a, wk, Epi::GroupScale, static_cast<hipStream_t>(stream));
}

int mq_linear_rowscale(const void* x, int x_dtype, int64_t ldx, int hblock, int act_bits, int swiglu, const void* qw,
                       int64_t ldw, int wbits, const float* ws, const void* bias, int bias_dtype, void* y,
                       int y_dtype, int64_t ldy, int64_t M, int64_t N, int64_t K, void* workspace,
                       int64_t workspace_bytes, void* stream) {
    clear_error();
    int rc = check_linear("linear_rowscale", act_bits, swiglu, M, N, K, workspace, workspace_bytes);
    if (rc) return rc == kEmpty ? MQ_OK : rc;
    auto* base = static_cast<uint8_t*>(workspace);
    const LinearWs w = linear_ws(M, N, K);
    GemmArgs a;
    WKind wk;
    rc = rowscale_args(reinterpret_cast<const int8_t*>(base + w.codes), K, reinterpret_cast<const float*>(base + w.scales),
                       qw, ldw, wbits, ws, bias, bias_dtype, y, y_dtype, ldy, M, N, K, base + w.split,
                       workspace_bytes - w.split, &a, &wk);
    if (rc) return rc == kEmpty ? MQ_OK : rc;
    a.atile = 1;   // the codes in 16-row tiles wherever the wide kernel reads them
    a.atile = gemm_runs_wide(a, wk, Epi::RowScale);
    if (swiglu == MQ_SWIGLU_NONE && gemv_quantizes_row(a, wk, Epi::RowScale))
        return launch_fused_row(a, wk, Epi::RowScale, x, x_dtype, ldx, hblock, act_bits, MQ_Q_BYTES, base, stream);
    rc = quantize_into(x, x_dtype, ldx, hblock, act_bits, swiglu, MQ_Q_BYTES, a.atile, M, K, base, stream);
    if (rc) return rc;
    return launch_gemm(a, wk, Epi::RowScale, static_cast<hipStream_t>(stream));
}

}  // extern "C"

// ---- The whole W4 group linear without a caller workspace (mq_linear_w4_group_noalloc): its codes,
// scales and split-K partials go to a fixed device array instead. Each GPU the library runs on
// holds its own copy of the array until the process ends. The host-side name `scratch` is only a
// stand-in for the symbol: its device address on the current GPU comes from hipGetSymbolAddress,
// taken once per device and kept.
namespace mq {

constexpr int64_t kScratchBytes = MQ_NOALLOC_SCRATCH_BYTES;
__device__ __attribute__((aligned(256))) uint8_t scratch[kScratchBytes];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of the current GPU's scratch array (looked up on its first use on that GPU).
int scratch_on_current_device(const char* what, void** out) {
    int dev = 0;
    const hipError_t ed = hipGetDevice(&dev);
    if (ed != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) {
        set_error("%s: no usable current device (%s)", what, hipGetErrorString(ed));
        return MQ_ELAUNCH;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            set_error("%s: cannot find the scratch array on device %d: %s", what, dev, hipGetErrorString(e));
            return MQ_ELAUNCH;
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return MQ_OK;
}

}  // namespace
}  // namespace mq

extern "C" {

int mq_linear_w4_group_noalloc(const void* x, int x_dtype, int64_t ldx, int hblock, int act_bits, int swiglu,
                               const uint8_t* qw, int64_t ldw, const uint16_t* ws, int64_t ldws, const uint8_t* wz,
                               int64_t ldwz, const void* bias, int bias_dtype, void* y, int y_dtype, int64_t ldy,
                               int64_t M, int64_t N, int64_t K, void* stream) {
    clear_error();
    if (M > 0 && N > 0 && K > 0) {
        const LinearWs w = linear_ws(M, N, K);
        if (w.need > kScratchBytes) {
            set_error("linear_w4_group_noalloc: the codes and scales of M=%lld K=%lld need %lld bytes, more than "
                      "the fixed scratch of %lld bytes",
                      (long long)M, (long long)K, (long long)w.need, (long long)kScratchBytes);
            return MQ_EINVAL;
        }
        void* ptr = nullptr;
        const int rc = scratch_on_current_device("linear_w4_group_noalloc", &ptr);
        if (rc) return rc;
        return mq_linear_w4_group(x, x_dtype, ldx, hblock, act_bits, swiglu, qw, ldw, ws, ldws, wz, ldwz, bias,
                                  bias_dtype, y, y_dtype, ldy, M, N, K, ptr, std::min(w.total, kScratchBytes),
                                  stream);
    }
    // empty or invalid shapes: the ordinary entry point's checks and messages (nothing is launched)
    return mq_linear_w4_group(x, x_dtype, ldx, hblock, act_bits, swiglu, qw, ldw, ws, ldws, wz, ldwz, bias, bias_dtype,
                              y, y_dtype, ldy, M, N, K, nullptr, 0, stream);
}

}  // extern "C"

