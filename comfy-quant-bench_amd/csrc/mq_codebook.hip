// Load-time decode of comfy-kitchen's shipped asym_w4a8_int8 weights (4-bit codebook indices,
// fp8 e4m3fn per-group scales s_rel, per-row s_channel) to an int8 weight whose per-row scale is
// the stored s_channel, the form the int8 row-scale GEMM takes. comfy-kitchen finishes a decoded
// W4A8 weight as dequantize_int8_convrot_weight_dtype(int8_weight, s_channel, ...)
// (patches/comfy_kitchen_w4a8_dequant_fused.patch:15-18): the int8 weight's row scale is s_channel
// unchanged, so level * s_rel is already in int8 units and
//
//   t[n,k]  = fp32(level(code[n,k]) * fp8(s_rel[n, k / gs]))   level = codebook[code], or the
//                                                               signed nibble without a codebook
//   q8[n,k] = clamp(rne(t[n,k]), -127, 127)                     (0 where t is NaN)
//   row_scale[n] = s_channel[n]
//
// One 256-thread workgroup per weight row, one pass; each thread takes 8 consecutive k per step
// (one dword of packed codes in, 8 bytes out). The decode runs once per weight; it is HBM-bound
// at 1.5 bytes per weight element.
#include "mq_device.h"
#include "mq_internal.h"

#pragma clang fp contract(off)

namespace mq {
namespace {

constexpr int kThreads = 256;

// OCP fp8 e4m3fn -> fp32, exact (bias 7; e = 0 subnormal; S.1111.111 NaN, no infinities).
__device__ __forceinline__ float fp8_e4m3fn(uint32_t b) {
    const uint32_t e = (b >> 3) & 0xfu, m = b & 7u;
    float v;
    if (e == 0) v = static_cast<float>(m) * 0x1p-9f;
    else v = __uint_as_float(((e + 120u) << 23) | (m << 20));
    if (e == 0xfu && m == 7u) v = __builtin_nanf("");
    return (b & 0x80u) ? -v : v;
}

__global__ void __launch_bounds__(kThreads)
decode_kernel(const uint8_t* __restrict__ qdata, int64_t ldq, const uint8_t* __restrict__ s_rel, int64_t lds,
              const float* __restrict__ s_channel, const float* __restrict__ codebook, int gs, int K,
              int8_t* __restrict__ q8, int64_t ldq8, float* __restrict__ row_scale) {
    __shared__ float lev[16];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    if (tid < 16) lev[tid] = codebook ? codebook[tid] : static_cast<float>(tid >= 8 ? tid - 16 : tid);
    if (tid == 0) row_scale[row] = s_channel[row];
    __syncthreads();
    const uint8_t* qr = qdata + row * ldq;
    const uint8_t* sr = s_rel + row * lds;
    int8_t* out = q8 + row * ldq8;
    for (int k0 = tid * 8; k0 < K; k0 += kThreads * 8) {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(qr + k0 / 2);
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float t = lev[(w >> (4 * i)) & 0xfu] * fp8_e4m3fn(sr[(k0 + i) / gs]);
            float q = __builtin_rintf(t);
            q = __builtin_fminf(__builtin_fmaxf(q, -127.0f), 127.0f);
            if (t != t) q = 0.0f;
            const uint32_t byte = static_cast<uint32_t>(static_cast<int>(q)) & 0xffu;
            if (i < 4) lo |= byte << (8 * i);
            else hi |= byte << (8 * (i - 4));
        }
        *reinterpret_cast<uint2*>(out + k0) = uint2{lo, hi};
    }
}

}  // namespace

int launch_decode_w4a8_codebook(const uint8_t* qdata, int64_t ldq, const uint8_t* s_rel, int64_t lds,
                                const float* s_channel, const float* codebook, int group_size, int64_t N,
                                int64_t K, int8_t* q8, int64_t ldq8, float* row_scale, hipStream_t stream) {
    hipLaunchKernelGGL(decode_kernel, dim3(static_cast<unsigned>(N)), dim3(kThreads), 0, stream, qdata, ldq, s_rel,
                       lds, s_channel, codebook, group_size, static_cast<int>(K), q8, ldq8, row_scale);
    return launch_status("decode_w4a8_codebook");
}

}  // namespace mq
