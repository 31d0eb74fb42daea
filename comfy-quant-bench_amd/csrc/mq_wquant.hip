// Offline weight quantizer (the converter side of the path): rotate each weight row by H_hblock and
// quantize it to one of the GEMMs' weight formats.
//
// One 256-thread workgroup per weight row. The row is staged in LDS as fp32 (K <= 32768, 128 KB),
// rotated in place by the pinned radix-4 FWHT (experiments/qwen21-kernel/kernels/g64_quant.cu:68-86:
// stages with element strides 1, 4, 16, 64, h = 0.5f * (((x0 + x1) + x2) + x3), y_i = h - x_{3-i},
// the same fp32 operations as the activation kernel and the torch / numpy quantizers), then
// quantized with IEEE divisions:
//   U4_ASYM_G64  lo = min(min w, 0), hi = max(max w, 0), s = fp16((hi - lo) / 15),
//                z = clamp(rne(-lo / s), 0, 15), q = clamp(rne(w / s) + z, 0, 15); s = 0 -> q = z = 0
//   I4_SYM_G64   s = fp16(max |w| / 7), q = clamp(rne(w / s), -7, 7); s = 0 -> q = 0
//   I4_ROW       s = max(max |w|, 1e-10) / 7,   q = clamp(rne(w / s), -7, 7)
//   I8_ROW       s = max(max |w|, 1e-10) / 127, q = clamp(rne(w / s), -127, 127)
// (the group formats are the configs' schemes, with the min / max code choice of
// custom_nodes/comfy-lowbit-loader/formats.py:131-149 and the symmetric form of
// tools/svdquant_probe.py:105-115; the row formats are tools/gptq_w4a4.py:197-203 and
// tools/_formats.py:128-167). The quantizer runs once per weight, so it favours a simple exact
// structure over speed: the row is read once from HBM and each output byte written once.
#include "mq_device.h"
#include <algorithm>
#include "mq_internal.h"

#pragma clang fp contract(off)

namespace mq {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxK = 32768;
constexpr int kMaxGroups = kMaxK / 64;

template <int DT>
__device__ __forceinline__ float load_w(const void* w, int64_t i) {
    if constexpr (DT == 0) return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(w)[i]) << 16);
    else if constexpr (DT == 1) return static_cast<float>(static_cast<const _Float16*>(w)[i]);
    else return static_cast<const float*>(w)[i];
}

__device__ __forceinline__ float clampf(float v, float lo, float hi) { return __builtin_fminf(__builtin_fmaxf(v, lo), hi); }

// Maximum over the workgroup (every thread gets it); red holds one float per wavefront.
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int i = 1; i < kThreads / 64; ++i) m = __builtin_fmaxf(m, red[i]);
    return m;
}

template <int DT, int FMT>
__global__ void __launch_bounds__(kThreads)
wquant_kernel(const void* __restrict__ w, int64_t ldw, int K, int hblock, uint8_t* __restrict__ q, int64_t ldq,
              void* __restrict__ scale, int64_t ld_scale, uint8_t* __restrict__ zero, int64_t ld_zero) {
    extern __shared__ float row[];                    // K fp32 values
    __shared__ float gs[kMaxGroups];                  // per-group scale (fp32 value of the fp16)
    __shared__ float gz[kMaxGroups];                  // per-group zero-point
    __shared__ float red[kThreads / 64];
    const int tid = threadIdx.x;
    const int64_t n = blockIdx.x;

    for (int i = tid; i < K; i += kThreads) row[i] = load_w<DT>(w, n * ldw + i);
    __syncthreads();

    // pinned radix-4 FWHT: butterfly b of a stage with stride st has x_j at i0 + j st,
    // i0 = (b / st) 4 st + b % st (4 st divides hblock, so butterflies never straddle blocks)
    for (int st = 1; st < hblock; st *= 4) {
        for (int b = tid; b < K / 4; b += kThreads) {
            const int i0 = (b / st) * 4 * st + b % st;
            const float x0 = row[i0], x1 = row[i0 + st], x2 = row[i0 + 2 * st], x3 = row[i0 + 3 * st];
            const float h = 0.5f * (((x0 + x1) + x2) + x3);
            row[i0] = h - x3;
            row[i0 + st] = h - x2;
            row[i0 + 2 * st] = h - x1;
            row[i0 + 3 * st] = h - x0;
        }
        __syncthreads();
    }

    if constexpr (FMT == 0 || FMT == 1) {
        const int G = K / 64;
        uint16_t* s16 = static_cast<uint16_t*>(scale) + n * ld_scale;
        for (int g = tid; g < G; g += kThreads) {
            const float* v = row + 64 * g;
            float s;
            if constexpr (FMT == 0) {
                float mn = v[0], mx = v[0];
                for (int e = 1; e < 64; ++e) {
                    mn = __builtin_fminf(mn, v[e]);
                    mx = __builtin_fmaxf(mx, v[e]);
                }
                const float lo = __builtin_fminf(mn, 0.0f), hi = __builtin_fmaxf(mx, 0.0f);
                const _Float16 h = static_cast<_Float16>((hi - lo) / 15.0f);
                s = static_cast<float>(h);
                gz[g] = s == 0.0f ? 0.0f : clampf(__builtin_rintf(-lo / s), 0.0f, 15.0f);
                s16[g] = __builtin_bit_cast(uint16_t, h);
            } else {
                float am = 0.0f;
                for (int e = 0; e < 64; ++e) am = __builtin_fmaxf(am, __builtin_fabsf(v[e]));
                const _Float16 h = static_cast<_Float16>(am / 7.0f);
                s = static_cast<float>(h);
                s16[g] = __builtin_bit_cast(uint16_t, h);
            }
            gs[g] = s;
        }
        __syncthreads();
        // eight consecutive codes per thread step: one packed dword
        uint8_t* qr = q + n * ldq;
        for (int i = 8 * tid; i < K; i += 8 * kThreads) {
            const int g = i / 64;
            const float s = gs[g];
            uint32_t word = 0;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                int c = 0;
                if (s != 0.0f) {
                    if constexpr (FMT == 0) c = static_cast<int>(clampf(__builtin_rintf(row[i + e] / s) + gz[g], 0.0f, 15.0f));
                    else c = static_cast<int>(clampf(__builtin_rintf(row[i + e] / s), -7.0f, 7.0f));
                }
                word |= (static_cast<uint32_t>(c) & 0xfu) << (4 * e);
            }
            *reinterpret_cast<uint32_t*>(qr + i / 2) = word;
        }
        if constexpr (FMT == 0) {
            uint8_t* zr = zero + n * ld_zero;
            for (int j = tid; j < (G + 1) / 2; j += kThreads) {
                const uint32_t z0 = static_cast<uint32_t>(gz[2 * j]);
                const uint32_t z1 = 2 * j + 1 < G ? static_cast<uint32_t>(gz[2 * j + 1]) : 0u;
                zr[j] = static_cast<uint8_t>(z0 | (z1 << 4));
            }
        }
    } else {
        constexpr float L = FMT == 2 ? 7.0f : 127.0f;
        float am = 0.0f;
        for (int i = tid; i < K; i += kThreads) am = __builtin_fmaxf(am, __builtin_fabsf(row[i]));
        am = block_max(am, red);
        const float s = __builtin_fmaxf(am, 1e-10f) / L;
        if (tid == 0) static_cast<float*>(scale)[n] = s;
        uint8_t* qr = q + n * ldq;
        for (int i = 8 * tid; i < K; i += 8 * kThreads) {
            int c[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) c[e] = static_cast<int>(clampf(__builtin_rintf(row[i + e] / s), -L, L));
            if constexpr (FMT == 2) {
                uint32_t word = 0;
#pragma unroll
                for (int e = 0; e < 8; ++e) word |= (static_cast<uint32_t>(c[e]) & 0xfu) << (4 * e);
                *reinterpret_cast<uint32_t*>(qr + i / 2) = word;
            } else {
                uint32_t lo = 0, hi = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    lo |= (static_cast<uint32_t>(c[e]) & 0xffu) << (8 * e);
                    hi |= (static_cast<uint32_t>(c[e + 4]) & 0xffu) << (8 * e);
                }
                *reinterpret_cast<uint2*>(qr + i) = uint2{lo, hi};
            }
        }
    }
}

template <int DT, int FMT>
int launch_fmt(const void* w, int64_t ldw, int64_t N, int64_t K, int hblock, void* q, int64_t ldq, void* scale,
               int64_t ld_scale, void* zero, int64_t ld_zero, hipStream_t stream) {
    auto kern = wquant_kernel<DT, FMT>;
    const size_t lds = static_cast<size_t>(K) * sizeof(float);
    if (lds > 65536 && hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) != hipSuccess) {
        set_error("quantize_weight: cannot reserve %zu bytes of LDS", lds);
        return -3;
    }
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(N)), dim3(kThreads), lds, stream, w, ldw, static_cast<int>(K),
                       hblock, static_cast<uint8_t*>(q), ldq, scale, ld_scale, static_cast<uint8_t*>(zero), ld_zero);
    return launch_status("quantize_weight");
}

template <int DT>
int launch_dt(const void* w, int64_t ldw, int64_t N, int64_t K, int hblock, int format, void* q, int64_t ldq,
              void* scale, int64_t ld_scale, void* zero, int64_t ld_zero, hipStream_t stream) {
    switch (format) {
        case 0: return launch_fmt<DT, 0>(w, ldw, N, K, hblock, q, ldq, scale, ld_scale, zero, ld_zero, stream);
        case 1: return launch_fmt<DT, 1>(w, ldw, N, K, hblock, q, ldq, scale, ld_scale, zero, ld_zero, stream);
        case 2: return launch_fmt<DT, 2>(w, ldw, N, K, hblock, q, ldq, scale, ld_scale, zero, ld_zero, stream);
        case 3: return launch_fmt<DT, 3>(w, ldw, N, K, hblock, q, ldq, scale, ld_scale, zero, ld_zero, stream);
        default: break;
    }
    set_error("quantize_weight: unknown format %d", format);
    return -1;
}

// int8 weights [N, K] (row stride ldw) to 16-row tiles [ceil(N / 16)][K / 64][16][64]: one thread
// per 16-byte unit u of the output, u = ((band * G + g) * 16 + row) * 4 + chunk; rows past N get 0.
__global__ void __launch_bounds__(256) tile16_kernel(const uint8_t* w, int64_t ldw, int64_t N, int64_t K,
                                                    uint8_t* out) {
    const int64_t G = K / 64, units = (N + 15) / 16 * 16 * (K / 16);
    for (int64_t u = blockIdx.x * int64_t(256) + threadIdx.x; u < units; u += int64_t(gridDim.x) * 256) {
        const int64_t chunk = u & 3, row = (u >> 2) & 15, g = (u >> 6) % G, band = (u >> 6) / G;
        const int64_t n = band * 16 + row;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (n < N) v = *reinterpret_cast<const uint4*>(w + n * ldw + g * 64 + chunk * 16);
        *reinterpret_cast<uint4*>(out + u * 16) = v;
    }
}

// Packed 4-bit weights [N, K/2] (row stride ldw bytes) expanded to int8 in the same 16-row tiles,
// one thread per 16-byte unit as in tile16_kernel. A unit holds 16 consecutive k of one row and
// K group g (its 8 packed bytes); value v = q - z (uint4 with zero-point nibble z of group g) or
// the signed nibble, then by layout: 0 (the group GEMM's int8 activation layout) negated in odd
// groups, 2 (its x16 int4 layout) 16 * v for signed weights, 3 (row scale) v as it is.
__global__ void __launch_bounds__(256) expand_w4_kernel(const uint8_t* qw, int64_t ldw, const uint8_t* wz,
                                                       int64_t ldwz, int64_t N, int64_t K, int layout,
                                                       uint8_t* out) {
    const int64_t G = K / 64, units = (N + 15) / 16 * 16 * (K / 16);
    for (int64_t u = blockIdx.x * int64_t(256) + threadIdx.x; u < units; u += int64_t(gridDim.x) * 256) {
        const int64_t chunk = u & 3, row = (u >> 2) & 15, g = (u >> 6) % G, band = (u >> 6) / G;
        const int64_t n = band * 16 + row;
        uint32_t o[4] = {0u, 0u, 0u, 0u};
        if (n < N) {
            const uint2 w = *reinterpret_cast<const uint2*>(qw + n * ldw + g * 32 + chunk * 8);
            const int z = wz ? (wz[n * ldwz + (g >> 1)] >> (4 * (g & 1))) & 15 : 0;
            const bool neg = layout == 0 && (g & 1);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t byte = (e < 8 ? w.x >> (8 * (e >> 1)) : w.y >> (8 * ((e - 8) >> 1))) & 0xffu;
                const int q = (byte >> (4 * (e & 1))) & 15;
                int v = wz ? q - z : (q >= 8 ? q - 16 : q);
                if (neg) v = -v;
                if (layout == 2 && !wz) v *= 16;
                o[e >> 2] |= (static_cast<uint32_t>(v) & 0xffu) << (8 * (e & 3));
            }
        }
        *reinterpret_cast<uint4*>(out + u * 16) = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

// fp16 group scales [N, G] (row stride ldws) as the expanded-weight group GEMM's lanes load them:
// dword [g][c][u] (u fastest, ld dwords per [g][c]) = ws[32 u + c, g] | ws[32 u + 16 + c, g] << 16,
// zero for columns past N and groups past G; G4 groups in all (G rounded up to four).
__global__ void __launch_bounds__(256) expand_scales_kernel(const uint16_t* ws, int64_t ldws, int64_t N, int64_t G,
                                                           int64_t G4, int64_t ld, uint32_t* out) {
    const int64_t total = G4 * 16 * ld;
    for (int64_t i = blockIdx.x * int64_t(256) + threadIdx.x; i < total; i += int64_t(gridDim.x) * 256) {
        const int64_t u = i % ld, c = (i / ld) % 16, g = i / (16 * ld);
        const int64_t n0 = 32 * u + c, n1 = n0 + 16;
        uint32_t v = 0u;
        if (g < G) {
            if (n0 < N) v = ws[n0 * ldws + g];
            if (n1 < N) v |= static_cast<uint32_t>(ws[n1 * ldws + g]) << 16;
        }
        out[i] = v;
    }
}

}  // namespace

int launch_expand_scales_w4(const uint16_t* ws, int64_t ldws, int64_t N, int64_t K, uint32_t* out,
                            hipStream_t stream) {
    const int64_t G = K / 64, G4 = (G + 3) / 4 * 4, ld = scale_pair_ld(N);
    const int64_t blocks = std::min<int64_t>((G4 * 16 * ld + 255) / 256, 65536);
    hipLaunchKernelGGL(expand_scales_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, ws, ldws, N, G,
                       G4, ld, out);
    return launch_status("expand_scales_w4");
}

int launch_expand_weight_w4(const uint8_t* qw, int64_t ldw, const uint8_t* wz, int64_t ldwz, int64_t N, int64_t K,
                            int layout, uint8_t* out, hipStream_t stream) {
    const int64_t units = (N + 15) / 16 * 16 * (K / 16);
    const int64_t blocks = std::min<int64_t>((units + 255) / 256, 65536);
    hipLaunchKernelGGL(expand_w4_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, qw, ldw, wz, ldwz,
                       N, K, layout, out);
    return launch_status("expand_weight_w4");
}

int launch_tile_weight_i8(const uint8_t* w, int64_t ldw, int64_t N, int64_t K, uint8_t* out, hipStream_t stream) {
    const int64_t units = (N + 15) / 16 * 16 * (K / 16);
    const int64_t blocks = std::min<int64_t>((units + 255) / 256, 65536);
    hipLaunchKernelGGL(tile16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, w, ldw, N, K, out);
    return launch_status("tile_weight_i8");
}

int launch_quantize_weight(const void* w, int dtype, int64_t N, int64_t K, int64_t ldw, int hblock, int format,
                           void* q, int64_t ldq, void* scale, int64_t ld_scale, void* zero, int64_t ld_zero,
                           hipStream_t stream) {
    switch (dtype) {
        case 0: return launch_dt<0>(w, ldw, N, K, hblock, format, q, ldq, scale, ld_scale, zero, ld_zero, stream);
        case 1: return launch_dt<1>(w, ldw, N, K, hblock, format, q, ldq, scale, ld_scale, zero, ld_zero, stream);
        case 2: return launch_dt<2>(w, ldw, N, K, hblock, format, q, ldq, scale, ld_scale, zero, ld_zero, stream);
        default: break;
    }
    set_error("quantize_weight: unknown dtype %d", dtype);
    return -1;
}

}  // namespace mq
