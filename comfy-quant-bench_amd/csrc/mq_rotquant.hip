// Fused Hadamard block rotation + per-token dynamic int8 / int4 quantizer for gfx950.
//
// Arithmetic (bit-exact with the CPU oracle):
//   rotation: the fp32 radix-4 FWHT of experiments/qwen21-kernel/kernels/g64_quant.cu:68-86,
//     stages with element strides 1, 4, 16, 64; each butterfly h = 0.5f*(((x0+x1)+x2)+x3),
//     y_i = h - x_{3-i};
//   quantizer: tools/activation_balance.py:65-71, s = max(absmax/L, 1e-10f),
//     q = clamp(rne(x / s), -L, L) with the IEEE quotient x / s.
//
// Layout: one wavefront per row. A row is processed in chunks of 1024 columns; in a chunk, lane
// L holds the 16 consecutive columns 16L..16L+15 in registers r = 0..15 (two 16-byte loads), so
// register bits r0..r3 are column bits e0..e3 and lane bits L0..L5 are column bits e4..e9.
// The radix-4 stages over e0e1 and e2e3 run in registers. The stage over e4e5 (blocks 64, 256)
// first swaps lane bits L0, L1 with register bits r2, r3 through DPP lane exchanges, and the
// stage over e6e7 (block 256) swaps L2, L3 with r2, r3 the same way; every butterfly then runs in
// registers in the reference's order. Afterwards r0r1 still hold e0e1, so each group of 4
// registers is 4 consecutive codes and stores as one dword (int8) or one 16-bit word (int4).
//
// Quantization without a per-element division: with r = 1/s (IEEE), m = fma(v, r, 1.5*2^23)
// rounds v*r to an integer n. |v*r - v/s| <= 2^-17 and |fl(v/s) - v/s| <= 2^-17 for |v/s| < 128,
// so rint(fl(v/s)) == n unless v*r lies within 2^-16 of a half-integer; those elements (flagged
// by |fma(v, r, -n)| > 0.5 - 2^-15) recompute rint(v / s) with the IEEE division. The clamp to
// [-L, L] never binds on the fast path: |v| <= absmax, so |v*r| <= L (1 + 2^-22).
#include "mq_device.h"
#include "mq_internal.h"

#pragma clang fp contract(off)

namespace mq {
namespace {

constexpr int kWaves = 4;                 // rows per workgroup (one per wavefront)
constexpr float kTieWindow = 0.5f - 0x1p-15f;

// Radix-4 butterflies over register bits J, J+1 (element stride 4^d mapped to register stride 2^J).
template <int J>
__device__ __forceinline__ void stage_reg(float (&v)[16]) {
    constexpr int st = 1 << J;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        if ((r >> J) & 3) continue;
        const float x0 = v[r], x1 = v[r + st], x2 = v[r + 2 * st], x3 = v[r + 3 * st];
        const float h = 0.5f * (((x0 + x1) + x2) + x3);
        v[r] = h - x3;
        v[r + st] = h - x2;
        v[r + 2 * st] = h - x1;
        v[r + 3 * st] = h - x0;
    }
}

// Exchange lane bit B with register bit J: afterwards the value with (lane bit B = u, register
// bit J = w) is the one that was at (lane bit B = w, register bit J = u).
template <int B, int J>
__device__ __forceinline__ void swap_lane_reg(float (&v)[16], int lane) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        if (r & (1 << J)) continue;
        const float x = v[r], y = v[r | (1 << J)];
        float xn, yn;
        if constexpr (B == 0) {
            const float ty = dpp_mov<kQuadPerm0022>(y);
            const float tx = dpp_mov<kQuadPerm1133>(x);
            const bool up = lane & 1;
            xn = up ? ty : x;
            yn = up ? y : tx;
        } else if constexpr (B == 1) {
            const float ty = dpp_mov<kQuadPerm0101>(y);
            const float tx = dpp_mov<kQuadPerm2323>(x);
            const bool up = lane & 2;
            xn = up ? ty : x;
            yn = up ? y : tx;
        } else if constexpr (B == 2) {
            xn = dpp_upd<kRowShr4, 0xA>(x, y);   // lanes 4-7, 12-15 of each row take y from lane-4
            yn = dpp_upd<kRowShl4, 0x5>(y, x);   // lanes 0-3, 8-11 take x from lane+4
        } else {
            static_assert(B == 3, "lane bit");
            xn = dpp_upd<kRowShr8, 0xC>(x, y);   // lanes 8-15 take y from lane-8
            yn = dpp_upd<kRowShl8, 0x3>(y, x);   // lanes 0-7 take x from lane+8
        }
        v[r] = xn;
        v[r | (1 << J)] = yn;
    }
}

template <int BLK>
__device__ __forceinline__ void rotate_chunk(float (&v)[16], int lane) {
    if constexpr (BLK >= 16) {
        stage_reg<0>(v);          // element stride 1  (e0 e1)
        stage_reg<2>(v);          // element stride 4  (e2 e3)
    }
    if constexpr (BLK >= 64) {
        swap_lane_reg<0, 2>(v, lane);
        swap_lane_reg<1, 3>(v, lane);
        stage_reg<2>(v);          // element stride 16 (e4 e5)
    }
    if constexpr (BLK >= 256) {
        swap_lane_reg<2, 2>(v, lane);
        swap_lane_reg<3, 3>(v, lane);
        stage_reg<2>(v);          // element stride 64 (e6 e7)
    }
}

// Column offset (within the chunk) of register group hi (registers 4*hi..4*hi+3) of lane L.
template <int BLK>
__device__ __forceinline__ int group_col(int lane, int hi) {
    if constexpr (BLK >= 256) return 4 * (lane & 15) + 64 * hi + 256 * (lane >> 4);
    else if constexpr (BLK >= 64) return 4 * (lane & 3) + 16 * hi + 64 * (lane >> 2);
    else return 16 * lane + 4 * hi;
}

template <int LIMIT>
__device__ __forceinline__ float quant_magic(float v, float r, float s) {
    float m = __builtin_fmaf(v, r, kMagic);
    const float n = m - kMagic;
    const float d = __builtin_fmaf(v, r, -n);
    if (__builtin_fabsf(d) > kTieWindow) {
        float qf = __builtin_rintf(v / s);
        qf = __builtin_fminf(__builtin_fmaxf(qf, -static_cast<float>(LIMIT)), static_cast<float>(LIMIT));
        m = kMagic + qf;
    }
    return m;
}

// OUT: 0 = int8 codes, 1 = int4 codes one per byte, 2 = int4 codes packed two per byte,
//      3 = int4 codes one per byte as 16 * q, negated in odd 64-column groups (the operand layout
//          the group-scale GEMM takes for int4 activations: exact, and 16x finer in its fp32 step).
template <int BLK, int OUT, int NCH>
__global__ void __launch_bounds__(64 * kWaves)
rotquant_kernel(const uint16_t* __restrict__ x, int64_t ldx, int M, int K,
                uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ scale) {
    constexpr int LIMIT = OUT == 0 ? 127 : 7;
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (row >= M) return;
    const uint16_t* xr = x + row * ldx;

    float v[NCH][16];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int e = c * 1024 + lane * 16;
        if (e < K) {
            const uint4 a = *reinterpret_cast<const uint4*>(xr + e);
            const uint4 b = *reinterpret_cast<const uint4*>(xr + e + 8);
            const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                v[c][2 * j] = bf16lo(w[j]);
                v[c][2 * j + 1] = bf16hi(w[j]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) v[c][j] = 0.0f;
        }
    }

    float am = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        rotate_chunk<BLK>(v[c], lane);
#pragma unroll
        for (int j = 0; j < 16; ++j) am = __builtin_fmaxf(am, __builtin_fabsf(v[c][j]));
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) am = __builtin_fmaxf(am, __shfl_xor(am, o, 64));

    const float s = __builtin_fmaxf(am / static_cast<float>(LIMIT), 1e-10f);
    const float r = 1.0f / s;
    if (lane == 0) scale[row] = s;

    uint8_t* qr = q + row * ldq;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        if (c * 1024 + lane * 16 >= K) continue;
        uint32_t word[4];
#pragma unroll
        for (int hi = 0; hi < 4; ++hi) {
            // quantization is odd-symmetric (rint and the clamp are), so negating the input of an
            // odd 64-column group negates its codes exactly
            float sg = 1.0f;
            if constexpr (OUT == 3) {
                const int col = c * 1024 + (BLK < 64 ? 16 * lane + 4 * hi : group_col<BLK>(lane, hi));
                sg = (col >> 6) & 1 ? -1.0f : 1.0f;
            }
            uint32_t m0 = __float_as_uint(quant_magic<LIMIT>(sg * v[c][4 * hi + 0], r, s));
            uint32_t m1 = __float_as_uint(quant_magic<LIMIT>(sg * v[c][4 * hi + 1], r, s));
            uint32_t m2 = __float_as_uint(quant_magic<LIMIT>(sg * v[c][4 * hi + 2], r, s));
            uint32_t m3 = __float_as_uint(quant_magic<LIMIT>(sg * v[c][4 * hi + 3], r, s));
            if constexpr (OUT == 3) {
                m0 <<= 4; m1 <<= 4; m2 <<= 4; m3 <<= 4;
            }
            if constexpr (OUT == 2) {
                word[hi] = (m0 & 0xfu) | ((m1 & 0xfu) << 4) | ((m2 & 0xfu) << 8) | ((m3 & 0xfu) << 12);
            } else {
                const uint32_t lo16 = __builtin_amdgcn_perm(m1, m0, 0x0c0c0400u);
                const uint32_t hi16 = __builtin_amdgcn_perm(m3, m2, 0x04000c0cu);
                word[hi] = lo16 | hi16;
            }
        }
        const int cbase = c * 1024;
        if constexpr (BLK < 64) {
            if constexpr (OUT == 2) {
                uint2 out = {word[0] | (word[1] << 16), word[2] | (word[3] << 16)};
                *reinterpret_cast<uint2*>(qr + (cbase + 16 * lane) / 2) = out;
            } else {
                uint4 out = {word[0], word[1], word[2], word[3]};
                *reinterpret_cast<uint4*>(qr + cbase + 16 * lane) = out;
            }
        } else {
#pragma unroll
            for (int hi = 0; hi < 4; ++hi) {
                const int col = cbase + group_col<BLK>(lane, hi);
                if constexpr (OUT == 2) {
                    *reinterpret_cast<uint16_t*>(qr + col / 2) = static_cast<uint16_t>(word[hi]);
                } else {
                    *reinterpret_cast<uint32_t*>(qr + col) = word[hi];
                }
            }
        }
    }
}

template <int BLK, int OUT>
int dispatch_nch(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, void* q, int64_t ldq,
                 float* scale, hipStream_t stream) {
    const int chunks = static_cast<int>((K + 1023) / 1024);
    const dim3 grid(static_cast<unsigned>((M + kWaves - 1) / kWaves));
    const dim3 block(64 * kWaves);
    auto* qp = static_cast<uint8_t*>(q);
    const int m = static_cast<int>(M), k = static_cast<int>(K);
#define MQ_RQ_CASE(N)                                                                            \
    if (chunks <= N) {                                                                           \
        hipLaunchKernelGGL((rotquant_kernel<BLK, OUT, N>), grid, block, 0, stream, x, ldx, m, k, \
                           qp, ldq, scale);                                                      \
        return launch_status("rotquant");                                                        \
    }
    MQ_RQ_CASE(1)
    MQ_RQ_CASE(2)
    MQ_RQ_CASE(3)
    MQ_RQ_CASE(4)
    MQ_RQ_CASE(6)
    MQ_RQ_CASE(8)
    MQ_RQ_CASE(12)
    MQ_RQ_CASE(14)
    MQ_RQ_CASE(16)
#undef MQ_RQ_CASE
    set_error("rotquant: K=%lld exceeds 16384", static_cast<long long>(K));
    return -2;
}

template <int BLK>
int dispatch_out(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int bits, int packed, void* q,
                 int64_t ldq, float* scale, hipStream_t stream) {
    if (bits == 8) return dispatch_nch<BLK, 0>(x, M, K, ldx, q, ldq, scale, stream);
    if (packed == 1) return dispatch_nch<BLK, 2>(x, M, K, ldx, q, ldq, scale, stream);
    if (packed == 2) return dispatch_nch<BLK, 3>(x, M, K, ldx, q, ldq, scale, stream);
    return dispatch_nch<BLK, 1>(x, M, K, ldx, q, ldq, scale, stream);
}

}  // namespace

int launch_rotquant(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int hblock, int bits,
                    int packed, void* q, int64_t ldq, float* scale, hipStream_t stream) {
    switch (hblock) {
        case 0: return dispatch_out<1>(x, M, K, ldx, bits, packed, q, ldq, scale, stream);
        case 16: return dispatch_out<16>(x, M, K, ldx, bits, packed, q, ldq, scale, stream);
        case 64: return dispatch_out<64>(x, M, K, ldx, bits, packed, q, ldq, scale, stream);
        case 256: return dispatch_out<256>(x, M, K, ldx, bits, packed, q, ldq, scale, stream);
        default: break;
    }
    set_error("rotquant: hblock must be 0, 16, 64 or 256 (got %d)", hblock);
    return -1;
}

}  // namespace mq
