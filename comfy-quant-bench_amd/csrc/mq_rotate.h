// Building blocks of the rotate + per-token quantizer that act on one wavefront's 1024-column
// chunk of a row (the lane and register layout described in mq_rotquant_kernel.h): the radix-4
// Hadamard stages, their lane / LDS exchanges, the division-free row scale and the 16-value
// quantizer. Shared by the rotate+quantize kernels and by the GEMV's fused single-row prologue,
// so both produce the same codes and scales from the same instructions.
#pragma once

#include "mq_device.h"

#pragma clang fp contract(off)

namespace mq {
namespace {

constexpr float kTieWindow = 0.5f - 0x1p-15f;

__device__ __forceinline__ float f16lo(uint32_t w) { return f16_bits_to_f32(static_cast<uint16_t>(w & 0xffffu)); }
__device__ __forceinline__ float f16hi(uint32_t w) { return f16_bits_to_f32(static_cast<uint16_t>(w >> 16)); }

// Radix-4 butterflies over register bits J, J+1 (element stride 4^d mapped to register stride 2^J).
// y_i = fma(t, 0.5, -x_{3-i}) with t = ((x0 + x1) + x2) + x3 is the reference's h - x_{3-i},
// h = 0.5f * t: halving is exact, so the fma rounds the same real number once. (For a subnormal t
// the product is exact where 0.5f * t may round; such values quantize to code 0 under any scale
// the quantizer can choose, s >= 1e-10, so codes and scales are unchanged.)
template <int J>
__device__ __forceinline__ void stage_reg(float (&v)[16]) {
    constexpr int st = 1 << J;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        if ((r >> J) & 3) continue;
        const float x0 = v[r], x1 = v[r + st], x2 = v[r + 2 * st], x3 = v[r + 3 * st];
        const float t = ((x0 + x1) + x2) + x3;
        v[r] = __builtin_fmaf(t, 0.5f, -x3);
        v[r + st] = __builtin_fmaf(t, 0.5f, -x2);
        v[r + 2 * st] = __builtin_fmaf(t, 0.5f, -x1);
        v[r + 3 * st] = __builtin_fmaf(t, 0.5f, -x0);
    }
}

// Exchange lane bit B (2..5) with register bit J of an array of N 32-bit values: afterwards the
// value with (lane bit B = u, register bit J = w) is the one that was at (lane bit B = w,
// register bit J = u).
template <int B, int J, int N, typename T>
__device__ __forceinline__ void swap_lane_reg(T (&v)[N], [[maybe_unused]] int lane) {
#pragma unroll
    for (int r = 0; r < N; ++r) {
        if (r & (1 << J)) continue;
        const uint32_t x = __builtin_bit_cast(uint32_t, v[r]), y = __builtin_bit_cast(uint32_t, v[r | (1 << J)]);
        uint32_t xn, yn;
        if constexpr (B == 2 || B == 3) {
            // lanes with the bit set take y from lane - 2^B, the others x from lane + 2^B: row
            // shifts within 16-lane rows, each written only into the lanes (DPP banks of 4 lanes =
            // lane bits 2, 3) that take it, so every moved value costs one v_mov_b32_dpp
            constexpr int shr = B == 2 ? kRowShr4 : kRowShr8, shl = B == 2 ? kRowShl4 : kRowShl8;
            constexpr int up = B == 2 ? 0xA : 0xC;        // banks with the lane bit set
            xn = __builtin_amdgcn_update_dpp(x, y, shr, 0xf, up, false);
            yn = __builtin_amdgcn_update_dpp(y, x, shl, 0xf, up ^ 0xf, false);
        } else if constexpr (B == 4) {
            const auto p = __builtin_amdgcn_permlane16_swap(x, y, false, false);
            xn = p[0];
            yn = p[1];
        } else {
            static_assert(B == 5, "lane bit");
            const auto p = __builtin_amdgcn_permlane32_swap(x, y, false, false);
            xn = p[0];
            yn = p[1];
        }
        v[r] = __builtin_bit_cast(T, xn);
        v[r | (1 << J)] = __builtin_bit_cast(T, yn);
    }
}

template <int BLK>
__device__ __forceinline__ void rotate_chunk(float (&v)[16], int lane) {
    if constexpr (BLK >= 16) {
        stage_reg<0>(v);          // element stride 1  (c0 c1)
        stage_reg<2>(v);          // element stride 4  (c2 c3)
    }
    if constexpr (BLK >= 64) {
        swap_lane_reg<2, 2>(v, lane);
        swap_lane_reg<3, 3>(v, lane);
        stage_reg<2>(v);          // element stride 16 (c4 c5)
    }
    if constexpr (BLK >= 256) {
        swap_lane_reg<4, 2>(v, lane);
        swap_lane_reg<5, 3>(v, lane);
        stage_reg<2>(v);          // element stride 64 (c6 c7)
    }
}

// The same rotation with the exchanges done through LDS instead of lane swaps (no VALU work for
// them). Within each group of 16 lanes that share lane bits L0 L1, lane bits L2..L5 hold c4..c7
// and the 16 registers c0..c3: a 16 x 16 transpose (lane index <-> register index) brings c4..c7
// into the registers, where the stages over (c4 c5) and (c6 c7) run, and the same transpose
// brings the load layout back. Lane (g, i) = (L & 3, L >> 2) writes its register j at float
// g * kTrG + j * kTrS + i and reads its new registers 4q .. 4q + 3 from g * kTrG + i * kTrS + 4q:
// 16 ds_write_b32, whose 64 lanes hit 64 different banks (kTrG = 16 mod 64 banks), and 4
// ds_read_b128, whose 16-lane quarters cover the 64 banks once (kTrS = 20). LDS operations of a
// wave execute in issue order, so a read sees the writes before it and the next transpose's
// writes never overtake earlier reads.
constexpr int kTrS = 20, kTrG = 336, kTrWave = 4 * kTrG;   // floats
struct LdsTranspose {
    float* w;   // this lane's write base: wave region + g * kTrG + i
    float* r;   // this lane's read base: wave region + g * kTrG + i * kTrS
    __device__ __forceinline__ void operator()(float (&v)[16]) const {
#pragma unroll
        for (int j = 0; j < 16; ++j) w[j * kTrS] = v[j];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 t = *reinterpret_cast<const float4*>(r + 4 * q);
            v[4 * q] = t.x;
            v[4 * q + 1] = t.y;
            v[4 * q + 2] = t.z;
            v[4 * q + 3] = t.w;
        }
    }
};

template <int BLK>
__device__ __forceinline__ void rotate_chunk_lds(float (&v)[16], const LdsTranspose& tr) {
    if constexpr (BLK >= 16) {
        stage_reg<0>(v);          // element stride 1  (c0 c1)
        stage_reg<2>(v);          // element stride 4  (c2 c3)
    }
    if constexpr (BLK >= 64) {
        tr(v);                    // registers now hold c4..c7
        stage_reg<0>(v);          // element stride 16 (c4 c5)
        if constexpr (BLK >= 256) stage_reg<2>(v);   // element stride 64 (c6 c7)
        tr(v);                    // back to the load layout
    }
}

// am / L rounded to nearest for every am in [0, +inf] (L = 127 or 7) without a division: with
// c = RN(1/L), q0 = RN(am c) is within an ulp of am / L, the residual am - q0 L is exact (one
// fma), and RN(q0 + residual c) is the correctly rounded quotient (Markstein's correction step).
// Checked bit for bit against the IEEE quotient for every non-negative float on the CPU
// (tests/test_rotquant_scale.py). +inf, whose residual is NaN, is passed through.
template <int L>
__device__ __forceinline__ float div_limit(float am) {
    constexpr float c = 1.0f / static_cast<float>(L);
    const float q0 = am * c;
    const float e = __builtin_fmaf(-q0, static_cast<float>(L), am);
    const float q1 = __builtin_fmaf(e, c, q0);
    return am == __builtin_inff() ? am : q1;
}

// 1/s for a row scale s in [1e-10, +inf]: v_rcp_f32 (within an ulp or so) refined by one Newton
// step, e = 1 - s r0 and r = r0 + e r0, which leaves a relative error within 2^-23 for any start
// within 8 ulps (the square of the first error plus the final rounding; checked on the CPU by
// tests/test_rotquant_scale.py); 1/inf = 0 as the IEEE quotient.
__device__ __forceinline__ float recip_row(float s) {
    const float r0 = __builtin_amdgcn_rcpf(s);
    const float e = __builtin_fmaf(-s, r0, 1.0f);
    const float r = __builtin_fmaf(e, r0, r0);
    return s == __builtin_inff() ? 0.0f : r;
}

// Column bit 6 (the parity of the 64-column group) of register r of lane L after rotate_chunk.
template <int BLK>
__device__ __forceinline__ int col_bit6(int lane, int r) {
    if constexpr (BLK >= 256) return (r >> 2) & 1;   // r2 r3 hold c6 c7
    else return (lane >> 4) & 1;                      // L4 holds c6
}

// Quantize 16 values: fast path for all, then (rarely, per lane) the exact path for the values
// whose product lies near a half-integer. Returns the magic-biased floats (code in the low bits).
template <int LIMIT>
__device__ __forceinline__ void quant16(const float (&v)[16], float sg, float r, float s, float (&m)[16]) {
    float dmax = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const float x = sg * v[j];
        m[j] = __builtin_fmaf(x, r, kMagic);
        const float n = m[j] - kMagic;
        dmax = __builtin_fmaxf(dmax, __builtin_fabsf(__builtin_fmaf(x, r, -n)));
    }
    if (dmax > kTieWindow) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const float x = sg * v[j];
            const float n = m[j] - kMagic;
            if (__builtin_fabsf(__builtin_fmaf(x, r, -n)) > kTieWindow) {
                float qf = __builtin_rintf(x / s);
                qf = __builtin_fminf(__builtin_fmaxf(qf, -static_cast<float>(LIMIT)), static_cast<float>(LIMIT));
                m[j] = kMagic + qf;
            }
        }
    }
}

// quant16's arithmetic on four consecutive values, packed into one dword of codes (value j in
// byte j; X16: as 16 * q). A value takes the exact path exactly when its own product lies near a
// half-integer, as in quant16, so the codes are the same; with four values live at a time instead
// of sixteen, it fits callers that hold other operands in flight.
template <int LIMIT, bool X16>
__device__ __forceinline__ uint32_t quant4_word(const float* v, float sg, float r, float s) {
    uint32_t m[4];
    bool near = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float x = sg * v[j];
        const float mf = __builtin_fmaf(x, r, kMagic);
        near |= __builtin_fabsf(__builtin_fmaf(x, r, -(mf - kMagic))) > kTieWindow;
        m[j] = __float_as_uint(mf);
    }
    if (near) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float x = sg * v[j];
            const float n = __uint_as_float(m[j]) - kMagic;
            if (__builtin_fabsf(__builtin_fmaf(x, r, -n)) > kTieWindow) {
                float qf = __builtin_rintf(x / s);
                qf = __builtin_fminf(__builtin_fmaxf(qf, -static_cast<float>(LIMIT)), static_cast<float>(LIMIT));
                m[j] = __float_as_uint(kMagic + qf);
            }
        }
    }
    if constexpr (X16) {
#pragma unroll
        for (int j = 0; j < 4; ++j) m[j] <<= 4;
    }
    return __builtin_amdgcn_perm(m[1], m[0], 0x0c0c0400u) | __builtin_amdgcn_perm(m[3], m[2], 0x04000c0cu);
}

}  // namespace
}  // namespace mq
