// Device helpers for gfx950 (CDNA4): bf16 bit conversions, DPP lane exchanges, magic rounding.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mq {

// 1.5 * 2^23: fma(v, r, kMagic) rounds v*r to the nearest integer n (ties to even) and leaves
// n in the low mantissa bits, for |v*r| < 2^22. bits(kMagic + n) = 0x4B400000 + n.
constexpr float kMagic = 12582912.0f;

__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// float -> bf16 bits, round to nearest even (finite values).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// Floating-point operand types chosen by the caller (MQ_DT_* of include/mq.h).
constexpr int kDtBf16 = 0, kDtF16 = 1, kDtF32 = 2;

// Element i of a vector of type dt, as fp32 (exact for every type).
__device__ __forceinline__ float load_as_f32(const void* p, int dt, int64_t i) {
    if (dt == kDtF32) return static_cast<const float*>(p)[i];
    const uint16_t h = static_cast<const uint16_t*>(p)[i];
    return dt == kDtF16 ? f16_bits_to_f32(h) : __uint_as_float(static_cast<uint32_t>(h) << 16);
}

typedef float mq_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 mq_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 mq_f16x2 __attribute__((ext_vector_type(2)));

// Two fp32 values rounded (to nearest, ties to even) to the 16-bit type dt (bf16 or fp16) and
// packed: v0 in bits 0-15, v1 in bits 16-31.
__device__ __forceinline__ uint32_t pack_16x2(float v0, float v1, int dt) {
    const mq_f32x2 v = {v0, v1};
    if (dt == kDtF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, mq_f16x2));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, mq_bf16x2));
}

// Store v rounded to type dt at element i of p.
__device__ __forceinline__ void store_from_f32(void* p, int dt, int64_t i, float v) {
    if (dt == kDtF32) {
        static_cast<float*>(p)[i] = v;
        return;
    }
    static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(pack_16x2(v, 0.0f, dt) & 0xffffu);
}

// v_mov_b32 with a DPP source: every lane reads `src` from the lane the control selects.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float src) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(src), CTRL, 0xf, 0xf, true));
}

// DPP move restricted to the banks in BANK_MASK (4-lane groups of each 16-lane row); lanes in
// other banks keep `old`.
template <int CTRL, int BANK_MASK>
__device__ __forceinline__ float dpp_upd(float old, float src) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(src), CTRL, 0xf, BANK_MASK, false));
}

// DPP controls (GFX9 encoding).
constexpr int kQuadXor1 = 0xB1;       // quad_perm [1, 0, 3, 2]: lane ^ 1
constexpr int kQuadXor2 = 0x4E;       // quad_perm [2, 3, 0, 1]: lane ^ 2
constexpr int kRowRor4 = 0x124;       // rotate right by 4 within a row of 16
constexpr int kRowRor8 = 0x128;
constexpr int kQuadPerm0022 = 0xA0;   // lane <- lane & ~1 within the quad
constexpr int kQuadPerm1133 = 0xF5;   // lane <- lane | 1
constexpr int kQuadPerm0101 = 0x44;   // lane <- lane & ~2
constexpr int kQuadPerm2323 = 0xEE;   // lane <- lane | 2
constexpr int kRowShl4 = 0x104;       // lane <- lane + 4 (within a row of 16)
constexpr int kRowShl8 = 0x108;
constexpr int kRowShr4 = 0x114;       // lane <- lane - 4
constexpr int kRowShr8 = 0x118;

// Maximum over the 64 lanes of a wavefront, returned in every lane: four DPP steps give each
// 16-lane row its maximum, then the four row maxima are read as scalars (no LDS round trip).
__device__ __forceinline__ float wave_max(float v) {
    v = __builtin_fmaxf(v, dpp_mov<kQuadXor1>(v));
    v = __builtin_fmaxf(v, dpp_mov<kQuadXor2>(v));
    v = __builtin_fmaxf(v, dpp_mov<kRowRor4>(v));
    v = __builtin_fmaxf(v, dpp_mov<kRowRor8>(v));
    const int b = __float_as_int(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(b, 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(b, 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(b, 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(b, 48));
    return __builtin_fmaxf(__builtin_fmaxf(r0, r1), __builtin_fmaxf(r2, r3));
}

// wave_max for values that are >= 0 and not NaN (+inf allowed): their bit patterns order as
// unsigned integers, so every step is an integer maximum, which takes its DPP operand directly
// (one instruction per step) and needs none of the float maximum's NaN handling; the four row
// maxima are combined on the scalar unit.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov_u(uint32_t src) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(src), CTRL, 0xf, 0xf, true));
}
__device__ __forceinline__ float wave_max_nonneg(float v) {
    uint32_t b = __float_as_uint(v);
    b = __builtin_elementwise_max(b, dpp_mov_u<kQuadXor1>(b));
    b = __builtin_elementwise_max(b, dpp_mov_u<kQuadXor2>(b));
    b = __builtin_elementwise_max(b, dpp_mov_u<kRowRor4>(b));
    b = __builtin_elementwise_max(b, dpp_mov_u<kRowRor8>(b));
    const uint32_t r0 = __builtin_amdgcn_readlane(b, 0), r1 = __builtin_amdgcn_readlane(b, 16);
    const uint32_t r2 = __builtin_amdgcn_readlane(b, 32), r3 = __builtin_amdgcn_readlane(b, 48);
    return __uint_as_float(__builtin_elementwise_max(__builtin_elementwise_max(r0, r1),
                                                     __builtin_elementwise_max(r2, r3)));
}

}  // namespace mq
