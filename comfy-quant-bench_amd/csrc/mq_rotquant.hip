// Fused Hadamard block rotation + per-token dynamic int8 / int4 quantizer for gfx950.
//
// Arithmetic (bit-exact with the CPU oracle):
//   rotation: the fp32 radix-4 FWHT of experiments/qwen21-kernel/kernels/g64_quant.cu:68-86,
//     stages with element strides 1, 4, 16, 64; each butterfly h = 0.5f*(((x0+x1)+x2)+x3),
//     y_i = h - x_{3-i};
//   quantizer: tools/activation_balance.py:65-71, s = max(absmax/L, 1e-10f),
//     q = clamp(rne(x / s), -L, L) with the IEEE quotient x / s.
//
// Layout. One wavefront per row; a row is processed in chunks of 1024 columns. Within a chunk,
// column c has bits c0..c9; lane L of the wave loads the 16 consecutive columns of segment
// s = (L >> 2) + 16 (L & 3) (two 16-byte bf16 loads), so register bits r0..r3 hold c0..c3 and
// lane bits L0..L5 hold c8 c9 c4 c5 c6 c7. The radix-4 stages over (c0 c1) and (c2 c3) run in
// registers. The stage over (c4 c5) (blocks 64, 256) first swaps lane bits L2, L3 with register
// bits r2, r3 through DPP row shifts; the stage over (c6 c7) (block 256) swaps L4, L5 with r2, r3
// through v_permlane16_swap / v_permlane32_swap (one instruction per register pair). Every
// butterfly then runs in registers in the reference's order. After quantization four codes of
// consecutive columns (r0 r1) sit in each dword; a final exchange of dwords across lane bits L2,
// L3 gives every lane 16 consecutive codes, written with one 16-byte (int8) or 8-byte (packed
// int4) store.
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

// Exchange lane bit B (2..5) with register bit J of an array of N 32-bit values: afterwards the
// value with (lane bit B = u, register bit J = w) is the one that was at (lane bit B = w,
// register bit J = u).
template <int B, int J, int N, typename T>
__device__ __forceinline__ void swap_lane_reg(T (&v)[N], int lane) {
#pragma unroll
    for (int r = 0; r < N; ++r) {
        if (r & (1 << J)) continue;
        const uint32_t x = __builtin_bit_cast(uint32_t, v[r]), y = __builtin_bit_cast(uint32_t, v[r | (1 << J)]);
        uint32_t xn, yn;
        if constexpr (B == 2 || B == 3) {
            // lanes with the bit set take y from lane - 2^B, the others x from lane + 2^B (row
            // shifts within 16-lane rows; the select folds into a DPP-sourced v_cndmask)
            constexpr int shr = B == 2 ? kRowShr4 : kRowShr8, shl = B == 2 ? kRowShl4 : kRowShl8;
            const bool up = (lane >> B) & 1;
            const uint32_t ty = __builtin_amdgcn_mov_dpp(y, shr, 0xf, 0xf, true);
            const uint32_t tx = __builtin_amdgcn_mov_dpp(x, shl, 0xf, 0xf, true);
            xn = up ? ty : x;
            yn = up ? y : tx;
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
    const int seg_ld = (lane >> 2) + 16 * (lane & 3);   // 16-column segment this lane loads

    float v[NCH][16];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int e = c * 1024 + seg_ld * 16;
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

    // After the final dword exchange a lane holds the 16 codes of segment seg_st.
    const int seg_st = BLK >= 256 ? (lane >> 4) + 4 * ((lane >> 2) & 3) + 16 * (lane & 3) : seg_ld;
    uint8_t* qr = q + row * ldq;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        // quantization is odd-symmetric (rint and the clamp are), so negating the input of an odd
        // 64-column group negates its codes exactly; for block 256 the group parity is register
        // bit r2, so the sign applies per dword below instead
        float mq[16];
        quant16<LIMIT>(v[c], OUT == 3 && BLK < 256 && col_bit6<BLK>(lane, 0) ? -1.0f : 1.0f, r, s, mq);
        uint32_t word[4];
#pragma unroll
        for (int hi = 0; hi < 4; ++hi) {
            uint32_t m0 = __float_as_uint(mq[4 * hi + 0]), m1 = __float_as_uint(mq[4 * hi + 1]);
            uint32_t m2 = __float_as_uint(mq[4 * hi + 2]), m3 = __float_as_uint(mq[4 * hi + 3]);
            if constexpr (OUT == 3 && BLK >= 256) {
                if (col_bit6<BLK>(lane, 4 * hi)) {   // negate the four codes (two's complement bytes)
                    m0 = -m0; m1 = -m1; m2 = -m2; m3 = -m3;
                }
            }
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
        // dword index bits hold (c6 c7) for block 256 and (c4 c5) for block 64; lane bits L2 L3
        // hold (c2 c3): exchange them so each lane's four dwords are consecutive columns
        if constexpr (BLK >= 64) {
            swap_lane_reg<2, 0>(word, lane);
            swap_lane_reg<3, 1>(word, lane);
        }
        const int col = c * 1024 + seg_st * 16;
        if (col >= K) continue;
        if constexpr (OUT == 2) {
            const uint2 out = {word[0] | (word[1] << 16), word[2] | (word[3] << 16)};
            *reinterpret_cast<uint2*>(qr + col / 2) = out;
        } else {
            const uint4 out = {word[0], word[1], word[2], word[3]};
            *reinterpret_cast<uint4*>(qr + col) = out;
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
