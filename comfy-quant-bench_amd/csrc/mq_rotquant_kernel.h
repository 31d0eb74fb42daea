// Fused Hadamard block rotation + per-token dynamic int8 / int4 quantizer for gfx950 (kernel
// templates, instantiated by mq_rotquant.hip for plain inputs and by mq_swiglu.hip for the
// SwiGLU prologue).
//
// Arithmetic (bit-exact with the CPU oracle):
//   rotation: the fp32 radix-4 FWHT of experiments/qwen21-kernel/kernels/g64_quant.cu:68-86,
//     stages with element strides 1, 4, 16, 64; each butterfly h = 0.5f*(((x0+x1)+x2)+x3),
//     y_i = h - x_{3-i};
//   quantizer: tools/activation_balance.py:65-71, s = max(absmax/L, 1e-10f),
//     q = clamp(rne(x / s), -L, L) with the IEEE quotient x / s.
//
// Layout. A row is processed in chunks of 1024 columns by W wavefronts (W = 1, 2 or 4 by K, so
// that each wave holds at most 4 chunks in registers and the kernel keeps several waves per SIMD);
// wave w of a row takes chunks w, w + W, ... and the row's absmax is combined through LDS. A
// workgroup of 4 waves handles 4 / W rows per step of a grid-stride loop over row groups. Within a chunk,
// column c has bits c0..c9; lane L of the wave loads the 16 consecutive columns of segment
// s = (L >> 2) + 16 (L & 3) (two 16-byte bf16 loads), so register bits r0..r3 hold c0..c3 and
// lane bits L0..L5 hold c8 c9 c4 c5 c6 c7. The radix-4 stages over (c0 c1) and (c2 c3) run in
// registers. Plain inputs then move c4..c7 into the registers with a 16 x 16 transpose through LDS
// (rotate_chunk_lds), run the stages over (c4 c5) and (c6 c7) there and transpose back, so the
// exchanges cost no VALU instructions and the codes leave in the load layout. The SwiGLU kernels
// exchange through lanes instead: the stage over (c4 c5) (blocks 64, 256) first swaps lane bits L2, L3 with register
// bits r2, r3 through DPP row shifts written into the lanes of the receiving DPP banks only (one
// v_mov_b32_dpp per moved value); the stage over (c6 c7) (block 256) swaps L4, L5 with r2, r3
// through v_permlane16_swap / v_permlane32_swap (one instruction per register pair). Every
// butterfly then runs in registers in the reference's order. After quantization four codes of
// consecutive columns (r0 r1) sit in each dword; a final exchange of dwords across lane bits L2,
// L3 gives every lane 16 consecutive codes, written with one 16-byte (int8) or 8-byte (packed
// int4) store.
//
// Quantization without a per-element division: with r within 2^-23 relative of 1/s,
// m = fma(v, r, 1.5*2^23) rounds v*r to an integer n. |v*r - v/s| < 2^-16 and
// |fl(v/s) - v/s| <= 2^-18 for |v/s| < 128, so rint(fl(v/s)) == n unless v*r lies within
// 2^-16 + 2^-18 of a half-integer; those elements (flagged by |fma(v, r, -n)| > 0.5 - 2^-15, the
// fma adding at most 2^-25) recompute rint(v / s) with the IEEE division. The clamp to [-L, L]
// never binds on the fast path: |v| <= absmax, so |v*r| <= L (1 + 2^-21).
//
// Per row, s = max(absmax / L, 1e-10) is the correctly rounded quotient, formed without a division
// (div_limit), and r comes from v_rcp_f32 and one Newton step (recip_row).
#pragma once

#include <algorithm>
#include <atomic>

#include "mq_device.h"
#include "mq_rotate.h"
#include "mq_silu_table.h"
#include "mq_internal.h"

#pragma clang fp contract(off)

namespace mq {
namespace {

constexpr int kWaves = 4;                 // wavefronts per workgroup

// --- SwiGLU prologue (tools/ck_swiglu/swiglu_quant.cu:56-66): a = silu(g) * u in fp32, rounded
// once to the input type, formed from the gate | up halves while loading. silu(g) = g / (1 +
// exp(-g)) is taken correctly rounded to fp32, from tables generated with exact decimal arithmetic
// (mq_silu_table.h). bf16 gates: every result that is not a closed form comes from a 32 KB table
// that each workgroup stages in LDS; closed forms: |g| < 2^-25 gives g / 2, g >= 128 gives g and
// g <= -128 gives -0. fp16 gates: a 256 KB table over all 65536 bit patterns, read from global
// memory (cached), provided by the translation unit that instantiates the fp16 SwiGLU kernels
// through SiluF16Table. Then a = T(fp32(silu(g) * u)) with T the input type.
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Large outputs store their codes non-temporally (`global_store ... nt`). On MI355X the kernel's
// traffic pattern (two 16-byte loads per lane per 1024-column chunk, one code store per chunk)
// streams at 78 % of 8 TB/s with ordinary stores and 89 % with non-temporal ones, measured on a
// shift-only copy of the pattern at M = 32760, K = 3072 (non-temporal loads lower it to 70 %, so
// the loads stay ordinary). Small outputs keep ordinary stores: the GEMM that follows reads its
// codes sooner from the caches (M = 256, K = 3072: a 21 us W8A8 linear takes 23 us with
// non-temporal code stores). kNtCodeBytes is the output size from which the stores are
// non-temporal.
constexpr int64_t kNtCodeBytes = int64_t{64} << 20;

__device__ __forceinline__ void store_codes(bool nt, uint8_t* p, uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
    if (nt) __builtin_nontemporal_store(u32x4{w0, w1, w2, w3}, reinterpret_cast<u32x4*>(p));
    else *reinterpret_cast<uint4*>(p) = uint4{w0, w1, w2, w3};
}
__device__ __forceinline__ void store_codes(bool nt, uint8_t* p, uint32_t w0, uint32_t w1) {
    if (nt) __builtin_nontemporal_store(u32x2{w0, w1}, reinterpret_cast<u32x2*>(p));
    else *reinterpret_cast<uint2*>(p) = uint2{w0, w1};
}

// fp32 bits of silu(g) for every fp16 bit pattern g; specialized where the table is compiled in.
template <int IN>
struct SiluF16Table;

__device__ __forceinline__ float silu_f32(uint32_t b, float g, const float* tab) {
    const uint32_t t = b & 0x7fffu;
    const uint32_t j = __builtin_elementwise_min(t - kSiluLo, kSiluEntries - 1u);   // in bounds always
    const uint32_t s = __float_as_uint(tab[j + ((b >> 15) << 12)]);
    const uint32_t big = (b >> 15) ? 0x80000000u : __float_as_uint(g);
    const uint32_t r = t < kSiluLo ? __float_as_uint(g * 0.5f) : s;
    return __uint_as_float(t >= kSiluLo + kSiluEntries ? big : r);
}

// Two activations from one dword of gates and one of ups (two bf16 each), as bf16-valued floats.
// EAGER = false: bf16(silu(g) * u), one rounding (the fused quantizer). EAGER = true: silu(g) is
// rounded to bf16 first and the product (exact in fp32: two 8-bit significands) then rounded again,
// bf16(bf16(silu(g)) * u): the eager torch path silu(gate).mul_(up) in bf16.
template <bool EAGER>
__device__ __forceinline__ void swiglu_pair(uint32_t wg, uint32_t wu, const float* tab, float& a0, float& a1) {
    float s0 = silu_f32(wg & 0xffffu, bf16lo(wg), tab), s1 = silu_f32(wg >> 16, bf16hi(wg), tab);
    if constexpr (EAGER) {
        const uint32_t sh = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{s0, s1}, bf16x2));
        s0 = __uint_as_float(sh << 16);
        s1 = __uint_as_float(sh & 0xffff0000u);
    }
    const float p0 = s0 * bf16lo(wu);
    const float p1 = s1 * bf16hi(wu);
    const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{p0, p1}, bf16x2));
    a0 = __uint_as_float(h << 16);
    a1 = __uint_as_float(h & 0xffff0000u);
}

// fp16 inputs: silu of both gates from the global fp16 table, the products rounded to fp16 (EAGER:
// silu(g) rounded to fp16 first; the product of two 11-bit significands is exact in fp32).
template <bool EAGER>
__device__ __forceinline__ void swiglu_pair_f16(uint32_t wg, uint32_t wu, const uint32_t* tab, float& a0, float& a1) {
    float s0 = __uint_as_float(tab[wg & 0xffffu]), s1 = __uint_as_float(tab[wg >> 16]);
    if constexpr (EAGER) {
        const uint32_t sh = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{s0, s1}, f16x2));
        s0 = f16lo(sh);
        s1 = f16hi(sh);
    }
    const float p0 = s0 * f16lo(wu);
    const float p1 = s1 * f16hi(wu);
    const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{p0, p1}, f16x2));
    a0 = f16lo(h);
    a1 = f16hi(h);
}

// OUT: 0 = int8 codes, 1 = int4 codes one per byte, 2 = int4 codes packed two per byte,
//      3 = int4 codes one per byte as 16 * q, negated in odd 64-column groups (the operand layout
//          the group-scale GEMM takes for int4 activations: exact, and 16x finer in its fp32 step).
// ACT: 0 = x is the activation itself; 1 = x holds gate | up halves of K columns each (the up
// half starts K elements into the row) and the activation is swiglu_pair(gate, up) rounded once;
// 2 = the same with the eager path's two roundings (swiglu_pair<true>).
// IN: 0 = bf16 input, 1 = fp16 input (either converts exactly to fp32), 2 = fp32 input.
// NCH: chunks per wave; W: waves per row (NCH * W * 1024 >= K).
// TL: codes in 16-row tiles (one code per byte only), chosen at compile time so that the
// row-major store keeps its exact code
template <int BLK, int OUT, int NCH, int ACT, int W, int IN, bool TL>
__global__ void __launch_bounds__(64 * kWaves)
rotquant_kernel(const uint16_t* __restrict__ x, int64_t ldx, int M, int K,
                uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ scale, bool nt) {
    constexpr int LIMIT = OUT == 0 ? 127 : 7;
    constexpr int RPG = kWaves / W;                      // rows per workgroup step
    // Plain inputs exchange lanes and registers through LDS (rotate_chunk_lds) and leave the
    // rotation in the load layout; the SwiGLU prologue, whose LDS holds its silu table, keeps the
    // lane swaps. LB: the block whose register layout the rotated values are in.
    constexpr bool kLdsT = ACT == 0 && BLK >= 64;
    constexpr int LB = kLdsT ? 16 : BLK;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wr = wave % W;                             // this wave's share of its row
    [[maybe_unused]] LdsTranspose tr{nullptr, nullptr};
    if constexpr (kLdsT) {
        __shared__ __attribute__((aligned(16))) float tr_lds[kWaves * kTrWave];
        float* base = tr_lds + wave * kTrWave + (lane & 3) * kTrG;
        tr.w = base + (lane >> 2);
        tr.r = base + (lane >> 2) * kTrS;
    }
    [[maybe_unused]] const float* tab = nullptr;
    [[maybe_unused]] const uint32_t* tab16 = nullptr;
    if constexpr (ACT >= 1 && IN == 1) tab16 = SiluF16Table<IN>::get();
    if constexpr (ACT >= 1 && IN == 0) {
        __shared__ __attribute__((aligned(16))) uint32_t silu_lds[2 * kSiluEntries];
        for (uint32_t i = threadIdx.x; i < 2 * kSiluEntries / 4; i += 64 * kWaves)
            reinterpret_cast<uint4*>(silu_lds)[i] = reinterpret_cast<const uint4*>(kSiluTable)[i];
        __syncthreads();
        tab = reinterpret_cast<const float*>(silu_lds);
    }
    [[maybe_unused]] float* red = nullptr;               // per-wave absmax, double-buffered by step
    if constexpr (W > 1) {
        __shared__ float red_lds[2][kWaves];
        red = &red_lds[0][0];
    }
    const int seg_ld = (lane >> 2) + 16 * (lane & 3);   // 16-column segment this lane loads
    // after the final dword exchange a lane holds the 16 codes of segment seg_st
    const int seg_st = LB >= 256 ? (lane >> 4) + 4 * ((lane >> 2) & 3) + 16 * (lane & 3) : seg_ld;
    const int64_t groups = (static_cast<int64_t>(M) + RPG - 1) / RPG;
    int parity = 0;
    // every wave runs the same number of steps (the bound is uniform over the workgroup), so the
    // barrier inside is reached by all of them
    for (int64_t rg = blockIdx.x; rg < groups; rg += gridDim.x, parity ^= 1) {
        const int64_t row = rg * RPG + wave / W;
        const bool live = row < M;
        if constexpr (W == 1) {
            if (!live) break;
        }
        // Lanes past the end of the row (a last chunk that K does not fill) and the waves of a
        // row past M (W > 1: they still take part in the barrier) load in-bounds data from the
        // row's start or from row M - 1 instead, and their values are left out of the absmax; their
        // codes are not stored. A Hadamard block lies wholly inside or outside the row (K is a
        // multiple of the block), so the rotation never mixes such values into stored ones.
        // (fp32 inputs: x and ldx count 16-bit units of the row buffer, two per element)
        constexpr int kU = IN == 2 ? 2 : 1;
        const uint16_t* xr = x + (live ? row : static_cast<int64_t>(M) - 1) * ldx * kU;

        float v[NCH][16];
        bool in[NCH];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int e0 = (c * W + wr) * 1024 + seg_ld * 16;
            in[c] = e0 < K;
            const int e = in[c] ? e0 : 0;
            if constexpr (IN == 2) {
                static_assert(ACT == 0, "the SwiGLU prologue takes bf16 or fp16 inputs");
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float4 f = *reinterpret_cast<const float4*>(xr + 2 * e + 8 * j);
                    v[c][4 * j] = f.x;
                    v[c][4 * j + 1] = f.y;
                    v[c][4 * j + 2] = f.z;
                    v[c][4 * j + 3] = f.w;
                }
                continue;
            }
            const uint4 a = *reinterpret_cast<const uint4*>(xr + e);
            const uint4 b = *reinterpret_cast<const uint4*>(xr + e + 8);
            const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            if constexpr (ACT >= 1) {
                const uint4 ua = *reinterpret_cast<const uint4*>(xr + K + e);
                const uint4 ub = *reinterpret_cast<const uint4*>(xr + K + e + 8);
                const uint32_t wu[8] = {ua.x, ua.y, ua.z, ua.w, ub.x, ub.y, ub.z, ub.w};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if constexpr (IN == 1) swiglu_pair_f16<ACT == 2>(w[j], wu[j], tab16, v[c][2 * j], v[c][2 * j + 1]);
                    else swiglu_pair<ACT == 2>(w[j], wu[j], tab, v[c][2 * j], v[c][2 * j + 1]);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    v[c][2 * j] = IN == 1 ? f16lo(w[j]) : bf16lo(w[j]);
                    v[c][2 * j + 1] = IN == 1 ? f16hi(w[j]) : bf16hi(w[j]);
                }
            }
        }

        float am = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            if constexpr (kLdsT) rotate_chunk_lds<BLK>(v[c], tr);
            else rotate_chunk<BLK>(v[c], lane);
            float amc = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) amc = __builtin_fmaxf(amc, __builtin_fabsf(v[c][j]));
            am = __builtin_fmaxf(am, live && in[c] ? amc : 0.0f);
        }
        am = wave_max_nonneg(am);
        if constexpr (W > 1) {
            if (lane == 0) red[parity * kWaves + wave] = am;
            __syncthreads();
            const int first = wave - wr;
#pragma unroll
            for (int i = 0; i < W; ++i) am = __builtin_fmaxf(am, red[parity * kWaves + first + i]);
            if (!live) continue;
        }

        const float s = __builtin_fmaxf(div_limit<LIMIT>(am), 1e-10f);
        const float r = recip_row(s);
        if (lane == 0 && wr == 0) scale[row] = s;

        // TL: codes in 16-row tiles [M / 16][K / 64][16][64], the operand layout of the wide
        // GEMM's whole-line activation loads
        constexpr bool tiled = TL && OUT != 2;
        uint8_t* qr = tiled ? q + (row >> 4) * (static_cast<int64_t>(K) << 4) + (row & 15) * 64 : q + row * ldq;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            // quantization is odd-symmetric (rint and the clamp are), so negating the input of an
            // odd 64-column group negates its codes exactly; in the block-256 lane-swap layout the
            // group parity is register bit r2, so the sign applies per dword below instead
            float mq[16];
            quant16<LIMIT>(v[c], OUT == 3 && LB < 256 && col_bit6<LB>(lane, 0) ? -1.0f : 1.0f, r, s, mq);
            uint32_t word[4];
#pragma unroll
            for (int hi = 0; hi < 4; ++hi) {
                uint32_t m0 = __float_as_uint(mq[4 * hi + 0]), m1 = __float_as_uint(mq[4 * hi + 1]);
                uint32_t m2 = __float_as_uint(mq[4 * hi + 2]), m3 = __float_as_uint(mq[4 * hi + 3]);
                if constexpr (OUT == 3 && LB >= 256) {
                    if (col_bit6<LB>(lane, 4 * hi)) {   // negate the four codes (two's complement bytes)
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
            // dword index bits hold (c6 c7) for block 256 and (c4 c5) for block 64; lane bits
            // L2 L3 hold (c2 c3): exchange them so each lane's four dwords are consecutive columns
            if constexpr (LB >= 64) {
                swap_lane_reg<2, 0>(word, lane);
                swap_lane_reg<3, 1>(word, lane);
            }
            const int col = (c * W + wr) * 1024 + seg_st * 16;
            if (col >= K) continue;
            if constexpr (OUT == 2)
                store_codes(nt, qr + col / 2, word[0] | (word[1] << 16), word[2] | (word[3] << 16));
            else
                store_codes(nt, qr + (tiled ? (col >> 6) * 1024 + (col & 63) : col), word[0], word[1], word[2], word[3]);
        }
    }
}

template <int BLK, int OUT, int NCH, int ACT, int W, int IN>
int launch_rq(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, void* q, int64_t ldq, float* scale,
              hipStream_t stream) {
    const int64_t groups = (M + kWaves / W - 1) / (kWaves / W);
    // plain inputs: one workgroup per row group; SwiGLU: a grid-stride loop over the row groups,
    // so each workgroup stages the LDS table once for many rows
    int64_t wgs = groups;
    if constexpr (ACT >= 1 && IN == 0) {
        // as many workgroups as are resident at once (the same number on every CU), each
        // striding over the row groups
        // resident workgroups per CU of this instantiation: queried once (every device this
        // library runs on is a gfx950 with the same per-CU resources)
        static std::atomic<int> per_cu_cache{0};
        int per_cu = per_cu_cache.load(std::memory_order_relaxed);
        if (per_cu <= 0) {
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                    &per_cu, reinterpret_cast<const void*>(&rotquant_kernel<BLK, OUT, NCH, ACT, W, IN, false>),
                    64 * kWaves,
                    0) != hipSuccess ||
                per_cu <= 0)
                per_cu = 1;
            else
                per_cu_cache.store(per_cu, std::memory_order_relaxed);
        }
        const int cus = device_cu_count();
        wgs = std::min<int64_t>(groups, static_cast<int64_t>(cus > 0 ? cus : 256) * per_cu);
    }
    if (wgs == 0) return 0;
    const bool nt = (OUT == 2 ? M * K / 2 : M * K) >= kNtCodeBytes;
    // a row stride of 0 asks for the codes in 16-row tiles (one code per byte)
    if (OUT != 2 && ldq == 0)
        hipLaunchKernelGGL((rotquant_kernel<BLK, OUT, NCH, ACT, W, IN, OUT != 2>), dim3(static_cast<unsigned>(wgs)),
                           dim3(64 * kWaves), 0, stream, x, ldx, static_cast<int>(M), static_cast<int>(K),
                           static_cast<uint8_t*>(q), ldq, scale, nt);
    else
        hipLaunchKernelGGL((rotquant_kernel<BLK, OUT, NCH, ACT, W, IN, false>), dim3(static_cast<unsigned>(wgs)),
                           dim3(64 * kWaves), 0, stream, x, ldx, static_cast<int>(M), static_cast<int>(K),
                           static_cast<uint8_t*>(q), ldq, scale, nt);
    return launch_status("rotquant");
}

template <int BLK, int OUT, int ACT, int IN>
int dispatch_nch(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, void* q, int64_t ldq,
                 float* scale, hipStream_t stream) {
    const int chunks = static_cast<int>((K + 1023) / 1024);
    // few rows (config 0, the text-token and single-token calls): four waves per row, so the launch
    // has four times the waves and each wave a quarter of the row's latency-bound chain (M = 1024,
    // K = 3072 inside the W4A8 linear: 27.2-27.4 -> 26.8-27.1 us per call; M = 4096 is 0.6 us
    // slower this way)
    if (M <= 1024 && chunks <= 8) {
        if (chunks <= 4) return launch_rq<BLK, OUT, 1, ACT, 4, IN>(x, M, K, ldx, q, ldq, scale, stream);
        return launch_rq<BLK, OUT, 2, ACT, 4, IN>(x, M, K, ldx, q, ldq, scale, stream);
    }
    switch (chunks) {
        case 1: return launch_rq<BLK, OUT, 1, ACT, 1, IN>(x, M, K, ldx, q, ldq, scale, stream);
        case 2: return launch_rq<BLK, OUT, 2, ACT, 1, IN>(x, M, K, ldx, q, ldq, scale, stream);
        case 3: return launch_rq<BLK, OUT, 3, ACT, 1, IN>(x, M, K, ldx, q, ldq, scale, stream);
        case 4: return launch_rq<BLK, OUT, 4, ACT, 1, IN>(x, M, K, ldx, q, ldq, scale, stream);
        case 5: case 6: return launch_rq<BLK, OUT, 3, ACT, 2, IN>(x, M, K, ldx, q, ldq, scale, stream);
        case 7: case 8: return launch_rq<BLK, OUT, 4, ACT, 2, IN>(x, M, K, ldx, q, ldq, scale, stream);
        case 9: case 10: case 11: case 12: return launch_rq<BLK, OUT, 3, ACT, 4, IN>(x, M, K, ldx, q, ldq, scale, stream);
        case 13: case 14: case 15: case 16: return launch_rq<BLK, OUT, 4, ACT, 4, IN>(x, M, K, ldx, q, ldq, scale, stream);
        default: break;
    }
    set_error("rotquant: K=%lld exceeds 16384", static_cast<long long>(K));
    return -2;
}

template <int BLK, int ACT, int IN>
int dispatch_out(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int bits, int packed, void* q,
                 int64_t ldq, float* scale, hipStream_t stream) {
    if (bits == 8) return dispatch_nch<BLK, 0, ACT, IN>(x, M, K, ldx, q, ldq, scale, stream);
    if (packed == 1) return dispatch_nch<BLK, 2, ACT, IN>(x, M, K, ldx, q, ldq, scale, stream);
    if (packed == 2) return dispatch_nch<BLK, 3, ACT, IN>(x, M, K, ldx, q, ldq, scale, stream);
    return dispatch_nch<BLK, 1, ACT, IN>(x, M, K, ldx, q, ldq, scale, stream);
}

template <int ACT, int IN>
int launch_rotquant_impl(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int hblock, int bits,
                         int packed, void* q, int64_t ldq, float* scale, hipStream_t stream) {
    switch (hblock) {
        case 0: return dispatch_out<1, ACT, IN>(x, M, K, ldx, bits, packed, q, ldq, scale, stream);
        case 16: return dispatch_out<16, ACT, IN>(x, M, K, ldx, bits, packed, q, ldq, scale, stream);
        case 64: return dispatch_out<64, ACT, IN>(x, M, K, ldx, bits, packed, q, ldq, scale, stream);
        case 256: return dispatch_out<256, ACT, IN>(x, M, K, ldx, bits, packed, q, ldq, scale, stream);
        default: break;
    }
    set_error("rotquant: hblock must be 0, 16, 64 or 256 (got %d)", hblock);
    return -1;
}

}  // namespace
}  // namespace mq
