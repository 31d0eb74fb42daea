// Quantized GEMM for M <= 4 rows (the adaLN modulation linear at M = 1 and other single-token
// calls): HBM-bound, so each weight byte is read once with 16-byte coalesced loads and multiplied
// on the VALU with v_dot4_i32_i8 (no MFMA, no LDS tiles for the weights).
//
// Workgroup: 4 wavefronts; each wavefront owns 4 output columns at a time and splits their K range
// over its lanes in 16-byte weight chunks (16 K values of int8 weights, 32 of packed 4-bit). The
// activation rows are staged once per workgroup in LDS; for 4-bit weights each 8-value block is
// stored de-interleaved (even K in one dword, odd K in the next), so a packed weight dword needs
// only nibble masks: (w & 0x0f0f0f0f) pairs with the even activations, (w >> 4) & 0x0f0f0f0f with
// the odd ones. Exact integer chunk sums D then enter the epilogue:
//   uint4 asym   D = sum a q - z * sum a (the per-chunk activation sums are staged too)
//   int4 sym     the nibble is moved to the top of its byte (16 v), so D = 16 sum a v
//   GroupScale   acc += s[n, g] * D * f in fp32, f = 1/16 (int4 sym) times (-1)^g / 16 for the
//                activation layout 16 q negated in odd groups: every factor a power of two;
//                y = T(acc * sa[m] + bias[n]) after a wavefront reduction (T: the output type)
//   RowScale     an int32 sum over all of K (exact), y = T(P * sa[m] * ws[n] + bias[n])
//   GroupPartials / RowAcc (parity entries) write the exact int32 group partials P[g, m, n] (the
//                two half-group chunk sums of adjacent lanes added, the x16 / sign factors of the
//                int4 layouts undone by exact shifts) or the full-K int32 sums
#include "mq_device.h"
#include "mq_internal.h"

namespace mq {
namespace {

constexpr int kWaves = 4;
constexpr int kCols = 4;        // output columns per wavefront step

// One row (the adaLN modulation linear, M = 1) is built for five waves per SIMD: 1280 resident
// workgroups, so config 1's N = 18432 (1152 workgroups) runs in one wave of workgroups instead of
// a full second wave for its last 128 (the uint4 kernel then keeps 12 bytes of values in scratch).
template <WKind WK, Epi EPI, int AM, int MR>
__global__ void __launch_bounds__(64 * kWaves, MR == 1 ? 5 : 4) gemv_kernel(GemmArgs a) {
    constexpr bool kPacked = WK != WKind::I8;
    constexpr int kChunkK = kPacked ? 32 : 16;          // K values per 16-byte weight chunk
    extern __shared__ __attribute__((aligned(16))) uint32_t gv_smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = static_cast<int>(a.K);
    const int nchunks = K / kChunkK;
    uint32_t* act = gv_smem;                            // [MR][K / 4] dwords
    int* asum = reinterpret_cast<int*>(gv_smem + MR * (K / 4));   // [MR][nchunks] (uint4 asym)
    const int64_t n_base = (static_cast<int64_t>(blockIdx.x) * kWaves + wave) * kCols;

    // Raw weight chunk, zero-point byte and fp16 scale of chunk ch for the wave's kCols columns
    // (zero past the row's end or past N). Decoding waits for the loads, so it happens at the use:
    // the first chunk is loaded before the activation staging and every later one an iteration
    // ahead, and the loads' latency overlaps the staging and the previous chunk's arithmetic.
    struct Chunk {
        uint4 w[kCols];
        uint32_t z[kCols], s[kCols];
    };
    auto load_chunk = [&](int ch, Chunk& t) {
        const int g = ch * kChunkK / 64;
#pragma unroll
        for (int c = 0; c < kCols; ++c) {
            const int64_t n = n_base + c;
            const bool ok = ch < nchunks && n < a.N;
            t.w[c] = ok ? *reinterpret_cast<const uint4*>(a.qw + n * a.ldw + ch * 16) : uint4{0u, 0u, 0u, 0u};
            t.z[c] = 0u;
            t.s[c] = 0u;
            if constexpr (WK == WKind::U4Asym) t.z[c] = ok ? a.wz[n * a.ldwz + (g >> 1)] : 0u;
            if constexpr (EPI == Epi::GroupScale) t.s[c] = ok ? a.ws16[n * a.ldws + g] : 0u;
        }
    };
    Chunk cur, next;
    load_chunk(lane, cur);

    // stage the activation rows (de-interleaved per 8 values for 4-bit weights)
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        for (int b = tid; b < K / 8; b += 64 * kWaves) {
            const uint2 x = m < a.M ? *reinterpret_cast<const uint2*>(a.qa + m * a.lda + 8 * b) : uint2{0u, 0u};
            uint2 o = x;
            if constexpr (kPacked) {
                o.x = __builtin_amdgcn_perm(x.y, x.x, 0x06040200u);   // values 0, 2, 4, 6
                o.y = __builtin_amdgcn_perm(x.y, x.x, 0x07050301u);   // values 1, 3, 5, 7
            }
            *reinterpret_cast<uint2*>(act + m * (K / 4) + 2 * b) = o;
        }
    }
    if constexpr (WK == WKind::U4Asym) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            for (int c = tid; c < nchunks; c += 64 * kWaves) {
                int s = 0;
                if (m < a.M) {
                    const uint4 x0 = *reinterpret_cast<const uint4*>(a.qa + m * a.lda + c * kChunkK);
                    const uint4 x1 = *reinterpret_cast<const uint4*>(a.qa + m * a.lda + c * kChunkK + 16);
                    const uint32_t w[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                    for (int j = 0; j < 8; ++j) s = __builtin_amdgcn_sdot4(static_cast<int>(w[j]), 0x01010101, s, false);
                }
                asum[m * nchunks + c] = s;
            }
        }
    }
    __syncthreads();

    float accf[kCols][MR];
    int acci[kCols][MR];
#pragma unroll
    for (int c = 0; c < kCols; ++c)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            accf[c][m] = 0.0f;
            acci[c][m] = 0;
        }
    for (int ch = lane; ch < nchunks; ch += 64) {
        load_chunk(ch + 64, next);
        const int g = ch * kChunkK / 64;
#pragma unroll
        for (int c = 0; c < kCols; ++c) {
            const uint32_t wd[4] = {cur.w[c].x, cur.w[c].y, cur.w[c].z, cur.w[c].w};
            int z = 0;
            if constexpr (WK == WKind::U4Asym) z = (cur.z[c] >> (4 * (g & 1))) & 0xf;
            [[maybe_unused]] float s = 0.0f;
            if constexpr (EPI == Epi::GroupScale) {
                s = f16_bits_to_f32(static_cast<uint16_t>(cur.s[c]));
                if constexpr (WK == WKind::I4Sym) s *= 0.0625f;
                if constexpr (AM == 2) s *= (g & 1) ? -0.0625f : 0.0625f;
            }
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const uint32_t* xr = act + m * (K / 4) + ch * (kChunkK / 4);
                int d = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if constexpr (WK == WKind::I8) {
                        d = __builtin_amdgcn_sdot4(static_cast<int>(wd[j]), static_cast<int>(xr[j]), d, false);
                    } else if constexpr (WK == WKind::U4Asym) {
                        d = __builtin_amdgcn_sdot4(static_cast<int>(wd[j] & 0x0f0f0f0fu), static_cast<int>(xr[2 * j]), d, false);
                        d = __builtin_amdgcn_sdot4(static_cast<int>((wd[j] >> 4) & 0x0f0f0f0fu),
                                                   static_cast<int>(xr[2 * j + 1]), d, false);
                    } else {   // signed int4 as 16 v
                        d = __builtin_amdgcn_sdot4(static_cast<int>((wd[j] << 4) & 0xf0f0f0f0u), static_cast<int>(xr[2 * j]), d, false);
                        d = __builtin_amdgcn_sdot4(static_cast<int>(wd[j] & 0xf0f0f0f0u), static_cast<int>(xr[2 * j + 1]), d, false);
                    }
                }
                if constexpr (WK == WKind::U4Asym) d -= z * asum[m * nchunks + ch];
                if constexpr (EPI == Epi::GroupScale) {
                    accf[c][m] = __builtin_fmaf(static_cast<float>(d), s, accf[c][m]);
                } else if constexpr (EPI == Epi::GroupPartials) {
                    // chunks 2g and 2g + 1 (the two halves of group g) sit in lanes 2j and 2j + 1 of
                    // the same iteration; both lanes of a pair are active or inactive together
                    // (the chunk count is even), so the exchange reads a live lane
                    static_assert(kPacked, "group partials are defined for 4-bit weights");
                    constexpr int shift = (WK == WKind::I4Sym ? 4 : 0) + (AM == 2 ? 4 : 0);
                    int pv = (d + __shfl_xor(d, 1, 64)) >> shift;   // exact: a multiple of 2^shift
                    if (AM == 2 && (g & 1)) pv = -pv;
                    const int64_t n = n_base + c;
                    if ((lane & 1) == 0 && m < a.M && n < a.N)
                        a.part[(static_cast<int64_t>(g) * a.M + m) * a.N + n] = pv;
                } else {
                    acci[c][m] += d;
                }
            }
        }
        cur = next;
    }
    if constexpr (EPI == Epi::GroupPartials) return;
    // wavefront reductions and the epilogue (lane 0 writes)
#pragma unroll
    for (int c = 0; c < kCols; ++c) {
        const int64_t n = n_base + c;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float t;
            if constexpr (EPI == Epi::GroupScale) {
                float v = accf[c][m];
#pragma unroll
                for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
                t = m < a.M ? v * a.sa[m] : 0.0f;
            } else {
                int v = acci[c][m];
#pragma unroll
                for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
                if constexpr (WK == WKind::I4Sym) v >>= 4;   // exact: a multiple of 16
                if constexpr (EPI == Epi::RowAcc) {
                    if (lane == 0 && m < a.M && n < a.N) a.part[m * a.N + n] = v;
                    continue;
                }
                t = m < a.M && n < a.N ? static_cast<float>(v) * a.sa[m] * a.ws32[n] : 0.0f;
            }
            if (lane == 0 && m < a.M && n < a.N) {
                if (a.bias) t += load_as_f32(a.bias, a.bias_dtype, n);
                store_from_f32(a.y, a.y_dtype, m * a.ldy + n, t);
            }
        }
    }
}

template <WKind WK, Epi EPI, int AM>
int launch_rows(const GemmArgs& a, hipStream_t stream) {
    const int64_t cols = kWaves * kCols;
    const dim3 grid(static_cast<unsigned>((a.N + cols - 1) / cols));
#define MQ_GV(MR)                                                                                       \
    do {                                                                                                \
        const size_t lds = MR * a.K + (WK == WKind::U4Asym ? MR * (a.K / 32) * 4 : 0);                  \
        auto kern = gemv_kernel<WK, EPI, AM, MR>;                                                       \
        if (lds > 65536 && hipFuncSetAttribute(reinterpret_cast<const void*>(kern),                     \
                                               hipFuncAttributeMaxDynamicSharedMemorySize,              \
                                               static_cast<int>(lds)) != hipSuccess) {                  \
            set_error("gemv: cannot reserve %zu bytes of LDS", lds);                                    \
            return -3;                                                                 \
        }                                                                                               \
        hipLaunchKernelGGL(kern, grid, dim3(64 * kWaves), lds, stream, a);                              \
        return launch_status("gemv");                                                                   \
    } while (0)
    switch (a.M) {
        case 1: MQ_GV(1);
        case 2: MQ_GV(2);
        case 3: MQ_GV(3);
        default: MQ_GV(4);
    }
#undef MQ_GV
}

template <WKind WK, Epi EPI>
int launch_am(const GemmArgs& a, hipStream_t stream) {
    if (a.act_mode == 2) return launch_rows<WK, EPI, 2>(a, stream);
    return launch_rows<WK, EPI, 0>(a, stream);   // int8 codes, or int4 codes one per byte
}

}  // namespace

int launch_gemv(const GemmArgs& a, WKind wk, Epi epi, hipStream_t stream) {
    if (epi == Epi::GroupScale) {
        if (wk == WKind::U4Asym) return launch_am<WKind::U4Asym, Epi::GroupScale>(a, stream);
        if (wk == WKind::I4Sym) return launch_am<WKind::I4Sym, Epi::GroupScale>(a, stream);
    } else if (epi == Epi::GroupPartials) {
        if (wk == WKind::U4Asym) return launch_am<WKind::U4Asym, Epi::GroupPartials>(a, stream);
        if (wk == WKind::I4Sym) return launch_am<WKind::I4Sym, Epi::GroupPartials>(a, stream);
    } else if (epi == Epi::RowScale) {
        if (wk == WKind::I4Sym) return launch_rows<WKind::I4Sym, Epi::RowScale, 0>(a, stream);
        if (wk == WKind::I8) return launch_rows<WKind::I8, Epi::RowScale, 0>(a, stream);
    } else if (epi == Epi::RowAcc) {
        if (wk == WKind::I4Sym) return launch_rows<WKind::I4Sym, Epi::RowAcc, 0>(a, stream);
        if (wk == WKind::I8) return launch_rows<WKind::I8, Epi::RowAcc, 0>(a, stream);
    }
    set_error("gemv: unsupported weight kind / epilogue combination");
    return -2;
}

}  // namespace mq
