// Quantized GEMM for M <= 4 rows (the adaLN modulation linear at M = 1 and other single-token
// calls): HBM-bound, so each weight byte is read once with 16-byte coalesced loads and multiplied
// on the VALU with v_dot4_i32_i8 (no MFMA, no LDS tiles for the weights).
//
// Workgroup: 4 wavefronts; each wavefront owns 4 output columns, 16 lanes per column (one DPP row).
// A column's weight row is read in 16-byte chunks (32 K values of packed 4-bit weights, 16 of int8):
// lane j takes chunks j, j + 16, j + 32, ..., so every load instruction reads 256 contiguous bytes
// of each of the wavefront's 4 rows, and every lane issues the loads of all its chunks (with their
// zero-points and scales) at once, after the activation loads: loads complete in issue order, so
// the activation staging and the barrier finish while the weights are still on their way, and each
// lane then works through its chunks as they arrive (rows longer than kH chunks per lane take one
// round of loads per kH chunks). The activation rows are staged once per workgroup in LDS in
// 16-value blocks (the first and second half of every packed chunk in separate arrays, so the 16
// lanes of a column read 256 contiguous bytes); for 4-bit weights each 8-value block is stored
// de-interleaved (even K in one dword, odd K in the next), so a packed weight dword needs only nibble
// masks: (w & 0x0f0f0f0f) pairs with the even activations, (w >> 4) & 0x0f0f0f0f with the odd ones.
// Each chunk's exact integer sum D:
//   uint4 asym   D = sum a q - z * sum a (sum a staged per 16-value block)
//   int4 sym     the nibble is moved to the top of its byte (16 v), so D = 16 sum a v
//   GroupScale   acc += s[n, g] * D * f in fp32, f = 1/16 (int4 sym) times (-1)^g / 16 for the
//                activation layout 16 q negated in odd groups: every factor a power of two;
//                y = T(acc * sa[m] + bias[n]) after a reduction over the column's 16 lanes (T: the
//                output type)
//   RowScale     an int32 sum over all of K (exact), y = T(P * sa[m] * ws[n] + bias[n])
//   GroupPartials / RowAcc (parity entries) write the exact int32 group partials P[g, m, n] (the
//                two chunks of a group sit in lanes 2i and 2i + 1 and are added by a DPP exchange;
//                the x16 / sign factors of the int4 layouts undone by exact shifts) or the full-K sums
//
// One-row whole linears (FQ != 0, M = 1, K <= 4096) hand the GEMV the activation row itself: the
// workgroup's four waves rotate and quantize it as the rotate+quantize kernel does with four waves
// per row (same load layout, same mq_rotate.h instructions, the same cross-wave maximum), write the
// codes straight into the LDS staging and keep the row scale in a register. The row's loads are
// issued before the weight loads, so the quantizer's work overlaps their flight, and the linear is
// one launch instead of two with the same codes, scale and output bits.
#include "mq_device.h"
#include "mq_internal.h"
#include "mq_rotate.h"

namespace mq {
namespace {

constexpr int kWaves = 4;
constexpr int kCols = 4;        // output columns per wavefront (16 lanes each)

// Sum over the 16 lanes of a DPP row, returned in every lane of the row.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_mov<kRowRor8>(v);
    v += dpp_mov<kRowRor4>(v);
    v += dpp_mov<kQuadXor2>(v);
    v += dpp_mov<kQuadXor1>(v);
    return v;
}
__device__ __forceinline__ int row16_sum(int v) {
    v += __builtin_amdgcn_mov_dpp(v, kRowRor8, 0xf, 0xf, true);
    v += __builtin_amdgcn_mov_dpp(v, kRowRor4, 0xf, 0xf, true);
    v += __builtin_amdgcn_mov_dpp(v, kQuadXor2, 0xf, 0xf, true);
    v += __builtin_amdgcn_mov_dpp(v, kQuadXor1, 0xf, 0xf, true);
    return v;
}

// One row (the adaLN modulation linear, M = 1) is built for five waves per SIMD: 1280 resident
// workgroups, so config 1's N = 18432 (1152 workgroups) runs in one wave of workgroups.
// FQ: 0 = int8 / int4 codes from qa and sa; else the row from x, rotated and quantized in the
// prologue to int8 codes (1), int4 codes one per byte (2) or the x16 alternating layout (3).
template <WKind WK, Epi EPI, int AM, int MR, int FQ = 0>
__global__ void __launch_bounds__(64 * kWaves, MR == 1 ? 5 : 4) gemv_kernel(GemmArgs a) {
    static_assert(FQ == 0 || MR == 1, "the fused quantizer serves one row");
    constexpr bool kPacked = WK != WKind::I8;
    constexpr int kChunkK = kPacked ? 32 : 16;          // K values per 16-byte weight chunk
    constexpr int kH = kPacked ? 6 : 12;                // chunks a lane holds in registers at once
    extern __shared__ __attribute__((aligned(16))) uint32_t gv_smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = static_cast<int>(a.K);
    const int nch = K / kChunkK;                        // chunks per weight row
    const int blocks = K / 16;                          // 16-value activation blocks per row
    // LDS: [MR][blocks][4] dwords of staged activation blocks (packed weights: the first halves of
    // the chunks, then the second halves), then [MR][blocks] block sums (uint4 asym)
    uint32_t* act = gv_smem;
    int* bsum = reinterpret_cast<int*>(gv_smem + MR * blocks * 4);
    const int sub = lane & 15;                                              // lane within its column
    const int64_t n = (static_cast<int64_t>(blockIdx.x) * kWaves + wave) * kCols + (lane >> 4);
    const bool col_ok = n < a.N;
    const int64_t nc = col_ok ? n : 0;
    // int8 weights in 16-row tiles: chunk c of row nc is at block c / 4 of the row's 16-row band,
    // row nc % 16 within it; the wave's 4 columns are 4 consecutive rows of one band, so a load
    // still reads 256 contiguous bytes per K group
    const bool wt = !kPacked && a.wtile;
    const uint8_t* wrow = wt ? a.qw + (nc >> 4) * (K / 64) * 1024 + (nc & 15) * 64 : a.qw + nc * a.ldw;

    // Every load below is unconditional, from an address inside the operands (chunks past the row
    // read its last chunk, columns past N column 0, rows past M row M - 1): a load whose value were
    // selected away afterwards would make the compiler wait for it on the spot. Such values are
    // never used (the chunk loop stops at the row's end; rows and columns past the matrix are never
    // stored).
    constexpr int kStage = 2;                           // activation blocks per thread loaded up front
    uint4 xs[MR][kStage];
    // FQ: this lane's 16 input values (the rotate+quantize kernel's layout with four waves per row:
    // wave w takes columns 1024 w .. 1024 w + 1023, lane L the 16 of segment (L >> 2) + 16 (L & 3));
    // lanes past K load the row's first columns, whose values are left out and never stored
    [[maybe_unused]] uint4 xv[4];
    [[maybe_unused]] const int e0 = wave * 1024 + 16 * ((lane >> 2) + 16 * (lane & 3));
    if constexpr (FQ != 0) {
        const int e = e0 < K ? e0 : 0;
        if (a.x_dtype == kDtF32) {
            const float* xr = static_cast<const float*>(a.x) + e;
#pragma unroll
            for (int j = 0; j < 4; ++j) xv[j] = *reinterpret_cast<const uint4*>(xr + 4 * j);
        } else {
            const uint16_t* xr = static_cast<const uint16_t*>(a.x) + e;
            xv[0] = *reinterpret_cast<const uint4*>(xr);
            xv[1] = *reinterpret_cast<const uint4*>(xr + 8);   // (xv[2], xv[3]: fp32 rows only)
        }
    } else {
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int it = 0; it < kStage; ++it) {
                const int bl = tid + it * 64 * kWaves;
                const int64_t mr = m < a.M ? m : a.M - 1;
                xs[m][it] = *reinterpret_cast<const uint4*>(a.qa + mr * a.lda + 16 * (bl < blocks ? bl : 0));
            }
    }
    __builtin_amdgcn_sched_barrier(0);   // keep the activation loads ahead of the weight loads

    // chunks c0 + 16 h, h0 <= h < h1, of this lane: weights (lw), zero-point byte and fp16 scale (lz)
    uint4 w[kH];
    uint32_t zb[kH], sb[kH];
    auto load_chunks = [&](int c0, int h0, int h1, bool lw, bool lz) {
#pragma unroll
        for (int h = 0; h < kH; ++h) {
            if (h < h0 || h >= h1) continue;
            const int c = min(c0 + 16 * h, nch - 1);
            const int g = c * kChunkK / 64;
            if (lw)
                w[h] = *reinterpret_cast<const uint4*>(wrow + (wt ? (c >> 2) * 1024 + (c & 3) * 16
                                                                     : 16 * static_cast<int64_t>(c)));
            if (lz) {
                zb[h] = 0u;
                sb[h] = 0u;
                if constexpr (WK == WKind::U4Asym) zb[h] = a.wz[nc * a.ldwz + (g >> 1)];
                if constexpr (EPI == Epi::GroupScale) sb[h] = a.ws16[nc * a.ldws + g];
            }
        }
    };
    // FQ: the first kPre weight chunks go out before the row's quantizer runs, the rest of the
    // round and the zero-points and scales after it, so that the registers of the loads in flight
    // leave the quantizer the ones it needs (a spill there would first wait for every load)
    constexpr int kPre = FQ == 0 ? kH : (kPacked ? kH : 8);
    // chunks whose zero-points and scales go out before it (as many as leave no spill)
    constexpr int kPreZ = FQ == 0 ? kH : WK == WKind::U4Asym ? 2 : 3;
    load_chunks(sub, 0, kPreZ, true, true);
    load_chunks(sub, kPreZ, kPre, true, false);
    __builtin_amdgcn_sched_barrier(0);

    // Stage block bl of row m (de-interleaved per 8 values for 4-bit weights): packed weights put
    // block 2c + e (half e of chunk c) at position e * nch + c, int8 weights block c at c.
    auto stage = [&](int m, int bl, uint4 x) {
        uint4 o = x;
        int pos = bl;
        if constexpr (kPacked) {
            o.x = __builtin_amdgcn_perm(x.y, x.x, 0x06040200u);   // values 0, 2, 4, 6
            o.y = __builtin_amdgcn_perm(x.y, x.x, 0x07050301u);   // values 1, 3, 5, 7
            o.z = __builtin_amdgcn_perm(x.w, x.z, 0x06040200u);   // values 8, 10, 12, 14
            o.w = __builtin_amdgcn_perm(x.w, x.z, 0x07050301u);   // values 9, 11, 13, 15
            pos = (bl & 1) * nch + (bl >> 1);
        }
        *reinterpret_cast<uint4*>(act + (m * blocks + pos) * 4) = o;
        if constexpr (WK == WKind::U4Asym) {
            int sm = __builtin_amdgcn_sdot4(static_cast<int>(x.x), 0x01010101, 0, false);
            sm = __builtin_amdgcn_sdot4(static_cast<int>(x.y), 0x01010101, sm, false);
            sm = __builtin_amdgcn_sdot4(static_cast<int>(x.z), 0x01010101, sm, false);
            sm = __builtin_amdgcn_sdot4(static_cast<int>(x.w), 0x01010101, sm, false);
            bsum[m * blocks + bl] = sm;
        }
    };
    [[maybe_unused]] float s_row = 0.0f;   // FQ: the row's scale
    if constexpr (FQ != 0) {
        // rotate_chunk_lds / rotate_chunk of the Hadamard block, the row's absmax over the four
        // waves, the division-free scale and quant16's arithmetic (quant4_word, four values at a
        // time), in the rotate+quantize kernel's order
        constexpr int LIMIT = FQ == 1 ? 127 : 7;
        __shared__ __attribute__((aligned(16))) float tr_lds[kWaves * kTrWave];
        __shared__ float red_lds[kWaves];
        float* tb = tr_lds + wave * kTrWave + (lane & 3) * kTrG;
        const LdsTranspose tr{tb + (lane >> 2), tb + (lane >> 2) * kTrS};
        float v[16];
        if (a.x_dtype == kDtF32) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[4 * j] = __uint_as_float(xv[j].x);
                v[4 * j + 1] = __uint_as_float(xv[j].y);
                v[4 * j + 2] = __uint_as_float(xv[j].z);
                v[4 * j + 3] = __uint_as_float(xv[j].w);
            }
        } else {
            const uint32_t w16[8] = {xv[0].x, xv[0].y, xv[0].z, xv[0].w, xv[1].x, xv[1].y, xv[1].z, xv[1].w};
            const bool f16 = a.x_dtype == kDtF16;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                v[2 * j] = f16 ? f16lo(w16[j]) : bf16lo(w16[j]);
                v[2 * j + 1] = f16 ? f16hi(w16[j]) : bf16hi(w16[j]);
            }
        }
        const int hb = a.hblock;
        if (hb >= 16) {
            stage_reg<0>(v);          // element stride 1  (c0 c1)
            stage_reg<2>(v);          // element stride 4  (c2 c3)
        }
        if (hb >= 64) {
            tr(v);                    // registers now hold c4..c7
            stage_reg<0>(v);          // element stride 16 (c4 c5)
            if (hb >= 256) stage_reg<2>(v);   // element stride 64 (c6 c7)
            tr(v);                    // back to the load layout
        }
        float amc = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) amc = __builtin_fmaxf(amc, __builtin_fabsf(v[j]));
        float am = __builtin_fmaxf(0.0f, e0 < K ? amc : 0.0f);
        am = wave_max_nonneg(am);
        if (lane == 0) red_lds[wave] = am;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kWaves; ++i) am = __builtin_fmaxf(am, red_lds[i]);
        const float s = __builtin_fmaxf(div_limit<LIMIT>(am), 1e-10f);
        const float r = recip_row(s);
        // the x16 layout negates odd 64-column groups: column bit 6 is lane bit 4 here
        const float sg = FQ == 3 && ((lane >> 4) & 1) ? -1.0f : 1.0f;
        uint32_t word[4];
#pragma unroll
        for (int hi = 0; hi < 4; ++hi) word[hi] = quant4_word<LIMIT, FQ == 3>(v + 4 * hi, sg, r, s);
        if (e0 < K) stage(0, e0 >> 4, make_uint4(word[0], word[1], word[2], word[3]));
        s_row = s;
        load_chunks(sub, kPre, kH, true, false);
        load_chunks(sub, kPreZ, kH, false, true);
    } else {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
#pragma unroll
            for (int it = 0; it < kStage; ++it) {
                const int bl = tid + it * 64 * kWaves;
                if (bl < blocks) stage(m, bl, xs[m][it]);
            }
            // rows longer than kStage * 256 blocks: the rest block by block
            for (int bl = tid + kStage * 64 * kWaves; bl < blocks; bl += 64 * kWaves)
                stage(m, bl, *reinterpret_cast<const uint4*>(a.qa + (m < a.M ? m : a.M - 1) * a.lda + 16 * bl));
        }
    }
    __syncthreads();

    float accf[MR];
    int acci[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        accf[m] = 0.0f;
        acci[m] = 0;
    }
    for (int c0 = sub; c0 < nch; c0 += 16 * kH) {
        if (c0 != sub) load_chunks(c0, 0, kH, true, true);
#pragma unroll
        for (int h = 0; h < kH; ++h) {
            const int c = c0 + 16 * h;
            if (c >= nch) break;
            const int g = c * kChunkK / 64;
            int z = 0;
            if constexpr (WK == WKind::U4Asym) z = (zb[h] >> (4 * (g & 1))) & 0xf;
            [[maybe_unused]] float s = 0.0f;
            if constexpr (EPI == Epi::GroupScale) {
                s = f16_bits_to_f32(static_cast<uint16_t>(sb[h]));
                if constexpr (WK == WKind::I4Sym) s *= 0.0625f;
                if constexpr (AM == 2) s *= (g & 1) ? -0.0625f : 0.0625f;
            }
            const uint32_t wd[4] = {w[h].x, w[h].y, w[h].z, w[h].w};
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                int d = 0;
                if constexpr (WK == WKind::I8) {
                    const uint4 x = *reinterpret_cast<const uint4*>(act + (m * blocks + c) * 4);
                    const uint32_t xr[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        d = __builtin_amdgcn_sdot4(static_cast<int>(wd[j]), static_cast<int>(xr[j]), d, false);
                } else {
                    // weight dword j holds k = 32 c + 8 j .. + 7 (low nibbles the even k): block
                    // half j / 2 of the chunk, de-interleaved dwords 2 (j % 2) (even) and + 1 (odd)
                    const uint4 x0 = *reinterpret_cast<const uint4*>(act + (m * blocks + c) * 4);
                    const uint4 x1 = *reinterpret_cast<const uint4*>(act + (m * blocks + nch + c) * 4);
                    const uint32_t xr[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t lo = WK == WKind::U4Asym ? wd[j] & 0x0f0f0f0fu : (wd[j] << 4) & 0xf0f0f0f0u;
                        const uint32_t hi = WK == WKind::U4Asym ? (wd[j] >> 4) & 0x0f0f0f0fu : wd[j] & 0xf0f0f0f0u;
                        d = __builtin_amdgcn_sdot4(static_cast<int>(lo), static_cast<int>(xr[2 * j]), d, false);
                        d = __builtin_amdgcn_sdot4(static_cast<int>(hi), static_cast<int>(xr[2 * j + 1]), d, false);
                    }
                    if constexpr (WK == WKind::U4Asym) {
                        const int2 bs = *reinterpret_cast<const int2*>(bsum + m * blocks + 2 * c);
                        d -= z * (bs.x + bs.y);
                    }
                }
                if constexpr (EPI == Epi::GroupScale) {
                    accf[m] = __builtin_fmaf(static_cast<float>(d), s, accf[m]);
                } else if constexpr (EPI == Epi::GroupPartials) {
                    // chunks 2g and 2g + 1 sit in lanes 2i and 2i + 1 of the same step (nch is even,
                    // so both lanes of a pair are inside the row or both past it)
                    static_assert(kPacked, "group partials are defined for 4-bit weights");
                    constexpr int shift = (WK == WKind::I4Sym ? 4 : 0) + (AM == 2 ? 4 : 0);
                    int pv = (d + __builtin_amdgcn_mov_dpp(d, kQuadXor1, 0xf, 0xf, true)) >> shift;   // exact
                    if (AM == 2 && (g & 1)) pv = -pv;
                    if ((sub & 1) == 0 && m < a.M && col_ok)
                        a.part[(static_cast<int64_t>(g) * a.M + m) * a.N + n] = pv;
                } else {
                    acci[m] += d;
                }
            }
        }
    }
    if constexpr (EPI == Epi::GroupPartials) return;
    // reductions over the column's 16 lanes; lane 0 of each row writes
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        float t;
        if constexpr (EPI == Epi::GroupScale) {
            const float v = row16_sum(accf[m]);
            t = m < a.M ? v * (FQ != 0 ? s_row : a.sa[m]) : 0.0f;
        } else {
            int v = row16_sum(acci[m]);
            if constexpr (WK == WKind::I4Sym) v >>= 4;   // exact: a multiple of 16
            if constexpr (EPI == Epi::RowAcc) {
                if (sub == 0 && m < a.M && col_ok) a.part[m * a.N + n] = v;
                continue;
            }
            t = m < a.M && col_ok ? static_cast<float>(v) * (FQ != 0 ? s_row : a.sa[m]) * a.ws32[n] : 0.0f;
        }
        if (sub == 0 && m < a.M && col_ok) {
            if (a.bias) t += load_as_f32(a.bias, a.bias_dtype, n);
            store_from_f32(a.y, a.y_dtype, m * a.ldy + n, t);
        }
    }
}

template <WKind WK, Epi EPI, int AM, int FQ = 0>
int launch_rows(const GemmArgs& a, hipStream_t stream) {
    const int64_t cols = kWaves * kCols;
    const dim3 grid(static_cast<unsigned>((a.N + cols - 1) / cols));
#define MQ_GV(MR)                                                                                       \
    do {                                                                                                \
        const size_t lds = MR * (a.K / 16) * (16 + (WK == WKind::U4Asym ? 4 : 0));                     \
        auto kern = gemv_kernel<WK, EPI, AM, MR, FQ>;                                                   \
        if (lds > 65536 && hipFuncSetAttribute(reinterpret_cast<const void*>(kern),                     \
                                               hipFuncAttributeMaxDynamicSharedMemorySize,              \
                                               static_cast<int>(lds)) != hipSuccess) {                  \
            set_error("gemv: cannot reserve %zu bytes of LDS", lds);                                    \
            return -3;                                                                 \
        }                                                                                               \
        hipLaunchKernelGGL(kern, grid, dim3(64 * kWaves), lds, stream, a);                              \
        return launch_status("gemv");                                                                   \
    } while (0)
    if constexpr (FQ != 0) {
        MQ_GV(1);
    } else {
        switch (a.M) {
            case 1: MQ_GV(1);
            case 2: MQ_GV(2);
            case 3: MQ_GV(3);
            default: MQ_GV(4);
        }
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
    if (a.x) {   // a one-row whole linear: the GEMV quantizes the row itself (gemv_quantizes_row)
        if (a.M != 1 || a.K > 4096) {
            set_error("gemv: the fused row quantizer takes one row of K <= 4096");
            return -2;
        }
        if (epi == Epi::GroupScale && a.act_mode == 2) {   // int4 codes, x16 alternating layout
            if (wk == WKind::U4Asym) return launch_rows<WKind::U4Asym, Epi::GroupScale, 2, 3>(a, stream);
            if (wk == WKind::I4Sym) return launch_rows<WKind::I4Sym, Epi::GroupScale, 2, 3>(a, stream);
        } else if (epi == Epi::GroupScale && a.act_mode == 0 && a.x_bits == 8) {
            if (wk == WKind::U4Asym) return launch_rows<WKind::U4Asym, Epi::GroupScale, 0, 1>(a, stream);
            if (wk == WKind::I4Sym) return launch_rows<WKind::I4Sym, Epi::GroupScale, 0, 1>(a, stream);
        } else if (epi == Epi::RowScale) {
            if (wk == WKind::I8)
                return a.x_bits == 4 ? launch_rows<WKind::I8, Epi::RowScale, 0, 2>(a, stream)
                                     : launch_rows<WKind::I8, Epi::RowScale, 0, 1>(a, stream);
            if (wk == WKind::I4Sym)
                return a.x_bits == 4 ? launch_rows<WKind::I4Sym, Epi::RowScale, 0, 2>(a, stream)
                                     : launch_rows<WKind::I4Sym, Epi::RowScale, 0, 1>(a, stream);
        }
        set_error("gemv: unsupported fused row quantizer combination");
        return -2;
    }
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
