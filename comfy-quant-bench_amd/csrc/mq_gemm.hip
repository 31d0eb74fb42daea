// Quantized GEMMs on gfx950 int8 MFMA (v_mfma_i32_32x32x32_i8) with LDS-staged tiles.
//
// Workgroup tile 128 (M) x 128 (N) x 64 (K = one weight group per k-step), 4 wavefronts in a
// 2 x 2 grid, each owning a 64 x 64 output tile made of 2 x 2 MFMA 32x32 tiles. Global loads of
// step k+1 are issued before the MFMAs of step k and land in the other half of a double-buffered
// LDS tile, so one barrier per k-step orders both reuse directions.
//
// 4-bit weights stay packed in HBM and are unpacked to int8 once per workgroup on their way into
// LDS: byte j of a packed row holds k = 2j (low nibble) and k = 2j + 1 (high nibble). For the
// uint4 asymmetric scheme each byte becomes (q - z) in [-15, 15] without inter-byte borrows by
// computing ((q | 0x80) - z) ^ 0x80 four bytes at a time; signed int4 is the same with q ^ 8 and
// z = 8.
//
// Epilogues:
//   GroupScale    acc[m,n] += float(P_g[m,n]) * ws[n,g] after every group; at the end
//                 y = T(acc * sa[m] + bias[n])      (g64_bench6.py:50-68 order of scales; T is
//                 the output type, bf16, fp16 or fp32).
//                 Activation layout 2 (16 * q, negated in odd groups) is undone through the scale.
//   GroupPartials writes P_g[m,n] (int32) for every group (parity entry)
//   RowScale      one int32 accumulator over all of K; y = T(P * sa[m] * ws[n] + bias[n])
//                 (policy 0 of experiments/qwen21-kernel/kernels/g64_gemm6.cu:5)
//   RowAcc        writes the full-K int32 accumulator (parity entry)
#include "mq_device.h"
#include "mq_internal.h"

namespace mq {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDS_ROW = 80;   // 64 bytes of K + 16 bytes of padding: conflict-free ds_read_b128

__device__ __forceinline__ void unpack8(uint32_t w, uint32_t zz, bool sym, uint32_t& o0, uint32_t& o1) {
    uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
    if (sym) {
        lo ^= 0x08080808u;
        hi ^= 0x08080808u;
    }
    lo = ((lo | 0x80808080u) - zz) ^ 0x80808080u;
    hi = ((hi | 0x80808080u) - zz) ^ 0x80808080u;
    o0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
    o1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
}

template <WKind WK, Epi EPI>
__global__ void __launch_bounds__(256) gemm_kernel(GemmArgs a) {
    constexpr bool kGroup = EPI == Epi::GroupScale || EPI == Epi::GroupPartials;
    __shared__ __attribute__((aligned(16))) int8_t As[2][BM * LDS_ROW];
    __shared__ __attribute__((aligned(16))) int8_t Bs[2][BN * LDS_ROW];
    __shared__ float Ss[2][BN];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * BM;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * BN;
    const int64_t M = a.M, N = a.N, K = a.K;
    const int KT = static_cast<int>(K / BK);

    // loader role: 2 threads per tile row, each 32 bytes of K (A, I8 weights) or 16 packed bytes
    const int lr = tid >> 1, lp = tid & 1;
    const bool a_ok = m0 + lr < M;
    const bool b_ok = n0 + lr < N;
    const int8_t* a_src = a.qa + (m0 + lr) * a.lda + lp * 32;
    const uint8_t* b_src = a.qw + (n0 + lr) * a.ldw + (WK == WKind::I8 ? lp * 32 : lp * 16);

    // Rows past M / N load from row 0 of the operand (always valid) and are zeroed afterwards,
    // so the loads stay unconditional and the fetched registers stay in registers.
    const int8_t* a_row = a_ok ? a_src : a.qa + lp * 32;
    const uint8_t* b_row = b_ok ? b_src : a.qw + (WK == WKind::I8 ? lp * 32 : lp * 16);
    const uint8_t* z_row = WK == WKind::U4Asym ? a.wz + (b_ok ? n0 + lr : 0) * a.ldwz : nullptr;
    const uint4 zero4 = make_uint4(0, 0, 0, 0);

    uint4 ra0, ra1, rb0, rb1 = zero4;
    uint32_t rz = 0;
    float rs = 0.0f;
    auto gload = [&](int kt) {
        const int64_t k0 = static_cast<int64_t>(kt) * BK;
        ra0 = *reinterpret_cast<const uint4*>(a_row + k0);
        ra1 = *reinterpret_cast<const uint4*>(a_row + k0 + 16);
        if constexpr (WK == WKind::I8) {
            rb0 = *reinterpret_cast<const uint4*>(b_row + k0);
            rb1 = *reinterpret_cast<const uint4*>(b_row + k0 + 16);
        } else {
            rb0 = *reinterpret_cast<const uint4*>(b_row + k0 / 2);
        }
        if constexpr (WK == WKind::U4Asym) {
            const uint32_t zb = z_row[kt >> 1];
            rz = (zb >> ((kt & 1) * 4)) & 0xfu;
        }
        if constexpr (EPI == Epi::GroupScale) {
            const int64_t n = n0 + (tid & (BN - 1));
            rs = n < N ? f16_bits_to_f32(a.ws16[n * a.ldws + kt]) : 0.0f;
            // layout 2 activations are 16 * q, negated in odd groups (exact power-of-two rescale)
            if (a.act_mode == 2) rs *= (kt & 1) ? -0.0625f : 0.0625f;
        }
    };
    auto fix_edges = [&]() {
        if (!a_ok) ra0 = ra1 = zero4;
        if (!b_ok) {
            rb0 = rb1 = zero4;
            rz = 0;
        }
    };
    auto lstore = [&](int buf) {
        fix_edges();
        *reinterpret_cast<uint4*>(&As[buf][lr * LDS_ROW + lp * 32]) = ra0;
        *reinterpret_cast<uint4*>(&As[buf][lr * LDS_ROW + lp * 32 + 16]) = ra1;
        if constexpr (WK == WKind::I8) {
            *reinterpret_cast<uint4*>(&Bs[buf][lr * LDS_ROW + lp * 32]) = rb0;
            *reinterpret_cast<uint4*>(&Bs[buf][lr * LDS_ROW + lp * 32 + 16]) = rb1;
        } else {
            constexpr bool sym = WK == WKind::I4Sym;
            const uint32_t zz = sym ? 0x08080808u : rz * 0x01010101u;
            uint4 u0, u1;
            unpack8(rb0.x, zz, sym, u0.x, u0.y);
            unpack8(rb0.y, zz, sym, u0.z, u0.w);
            unpack8(rb0.z, zz, sym, u1.x, u1.y);
            unpack8(rb0.w, zz, sym, u1.z, u1.w);
            *reinterpret_cast<uint4*>(&Bs[buf][lr * LDS_ROW + lp * 32]) = u0;
            *reinterpret_cast<uint4*>(&Bs[buf][lr * LDS_ROW + lp * 32 + 16]) = u1;
        }
        if constexpr (EPI == Epi::GroupScale) {
            if (tid < BN) Ss[buf][tid] = rs;
        }
    };

    const int fr = lane & 31, fk = (lane >> 5) * 16;
    v16i p[2][2];
    float acc[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                p[i][j][r] = 0;
                acc[i][j][r] = 0.0f;
            }
        }

    gload(0);
    lstore(0);
    __syncthreads();

    for (int kt = 0; kt < KT; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < KT) gload(kt + 1);

        v4i af[2][2], bfr[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
                af[i][kk] = *reinterpret_cast<const v4i*>(&As[buf][(wm * 64 + i * 32 + fr) * LDS_ROW + kk * 32 + fk]);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
                bfr[j][kk] = *reinterpret_cast<const v4i*>(&Bs[buf][(wn * 64 + j * 32 + fr) * LDS_ROW + kk * 32 + fk]);

#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if constexpr (kGroup) {
                    v16i z = {};
                    p[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i][0], bfr[j][0], z, 0, 0, 0);
                } else {
                    p[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i][0], bfr[j][0], p[i][j], 0, 0, 0);
                }
                p[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i][1], bfr[j][1], p[i][j], 0, 0, 0);
            }

        if constexpr (EPI == Epi::GroupScale) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float s = Ss[buf][wn * 64 + j * 32 + fr];
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        acc[i][j][r] = __builtin_fmaf(static_cast<float>(p[i][j][r]), s, acc[i][j][r]);
            }
        } else if constexpr (EPI == Epi::GroupPartials) {
            int32_t* part = a.part + static_cast<int64_t>(kt) * M * N;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int64_t col = n0 + wn * 64 + j * 32 + fr;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int64_t row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                        int32_t v = p[i][j][r];
                        if (a.act_mode == 2) v = (kt & 1) ? -(v >> 4) : (v >> 4);   // exact: a multiple of 16
                        if (row < M && col < N) part[row * N + col] = v;
                    }
                }
        }

        if (kt + 1 < KT) lstore(buf ^ 1);
        __syncthreads();
    }

    if constexpr (EPI == Epi::GroupPartials) return;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t col = n0 + wn * 64 + j * 32 + fr;
            if (col >= N) continue;
            if constexpr (EPI == Epi::RowAcc) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int64_t row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (row < M) a.part[row * N + col] = p[i][j][r];
                }
            } else {
                const float bias = a.bias ? load_as_f32(a.bias, a.bias_dtype, col) : 0.0f;
                const float wsc = EPI == Epi::RowScale ? a.ws32[col] : 1.0f;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int64_t row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (row >= M) continue;
                    float v;
                    if constexpr (EPI == Epi::RowScale)
                        v = static_cast<float>(p[i][j][r]) * a.sa[row] * wsc + bias;
                    else
                        v = acc[i][j][r] * a.sa[row] + bias;
                    store_from_f32(a.y, a.y_dtype, row * a.ldy + col, v);
                }
            }
        }
}

template <WKind WK>
int launch_wk(const GemmArgs& a, Epi epi, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((a.N + BN - 1) / BN), static_cast<unsigned>((a.M + BM - 1) / BM));
    const dim3 block(256);
    switch (epi) {
        case Epi::GroupScale:
            hipLaunchKernelGGL((gemm_kernel<WK, Epi::GroupScale>), grid, block, 0, stream, a);
            break;
        case Epi::GroupPartials:
            hipLaunchKernelGGL((gemm_kernel<WK, Epi::GroupPartials>), grid, block, 0, stream, a);
            break;
        case Epi::RowScale:
            hipLaunchKernelGGL((gemm_kernel<WK, Epi::RowScale>), grid, block, 0, stream, a);
            break;
        case Epi::RowAcc:
            hipLaunchKernelGGL((gemm_kernel<WK, Epi::RowAcc>), grid, block, 0, stream, a);
            break;
    }
    return launch_status("gemm");
}

}  // namespace

namespace {

bool runs_gemv(const GemmArgs& a, WKind wk, Epi epi) {
    return a.M <= 4 && a.M * a.K <= 131072 && !(wk == WKind::I8 && epi == Epi::GroupPartials) &&
           !(wk == WKind::U4Asym && epi == Epi::RowAcc);
}

}  // namespace

bool gemv_quantizes_row(const GemmArgs& a, WKind wk, Epi epi) {
    return runs_gemv(a, wk, epi) && a.M == 1 && a.K <= 4096 && (epi == Epi::GroupScale || epi == Epi::RowScale);
}

bool gemm_runs_wide(const GemmArgs& a, WKind wk, Epi epi) {
    if (runs_gemv(a, wk, epi)) return false;
    // The 256 x 256-tile kernel addresses each operand with 32-bit buffer offsets.
    // (4-bit weights with wtile set come expanded to int8 tiles, K bytes per row)
    const int64_t wbytes = wk == WKind::I8 || a.wtile ? a.K : a.K / 2;
    const bool fits32 = a.M * a.lda < (int64_t(1) << 31) && a.N * a.ldw < (int64_t(1) << 31) &&
                        (a.N * a.ldws + a.K / 64) * 2 < (int64_t(1) << 31) && wbytes <= a.ldw &&
                        (!a.atile || (a.M + 15) / 16 * 16 * a.K < (int64_t(1) << 31)) &&
                        (!a.wtile || (a.N + 15) / 16 * 16 * a.K < (int64_t(1) << 31));
    // (activation layout 1, int4 codes scaled in the kernel, is served by the 128-tile kernel only)
    // the wide kernel loads the zero-points of four groups as one 2-byte word and two groups'
    // scales as one dword per weight row
    const bool zs_aligned =
        (wk != WKind::U4Asym || a.wtile || (a.ldwz % 2 == 0 && reinterpret_cast<uintptr_t>(a.wz) % 2 == 0)) &&
        (epi != Epi::GroupScale || (a.ldws % 2 == 0 && reinterpret_cast<uintptr_t>(a.ws16) % 4 == 0));
    // (K >= 192: the wide kernel's last-row load correction needs at least three K groups)
    // Weights in 16-row tiles are read by the wide kernel at every M above the GEMV's few rows.
    return (a.M > 128 || a.wtile) && a.K >= 192 && fits32 && zs_aligned && a.act_mode != 1;
}

int launch_gemm(const GemmArgs& a, WKind wk, Epi epi, hipStream_t stream) {
    if (a.M == 0 || a.N == 0) return 0;
    if (a.atile && !gemm_runs_wide(a, wk, epi)) {
        set_error("gemm: activation codes in 16-row tiles are read by the wide kernel only");
        return -2;
    }
    if (a.wtile && wk != WKind::I8 && !gemm_runs_wide(a, wk, epi)) {
        set_error("gemm: expanded 4-bit weights are read by the wide kernel only (M > 4, K >= 192, "
                  "operands under 2 GiB); pass the packed weights");
        return -2;
    }
    // a few rows: HBM-bound, served by the dot4 kernel (activation rows staged in LDS); its parity
    // entries (exact group partials, full-K sums) run the same kernel
    if (runs_gemv(a, wk, epi)) return launch_gemv(a, wk, epi, stream);
    if (gemm_runs_wide(a, wk, epi)) {
        GemmArgs w = a;
        w.ksplit = 1;
        w.tile = 0;
        if (epi == Epi::GroupScale || epi == Epi::RowScale) {
            const bool int_sums = epi == Epi::RowScale;
            // a last, nearly empty wave of whole tile rows: those rows run as their own product
            // (smaller tiles, split along K where the workspace allows), the rest without them
            const int64_t tail = tail_rows(a.M, a.N, a.K);
            if (tail > 0) {
                GemmArgs t = w;
                t.M = tail;
                t.qa = a.atile ? a.qa + ((a.M - tail) >> 4) * (a.K << 4) : a.qa + (a.M - tail) * a.lda;
                t.sa = a.sa + (a.M - tail);
                t.y = static_cast<char*>(a.y) + (a.M - tail) * a.ldy * (a.y_dtype == kDtF32 ? 4 : 2);
                if (a.work) t.ksplit = choose_ksplit(t.M, t.N, t.K, t.work_bytes, &t.kgroups, int_sums);
                w.M = a.M - tail;
                w.work = nullptr;
                w.work_bytes = 0;
                const int rc = launch_gemm_wide(w, wk, epi, stream);
                return rc ? rc : launch_gemm_wide(t, wk, epi, stream);
            }
            if (a.work) w.ksplit = choose_ksplit(a.M, a.N, a.K, a.work_bytes, &w.kgroups, int_sums);
        }
        return launch_gemm_wide(w, wk, epi, stream);
    }
    if (a.wtile) {
        set_error("gemm: int8 weights in 16-row tiles need K >= 192 and operands under 2 GiB");
        return -2;
    }
    switch (wk) {
        case WKind::U4Asym:
            if (epi == Epi::RowScale || epi == Epi::RowAcc) break;
            return launch_wk<WKind::U4Asym>(a, epi, stream);
        case WKind::I4Sym: return launch_wk<WKind::I4Sym>(a, epi, stream);
        case WKind::I8:
            if (epi == Epi::GroupScale || epi == Epi::GroupPartials) break;
            return launch_wk<WKind::I8>(a, epi, stream);
    }
    set_error("gemm: unsupported weight kind / epilogue combination");
    return -2;
}

}  // namespace mq
