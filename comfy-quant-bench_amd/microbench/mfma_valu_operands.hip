// Microbenchmark: does the register file an MFMA reads decide how well VALU work overlaps it?
// v_mfma_i32_16x16x64_i8 (written as inline asm, so the operand files are exactly as stated) with
// 0, 2 or 4 VALU instructions per MFMA that read the result of the MFMA three back, 2 waves per
// SIMD, random full-range int8 operands. Variants: A / B operands in VGPRs or AGPRs (C / D stay in
// VGPRs, where the VALU reads them), fp32 fmas or integer adds, and the 32x32x32 MFMA with its 16
// results per lane.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v4i mfma_av(v4i a, v4i b, v4i c) {   // A, B in AGPRs; C, D in VGPRs
    v4i d;
    asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %3" : "=v"(d) : "a"(a), "a"(b), "v"(c));
    return d;
}
__device__ __forceinline__ v4i mfma_vv(v4i a, v4i b, v4i c) {   // every operand in VGPRs
    v4i d;
    asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
}
__device__ __forceinline__ v16i mfma32_av(v4i a, v4i b, v16i c) {
    v16i d;
    asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, %3" : "=v"(d) : "a"(a), "a"(b), "v"(c));
    return d;
}
__device__ __forceinline__ v16i mfma32_vv(v4i a, v4i b, v16i c) {
    v16i d;
    asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
}

// AG: A / B in AGPRs; NV: VALU instructions per MFMA (0, 2, 4); ADD: integer adds instead of fmas
template <bool AG, int NV, bool ADD>
__global__ void __launch_bounds__(512) k16(int iters, float* outf) {
    const uint32_t lane = threadIdx.x + blockIdx.x * 512u;
    v4i a[4], b[8];
    for (int i = 0; i < 4; ++i)
        for (int r = 0; r < 4; ++r) a[i][r] = (int)((lane * 0x9E3779B1u + i * 3 + r) * 2654435761u);
    for (int i = 0; i < 8; ++i)
        for (int r = 0; r < 4; ++r) b[i][r] = (int)((lane * 0x85EBCA77u + i + r * 11) * 2246822519u);
    if constexpr (AG) {
        for (int i = 0; i < 4; ++i) asm volatile("" : "+a"(a[i]));
        for (int i = 0; i < 8; ++i) asm volatile("" : "+a"(b[i]));
    }
    const v4i c = {0x4B400000, 0x4B400000, 0x4B400000, 0x4B400000};
    v4i d[4];
    float acc[8][4];
    for (int t = 0; t < 8; ++t) for (int r = 0; r < 4; ++r) acc[t][r] = 0.f;
    for (int t = 0; t < 4; ++t) for (int r = 0; r < 4; ++r) d[t][r] = 0;
    const float s = 1.0f + (float)(lane & 7) * 0.001f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int t = 0; t < 32; ++t) {
            // NV == 0 accumulates into d (a chain per ring slot) so no MFMA is dead code
            const v4i cin = NV == 0 ? d[t & 3] : c;
            d[t & 3] = AG ? mfma_av(a[t & 3], b[t >> 2], cin) : mfma_vv(a[t & 3], b[t >> 2], cin);
            __builtin_amdgcn_sched_barrier(0);
            const int tp = (t + 32 - 3) & 7;
#pragma unroll
            for (int r = 0; r < NV; ++r) {
                if constexpr (ADD) acc[tp][r] = __int_as_float(__float_as_int(acc[tp][r]) + d[tp & 3][r]);
                else acc[tp][r] = __builtin_fmaf(__int_as_float(d[tp & 3][r]), s, acc[tp][r]);
            }
            if constexpr (NV >= 4) asm volatile("" : "+v"(acc[tp][0]), "+v"(acc[tp][1]), "+v"(acc[tp][2]), "+v"(acc[tp][3]));
            else if constexpr (NV >= 2) asm volatile("" : "+v"(acc[tp][0]), "+v"(acc[tp][1]));
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    float y = 0;
    for (int t = 0; t < 8; ++t) for (int r = 0; r < 4; ++r) y += acc[t][r];
    for (int t = 0; t < 4; ++t) for (int r = 0; r < 4; ++r) y += (float)d[t][r];
    outf[lane] = y;
}

// 32x32x32: two MFMAs per 64-wide K group, 16 results per lane each; NV = 0 or 16 fmas per MFMA
template <bool AG, int NV>
__global__ void __launch_bounds__(512) k32(int iters, float* outf) {
    const uint32_t lane = threadIdx.x + blockIdx.x * 512u;
    v4i a[2], b[4];
    for (int i = 0; i < 2; ++i)
        for (int r = 0; r < 4; ++r) a[i][r] = (int)((lane * 0x9E3779B1u + i * 3 + r) * 2654435761u);
    for (int i = 0; i < 4; ++i)
        for (int r = 0; r < 4; ++r) b[i][r] = (int)((lane * 0x85EBCA77u + i + r * 11) * 2246822519u);
    if constexpr (AG) {
        for (int i = 0; i < 2; ++i) asm volatile("" : "+a"(a[i]));
        for (int i = 0; i < 4; ++i) asm volatile("" : "+a"(b[i]));
    }
    v16i c;
    for (int r = 0; r < 16; ++r) c[r] = 0x4B400000;
    v16i d[2];
    float acc[4][16];
    for (int t = 0; t < 4; ++t) for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;
    for (int t = 0; t < 2; ++t) for (int r = 0; r < 16; ++r) d[t][r] = 0;
    const float s = 1.0f + (float)(lane & 7) * 0.001f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const v16i cin = NV == 0 ? d[t & 1] : c;
            d[t & 1] = AG ? mfma32_av(a[t & 1], b[t >> 1], cin) : mfma32_vv(a[t & 1], b[t >> 1], cin);
            __builtin_amdgcn_sched_barrier(0);
            const int tp = (t + 8 - 1) & 3;
#pragma unroll
            for (int r = 0; r < NV; ++r) acc[tp][r] = __builtin_fmaf(__int_as_float(d[tp & 1][r]), s, acc[tp][r]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    float y = 0;
    for (int t = 0; t < 4; ++t) for (int r = 0; r < 16; ++r) y += acc[t][r];
    for (int t = 0; t < 2; ++t) for (int r = 0; r < 16; ++r) y += (float)d[t][r];
    outf[lane] = y;
}

template <typename F>
void run(const char* name, F kern, int mfma_per_iter, double per16) {
    const int iters = 2000, blocks = 512;
    float* of;
    (void)hipMalloc(&of, blocks * 512 * 4);
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(512), 0, 0, 10, of);
    (void)hipDeviceSynchronize();
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    float best = 1e30f;
    for (int rep = 0; rep < 3; ++rep) {
        (void)hipEventRecord(e0);
        hipLaunchKernelGGL(kern, dim3(blocks), dim3(512), 0, 0, iters, of);
        (void)hipEventRecord(e1);
        (void)hipEventSynchronize(e1);
        float ms;
        (void)hipEventElapsedTime(&ms, e0, e1);
        if (ms < best) best = ms;
    }
    // per16: how many 16x16x64 MFMAs one instruction is worth (1 or 2)
    const double mfma_per_simd = (double)iters * mfma_per_iter * per16 * (blocks * 8.0 / 1024.0);
    printf("%-46s %5.1f cycles per 16x16x64-equivalent at 2.4 GHz, %5.0f TOPS\n", name,
           best * 1e6 / mfma_per_simd * 2.4, mfma_per_simd * 1024.0 * 32768.0 / (best * 1e-3) / 1e12);
    (void)hipFree(of);
}

int main() {
    for (int rep = 0; rep < 2; ++rep) {
        run("16x16x64, VGPR A/B, MFMA only", k16<false, 0, false>, 32, 1.0);
        run("16x16x64, AGPR A/B, MFMA only", k16<true, 0, false>, 32, 1.0);
        run("16x16x64, VGPR A/B + 2 fma", k16<false, 2, false>, 32, 1.0);
        run("16x16x64, VGPR A/B + 4 fma", k16<false, 4, false>, 32, 1.0);
        run("16x16x64, AGPR A/B + 4 fma", k16<true, 4, false>, 32, 1.0);
        run("16x16x64, AGPR A/B + 4 integer adds", k16<true, 4, true>, 32, 1.0);
        run("32x32x32, AGPR A/B, MFMA only", k32<true, 0>, 8, 2.0);
        run("32x32x32, VGPR A/B + 16 fma", k32<false, 16>, 8, 2.0);
        run("32x32x32, AGPR A/B + 16 fma", k32<true, 16>, 8, 2.0);
    }
    return 0;
}
