// Microbenchmark: does moving the fp32 work to the other wave of a SIMD (ping-pong roles) let it
// overlap the MFMAs? MFMAs with every operand in AGPRs next to VGPR-only fmas, in one wave or split
// across the two waves of a SIMD (512 threads per block, 2 waves per SIMD; waves w and w + 4 of a
// block share a SIMD), random full-range int8 operands.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void mfma_aaaa(v4i& d, v4i a, v4i b) {   // d (AGPR) += a * b (AGPR)
    asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(d) : "a"(a), "a"(b));
}
__device__ __forceinline__ void mfma_vvvv(v4i& d, v4i a, v4i b) {
    asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
}

// MODE 0: all-AGPR MFMA only. 1: all-AGPR MFMA + 4 indep VGPR fma each. 2: roles split (wave>>2):
// MFMA waves (all AGPR) / fma waves (128 fmas per 32-MFMA step). 3: roles split, MFMA waves VGPR.
// 4: all-VGPR MFMA + 4 indep fma. 5: roles split, both roles do half: MFMA wave also does 2 fma per
// MFMA, fma wave 64 fmas per step. 6: all-AGPR MFMA + 2 indep fma.
template <int MODE>
__global__ void __launch_bounds__(512) k(int iters, float* outf) {
    const uint32_t lane = threadIdx.x + blockIdx.x * 512u;
    const int role = (threadIdx.x >> 8) & 1;   // waves 4..7
    v4i a[4], b[8];
    for (int i = 0; i < 4; ++i)
        for (int r = 0; r < 4; ++r) a[i][r] = (int)((lane * 0x9E3779B1u + i * 3 + r) * 2654435761u);
    for (int i = 0; i < 8; ++i)
        for (int r = 0; r < 4; ++r) b[i][r] = (int)((lane * 0x85EBCA77u + i + r * 11) * 2246822519u);
    v4i d[4];
    for (int t = 0; t < 4; ++t) for (int r = 0; r < 4; ++r) d[t][r] = t + r;
    const float s = 1.0f + (float)(lane & 7) * 0.001f;
    float x[16];
    for (int q = 0; q < 16; ++q) x[q] = s * (q + 1);
    constexpr bool agpr = MODE == 0 || MODE == 1 || MODE == 2 || MODE == 5 || MODE == 6;
    if constexpr (agpr) {
        for (int i = 0; i < 4; ++i) asm volatile("" : "+a"(a[i]));
        for (int i = 0; i < 8; ++i) asm volatile("" : "+a"(b[i]));
        for (int i = 0; i < 4; ++i) asm volatile("" : "+a"(d[i]));
    }
    const bool split = MODE == 2 || MODE == 3 || MODE == 5;
    if (!split || role == 0) {
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int t = 0; t < 32; ++t) {
                if constexpr (agpr) mfma_aaaa(d[t & 3], a[t & 3], b[t >> 2]);
                else mfma_vvvv(d[t & 3], a[t & 3], b[t >> 2]);
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (MODE == 1 || MODE == 4) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) x[(4 * t + q) & 15] = __builtin_fmaf(x[(4 * t + q) & 15], s, 0.5f);
                    asm volatile("" : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]));
                } else if constexpr (MODE == 5 || MODE == 6) {
#pragma unroll
                    for (int q = 0; q < 2; ++q) x[(2 * t + q) & 15] = __builtin_fmaf(x[(2 * t + q) & 15], s, 0.5f);
                    asm volatile("" : "+v"(x[0]), "+v"(x[1]));
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else {
        constexpr int NF = MODE == 5 ? 64 : 128;
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int t = 0; t < NF; ++t) {
                x[t & 15] = __builtin_fmaf(x[t & 15], s, 0.5f);
                if ((t & 3) == 3) asm volatile("" : "+v"(x[(t - 3) & 15]), "+v"(x[(t - 2) & 15]), "+v"(x[(t - 1) & 15]), "+v"(x[t & 15]));
            }
        }
    }
    float y = 0;
    for (int q = 0; q < 16; ++q) y += x[q];
    for (int t = 0; t < 4; ++t) for (int r = 0; r < 4; ++r) y += (float)d[t][r];
    outf[lane] = y;
}

template <typename F>
void run(const char* name, F kern, double mfma_share) {
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
    // mfma_share: the fraction of waves that issue the 32 MFMAs per step (1, or 0.5 when roles split);
    // every configuration carries 4 fmas per MFMA issued (0 for the MFMA-only row)
    const double mfma_per_simd = (double)iters * 32 * mfma_share * (blocks * 8.0 / 1024.0);
    printf("%-52s %.1f cycles per MFMA at 2.4 GHz\n", name, best * 1e6 / mfma_per_simd * 2.4);
    (void)hipFree(of);
}

int main() {
    for (int rep = 0; rep < 2; ++rep) {
        run("0 all-agpr mfma only (both waves)", k<0>, 1.0);
        run("4 all-vgpr mfma + 4 indep fma (both waves)", k<4>, 1.0);
        run("1 all-agpr mfma + 4 indep fma (both waves)", k<1>, 1.0);
        run("6 all-agpr mfma + 2 indep fma (both waves)", k<6>, 1.0);
        run("2 split: agpr mfma wave | 128-fma wave", k<2>, 0.5);
        run("3 split: vgpr mfma wave | 128-fma wave", k<3>, 0.5);
        run("5 split: agpr mfma+2fma wave | 64-fma wave", k<5>, 0.5);
    }
    return 0;
}
