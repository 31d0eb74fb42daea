// Microbenchmark: v_mfma_i32_16x16x64_i8 followed by the 4 fmas that read the VGPR result of the
// MFMA issued LAG tiles earlier (the W4A8 GEMM's per-group epilogue pattern), 2 waves per SIMD, with
// the scheduling constructs the GEMM kernel could use: an empty asm that "writes" the MFMA's C
// operand (pinning the MFMA), sched_barriers after the MFMA and after the fmas, an empty asm on the
// accumulators. Operand data: MASK selects the operand bits (0x0f0f0f0f small, 0xffffffff random).
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#ifndef MASK
#define MASK 0x0f0f0f0f
#endif
typedef int v4i __attribute__((ext_vector_type(4)));

template <int LAG, int PIN>
__global__ void __launch_bounds__(512) k(int iters, float* outf) {
    const uint32_t lane = threadIdx.x + blockIdx.x * 512u;
    // 4 A and 8 B operands: the 32 MFMAs of a step sequence are all distinct (with fewer operand
    // combinations the compiler merges identical MFMAs)
    v4i a[4], b[8];
    for (int i = 0; i < 4; ++i)
        for (int r = 0; r < 4; ++r) a[i][r] = (int)((lane * 0x9E3779B1u + i * 3 + r) * 2654435761u) & (int)MASK;
    for (int i = 0; i < 8; ++i)
        for (int r = 0; r < 4; ++r) b[i][r] = (int)((lane * 0x85EBCA77u + i + r * 11) * 2246822519u) & (int)MASK;
    v4i c = {0x4B400000, 0x4B400000, 0x4B400000, 0x4B400000};
    v4i d[8];
    float acc[32][4];
    for (int t = 0; t < 32; ++t) for (int r = 0; r < 4; ++r) acc[t][r] = 0.f;
    for (int t = 0; t < 8; ++t) for (int r = 0; r < 4; ++r) d[t][r] = 0;
    const float s = 1.0f + (float)(lane & 7) * 0.001f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int t = 0; t < 32; ++t) {
            if constexpr (PIN & 1) asm volatile("" : "+v"(c));
            d[t & 7] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t & 3], b[t >> 2], c, 0, 0, 0);
            if constexpr (PIN & 2) __builtin_amdgcn_sched_barrier(0);
            const int tp = (t + 32 - LAG) & 31;
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[tp][r] = __builtin_fmaf(__int_as_float(d[tp & 7][r]), s, acc[tp][r]);
            if constexpr (PIN & 4) asm volatile("" : "+v"(acc[tp][0]), "+v"(acc[tp][1]), "+v"(acc[tp][2]), "+v"(acc[tp][3]));
            if constexpr (PIN & 8) __builtin_amdgcn_sched_barrier(0);
        }
    }
    float y = 0.f;
    for (int t = 0; t < 32; ++t) for (int r = 0; r < 4; ++r) y += acc[t][r];
    outf[lane] = y;
}

template <int LAG, int PIN>
void run(const char* name, int blocks) {
    const int iters = 1000;
    float* of;
    (void)hipMalloc(&of, blocks * 512 * 4);
    hipLaunchKernelGGL((k<LAG, PIN>), dim3(blocks), dim3(512), 0, 0, 10, of);
    (void)hipDeviceSynchronize();
    hipEvent_t e0, e1; (void)hipEventCreate(&e0); (void)hipEventCreate(&e1);
    (void)hipEventRecord(e0);
    for (int rep = 0; rep < 3; ++rep) hipLaunchKernelGGL((k<LAG, PIN>), dim3(blocks), dim3(512), 0, 0, iters, of);
    (void)hipEventRecord(e1); (void)hipEventSynchronize(e1);
    float ms; (void)hipEventElapsedTime(&ms, e0, e1);
    const double mfma_per_simd = 3.0 * iters * 32 * (blocks * 8.0 / 1024.0);
    printf("%-30s blocks %4d: %.1f cycles per MFMA+4fma at 2.4 GHz\n", name, blocks, ms * 1e6 / mfma_per_simd * 2.4);
    (void)hipFree(of);
}

int main() {
    for (int rep = 0; rep < 2; ++rep) {
        run<3, 0>("lag3 free", 512);
        run<3, 1>("lag3 seed asm", 512);
        run<3, 2>("lag3 barrier after mfma", 512);
        run<3, 4>("lag3 acc asm", 512);
        run<3, 8>("lag3 barrier after fmas", 512);
        run<3, 10>("lag3 both barriers", 512);
        run<3, 14>("lag3 barriers + acc asm", 512);
        run<3, 15>("lag3 all pins", 512);
    }
    return 0;
}
