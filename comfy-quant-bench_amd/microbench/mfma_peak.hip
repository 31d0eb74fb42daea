// Microbenchmark: sustained v_mfma_i32_16x16x64_i8 throughput on register operands (no memory
// traffic), with zero, random or small operand data, and with 0 / 2 / 4 fp32 fmas per MFMA reading
// earlier MFMA results (the per-group scale epilogue of the W4A8 GEMM issues 4 per MFMA).
// 2048 blocks of 256 threads (8 waves per SIMD), each wave 20000 x 8 MFMAs.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
typedef int v4i __attribute__((ext_vector_type(4)));

template <int FMAS>
__global__ void __launch_bounds__(256) k(int iters, uint32_t seedv, int* out, float* outf) {
    const uint32_t lane = threadIdx.x + blockIdx.x * 256u;
    v4i a[4], b[4];
    for (int i = 0; i < 4; ++i) {
        uint32_t h = (lane * 2654435761u) ^ (seedv * (i + 1) * 40503u);
        for (int r = 0; r < 4; ++r) { h = h * 1664525u + 1013904223u; a[i][r] = (int)(h & seedv); h = h * 1664525u + 1013904223u; b[i][r] = (int)(h & seedv); }
    }
    v4i c = {0x4B400000, 0x4B400000, 0x4B400000, 0x4B400000};
    v4i d[8];
    float acc[8][4];
    for (int t = 0; t < 8; ++t) for (int r = 0; r < 4; ++r) { acc[t][r] = 0.f; d[t][r] = 0; }
    float s = 1.0f + (float)(lane & 7) * 0.001f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            d[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t & 3], b[(t >> 2) + (t & 1)], c, 0, 0, 0);
            if constexpr (FMAS > 0) {
                const int tp = (t + 5) & 7;
#pragma unroll
                for (int r = 0; r < FMAS; ++r) acc[tp][r] = __builtin_fmaf(__int_as_float(d[tp][r]), s, acc[tp][r]);
            }
        }
    }
    int x = 0; float y = 0.f;
    for (int t = 0; t < 8; ++t) for (int r = 0; r < 4; ++r) { x ^= d[t][r]; y += acc[t][r]; }
    out[lane] = x; outf[lane] = y;
}

template <int FMAS>
double run(uint32_t seedv, int iters) {
    const int blocks = 256 * 8;
    int* o; float* of;
    (void)hipMalloc(&o, blocks * 256 * 4); (void)hipMalloc(&of, blocks * 256 * 4);
    hipLaunchKernelGGL(k<FMAS>, dim3(blocks), dim3(256), 0, 0, 10, seedv, o, of);
    (void)hipDeviceSynchronize();
    hipEvent_t e0, e1; (void)hipEventCreate(&e0); (void)hipEventCreate(&e1);
    (void)hipEventRecord(e0);
    for (int rep = 0; rep < 5; ++rep) hipLaunchKernelGGL(k<FMAS>, dim3(blocks), dim3(256), 0, 0, iters, seedv, o, of);
    (void)hipEventRecord(e1); (void)hipEventSynchronize(e1);
    float ms; (void)hipEventElapsedTime(&ms, e0, e1);
    const double ops = 5.0 * blocks * 4.0 /*waves*/ * iters * 8 * 16 * 16 * 64 * 2;
    (void)hipFree(o); (void)hipFree(of);
    return ops / (ms * 1e-3) / 1e12;
}

int main() {
    const int iters = 20000;
    printf("zero data, 0 fma:   %.0f TOPS\n", run<0>(0u, iters));
    printf("random data, 0 fma: %.0f TOPS\n", run<0>(0xffffffffu, iters));
    printf("random small (|v|<16), 0 fma: %.0f TOPS\n", run<0>(0x0f0f0f0fu, iters));
    printf("zero data, 4 fma:   %.0f TOPS\n", run<4>(0u, iters));
    printf("random data, 4 fma: %.0f TOPS\n", run<4>(0xffffffffu, iters));
    printf("random data, 2 fma: %.0f TOPS\n", run<2>(0xffffffffu, iters));
    return 0;
}
