// Microbenchmark: LDS read throughput of ds_read_b128 for several per-lane address patterns, 8
// waves per CU. Pattern 1 is the fragment read of the W4A8 GEMM (lane l reads 16-byte chunk
// (l / 16) ^ ((row >> 1) & 3) of 64-byte row l % 16).
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

template <int PAT>
__device__ __forceinline__ int addr_of(int lane, int blk) {
    const int row = lane & 15, q = lane >> 4;
    int a;
    if constexpr (PAT == 0) a = lane * 16;                                   // linear
    else if constexpr (PAT == 1) a = row * 64 + ((q ^ ((row >> 1) & 3)) << 4); // current swizzle
    else if constexpr (PAT == 2) a = row * 64 + (q << 4);                     // unswizzled 64 B rows
    else if constexpr (PAT == 3) a = row * 80 + (q << 4);                     // padded 80 B rows
    else if constexpr (PAT == 4) a = row * 64 + ((q ^ (row & 3)) << 4);       // swizzle by row & 3
    else if constexpr (PAT == 5) a = row * 64 + ((q ^ ((row >> 2) & 3)) << 4); // swizzle by (row >> 2) & 3
    else a = row * 64 + ((q ^ (row & 3) ^ ((row >> 2) & 3)) << 4);
    return a + blk * (PAT == 3 ? 1280 : 1024);
}

template <int PAT>
__global__ void __launch_bounds__(512) k(int iters, uint32_t* out) {
    __shared__ __attribute__((aligned(16))) uint8_t s[65536];
    for (int i = threadIdx.x; i < 65536 / 4; i += 512) reinterpret_cast<uint32_t*>(s)[i] = i * 2654435761u;
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int base[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) base[b] = addr_of<PAT>(lane, b) + wave * 2048 % 32768;
    u4 acc = {0, 0, 0, 0};
    for (int it = 0; it < iters; ++it) {
        u4 v[8];
#pragma unroll
        for (int b = 0; b < 8; ++b) v[b] = *reinterpret_cast<const u4*>(s + ((base[b] + it * 16384) & 65535));
#pragma unroll
        for (int b = 0; b < 8; ++b) acc ^= v[b];
    }
    out[blockIdx.x * 512 + threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

template <int PAT>
void run(const char* name) {
    const int blocks = 256 * 4, iters = 2000;
    uint32_t* o;
    (void)hipMalloc(&o, blocks * 512 * 4);
    hipLaunchKernelGGL((k<PAT>), dim3(blocks), dim3(512), 0, 0, 10, o);
    (void)hipDeviceSynchronize();
    hipEvent_t e0, e1; (void)hipEventCreate(&e0); (void)hipEventCreate(&e1);
    (void)hipEventRecord(e0);
    hipLaunchKernelGGL((k<PAT>), dim3(blocks), dim3(512), 0, 0, iters, o);
    (void)hipEventRecord(e1); (void)hipEventSynchronize(e1);
    float ms; (void)hipEventElapsedTime(&ms, e0, e1);
    const double bytes = (double)blocks * 8 * iters * 8 * 1024;   // waves * iters * 8 reads * 1 KB
    printf("%-28s %.0f GB/s total, %.1f B/clk/CU at 2.4 GHz\n", name, bytes / ms / 1e6, bytes / (ms * 1e-3) / 256 / 2.4e9);
    (void)hipFree(o);
}

int main() {
    run<0>("linear");
    run<1>("swizzle (row>>1)&3");
    run<2>("unswizzled 64B rows");
    run<3>("padded 80B rows");
    run<4>("swizzle row&3");
    run<5>("swizzle (row>>2)&3");
    run<6>("swizzle row&3 ^ (row>>2)&3");
    return 0;
}
