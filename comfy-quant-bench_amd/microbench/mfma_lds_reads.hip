// Probe: MFMA throughput with interleaved ds_read_b128 (results consumed by later MFMAs through a
// ring of fragment registers and explicit lgkmcnt waits), 2 waves per SIMD, 512 threads per block,
// 64 KB of LDS per block (1 block per CU at most 2 with 160 KB; we force 1 via 96 KB).
// RPM: ds_read_b128 per 4 MFMAs (0, 1, 2, 4). DST: 0 fragments in VGPRs, 1 in AGPRs.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
typedef int v4i __attribute__((ext_vector_type(4)));

template <int RPM, int DST>
__global__ void __launch_bounds__(512) k(int iters, int* out) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[96 * 1024];
    const int tid = threadIdx.x, lane = tid & 63;
    for (int i = tid; i < 96 * 1024 / 4; i += 512) reinterpret_cast<int*>(smem)[i] = i * 2654435761u;
    __syncthreads();
    // lane reads 16 bytes at a conflict-free swizzled position inside a 16 KB window per wave
    const int wave = tid >> 6;
    const int fr = lane & 15, fk = ((lane >> 4) ^ ((fr >> 1) & 3)) << 4;
    int base = (wave & 3) * 16384 + fr * 64 + fk;
    asm volatile("" : "+v"(base));
    v4i acc[8];
    for (int t = 0; t < 8; ++t) for (int r = 0; r < 4; ++r) acc[t][r] = 0;
    for (int t = 0; t < 8; ++t) asm volatile("" : "+a"(acc[t]));
    v4i fa = {tid, tid * 3, tid * 5, tid * 7}, f[8];
    for (int q = 0; q < 8; ++q) f[q] = v4i{q, q + 1, q + 2, q + 3};
    if constexpr (DST) for (int q = 0; q < 8; ++q) asm volatile("" : "+a"(f[q]));
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int t = 0; t < 32; ++t) {
            // issue the reads of this step (ring slot (t + 4) & 7 .. for RPM reads per 4 MFMAs)
            if constexpr (RPM > 0) {
                constexpr int every = RPM >= 4 ? 1 : 4 / RPM;     // one read every `every` MFMAs
                constexpr int per = RPM >= 4 ? RPM / 4 : 1;
                if (t % every == 0) {
#pragma unroll
                    for (int p = 0; p < per; ++p) {
                        const int slot = (t / every * per + p + 4) & 7;
                        if constexpr (DST)
                            asm volatile("ds_read_b128 %0, %1 offset:%2" : "=a"(f[slot]) : "v"(base), "i"(((t * 7 + p * 3) & 15) * 1024) : "memory");
                        else
                            asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(f[slot]) : "v"(base), "i"(((t * 7 + p * 3) & 15) * 1024) : "memory");
                    }
                    asm volatile("s_waitcnt lgkmcnt(%0)" :: "n"(3 * per) : "memory");
                }
            }
            const int slot = (t / 4) & 7;
            if constexpr (DST)
                asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(acc[t & 7]) : "v"(fa), "a"(f[slot]));
            else
                asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(acc[t & 7]) : "v"(fa), "v"(f[slot]));
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    int x = 0;
    for (int t = 0; t < 8; ++t) for (int r = 0; r < 4; ++r) x ^= acc[t][r];
    for (int q = 0; q < 8; ++q) x ^= f[q][0];
    out[blockIdx.x * 512 + tid] = x;
}

template <typename F>
void run(const char* name, F kern) {
    const int iters = 2000, blocks = 512;
    int* o;
    (void)hipMalloc(&o, blocks * 512 * 4);
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(512), 0, 0, 10, o);
    (void)hipDeviceSynchronize();
    hipEvent_t e0, e1; (void)hipEventCreate(&e0); (void)hipEventCreate(&e1);
    float best = 1e30f;
    for (int rep = 0; rep < 3; ++rep) {
        (void)hipEventRecord(e0);
        hipLaunchKernelGGL(kern, dim3(blocks), dim3(512), 0, 0, iters, o);
        (void)hipEventRecord(e1); (void)hipEventSynchronize(e1);
        float ms; (void)hipEventElapsedTime(&ms, e0, e1);
        if (ms < best) best = ms;
    }
    const double mfma_per_simd = (double)iters * 32 * (blocks * 8.0 / 1024.0);
    printf("%-44s %.1f cycles per MFMA at 2.4 GHz\n", name, best * 1e6 / mfma_per_simd * 2.4);
    (void)hipFree(o);
}

int main() {
    for (int rep = 0; rep < 2; ++rep) {
        run("no reads", k<0, 0>);
        run("1 ds_read_b128 per 4 MFMA, vgpr dst", k<1, 0>);
        run("2 per 4 MFMA (GEMM ratio 12/32 ~ 1.5), vgpr", k<2, 0>);
        run("4 per 4 MFMA, vgpr", k<4, 0>);
        run("1 per 4 MFMA, agpr dst", k<1, 1>);
        run("2 per 4 MFMA, agpr dst", k<2, 1>);
        run("4 per 4 MFMA, agpr dst", k<4, 1>);
    }
    return 0;
}
