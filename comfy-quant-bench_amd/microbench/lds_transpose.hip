// Microbenchmark: the 16 x 16 register transpose through LDS of the rotate+quantize kernel, for a
// range of paddings. Each group of 16 lanes sharing (lane & 3) swaps lane index (lane >> 2) and
// register index: lane L writes its 16 values as ds_write_b32 at G*(L & 3) + (L >> 2) + S*j and
// reads them back as four ds_read_b128 at G*(L & 3) + S*(L >> 2) + 4q (floats; S and G multiples
// of 4, G >= 15*S + 16 keeps the four groups of a wave apart). The loop is the transpose alone
// (plus one VALU op per value), 4 waves per workgroup, so its time is the LDS pattern's cost.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <vector>

__global__ void __launch_bounds__(256) transpose_loop(int iters, int S, int G, float* out) {
    extern __shared__ float lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float* base = lds + wave * 4 * G + (lane & 3) * G;
    float* w = base + (lane >> 2);
    const float* r = base + (lane >> 2) * S;
    float v[16];
    for (int j = 0; j < 16; ++j) v[j] = (float)(lane * 16 + j);
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 16; ++j) w[j * S] = v[j];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 t = *reinterpret_cast<const float4*>(r + 4 * q);
            v[4 * q] = t.x + 1.0f;
            v[4 * q + 1] = t.y + 1.0f;
            v[4 * q + 2] = t.z + 1.0f;
            v[4 * q + 3] = t.w + 1.0f;
        }
    }
    float y = 0.f;
    for (int j = 0; j < 16; ++j) y += v[j];
    out[blockIdx.x * 256 + threadIdx.x] = y;
}

int main() {
    const int blocks = 4096, iters = 400;
    float* out;
    (void)hipMalloc(&out, (size_t)blocks * 256 * 4);
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    struct R { int S, G; float us; };
    std::vector<R> res;
    for (int S : {16, 20, 24, 28, 36, 52}) {
        const int gmin = 15 * S + 16;
        for (int G = gmin; G < gmin + 64; G += 4) {
            const size_t lds = (size_t)16 * G * 4;      // 4 waves x 4 groups x G floats
            if (lds > 64 * 1024) continue;
            hipLaunchKernelGGL(transpose_loop, dim3(blocks), dim3(256), lds, 0, 4, S, G, out);
            (void)hipDeviceSynchronize();
            float best = 1e30f;
            for (int rep = 0; rep < 3; ++rep) {
                (void)hipEventRecord(e0);
                hipLaunchKernelGGL(transpose_loop, dim3(blocks), dim3(256), lds, 0, iters, S, G, out);
                (void)hipEventRecord(e1);
                (void)hipEventSynchronize(e1);
                float ms;
                (void)hipEventElapsedTime(&ms, e0, e1);
                best = ms < best ? ms : best;
            }
            res.push_back({S, G, best * 1000.f});
        }
    }
    float lo = 1e30f;
    for (auto& r : res) lo = r.us < lo ? r.us : lo;
    for (auto& r : res)
        printf("S=%2d G=%4d (G mod 64 = %2d, S mod 64 = %2d): %8.1f us  x%.2f of the fastest\n", r.S, r.G, r.G % 64,
               r.S % 64, r.us, r.us / lo);
    (void)hipFree(out);
    return 0;
}
