// Read-bandwidth floor for a ~30.6 MB single launch (the M = 1 GEMV's weight bytes): each thread
// reads B bytes (16-byte loads) and the workgroup writes one word. Ten buffer copies (306 MB, past
// the 256 MB MALL) are cycled; 200 launches timed with events.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
template <int NV>   // uint4 loads per thread
__global__ void __launch_bounds__(256) rd(const uint4* __restrict__ p, uint32_t* out) {
    const int64_t base = (int64_t)blockIdx.x * 256 * NV;
    uint4 v[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = p[base + (int64_t)i * 256 + threadIdx.x];
    uint32_t x = 0;
#pragma unroll
    for (int i = 0; i < NV; ++i) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if (x == 0x12345678u) out[blockIdx.x] = x;
}
template <int NV>
void run(const char* name, uint4* const* bufs, int64_t bytes, uint32_t* out) {
    const int blocks = (int)(bytes / (256 * 16 * NV));
    for (int i = 0; i < 20; ++i) hipLaunchKernelGGL(rd<NV>, dim3(blocks), dim3(256), 0, 0, bufs[i % 10], out);
    (void)hipDeviceSynchronize();
    hipEvent_t e0, e1; (void)hipEventCreate(&e0); (void)hipEventCreate(&e1);
    (void)hipEventRecord(e0);
    for (int i = 0; i < 200; ++i) hipLaunchKernelGGL(rd<NV>, dim3(blocks), dim3(256), 0, 0, bufs[i % 10], out);
    (void)hipEventRecord(e1); (void)hipEventSynchronize(e1);
    float ms; (void)hipEventElapsedTime(&ms, e0, e1);
    const double us = ms * 1000.0 / 200;
    printf("%-28s blocks %6d: %.2f us per launch, %.0f GB/s\n", name, blocks, us, blocks * 256.0 * 16 * NV / (us * 1e3));
}
int main() {
    const int64_t bytes = 30600192;   // multiple of 256 * 16 * 6 * ... (rounded per variant)
    uint4* bufs[10];
    uint32_t* out;
    for (int i = 0; i < 10; ++i) { (void)hipMalloc(&bufs[i], bytes + (1 << 20)); (void)hipMemset(bufs[i], i, bytes + (1 << 20)); }
    (void)hipMalloc(&out, 1 << 20);
    for (int r = 0; r < 2; ++r) {
        run<1>("16 B/thread", bufs, bytes, out);
        run<2>("32 B/thread", bufs, bytes, out);
        run<4>("64 B/thread", bufs, bytes, out);
        run<6>("96 B/thread (GEMV-like)", bufs, bytes, out);
        run<8>("128 B/thread", bufs, bytes, out);
        run<16>("256 B/thread", bufs, bytes, out);
    }
    return 0;
}
