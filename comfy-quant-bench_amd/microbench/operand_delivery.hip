// Microbenchmark: operand delivery alone. The W8A8 wide GEMM's per-K-group A and B tiles (256 rows
// x 64 bytes of int8 each, 32 KB per group) go into an LDS ring with one barrier per group and no
// math, over the north-star product's 768 tiles (M = 4096, N = 12288, K = 3072: three rounds of 48
// groups on 256 compute units). DMA: buffer_load ... lds, S - 1 groups ahead for an S-stage ring of
// 32 KB stages (the kernel's path, S = 4); registers: buffer_load_dwordx4 into registers two groups
// ahead, then ds_write_b128 into a 4-stage ring. The barriers are bare s_barrier and the one LDS
// read per group is inline asm, so the compiler adds no wait for the DMA in flight (a fence or a
// plain LDS read would make it wait for every pending DMA). The time is the floor that delivering
// the operands puts under the GEMM.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cstdio>
#include <vector>
typedef uint32_t u4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float lds_read(const uint8_t* smem, int off) {
    float v;
    const int addr = static_cast<int>(reinterpret_cast<uintptr_t>(smem)) + off;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
    return v;
}

// S stages of 32 KB filled by DMA, S - 1 groups ahead
template <int S>
__global__ void __launch_bounds__(512) dma_kernel(const uint8_t* A, const uint8_t* B, int K, int tiles_n, float* out) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[S * 32768];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
    const auto ra = rsrc(A + (int64_t)tm * 256 * K, (int64_t)256 * K);
    const auto rb = rsrc(B + (int64_t)tn * 256 * K, (int64_t)256 * K);
    const int G = K / 64;
    float acc = 0.f;
    int off[2];
    for (int h = 0; h < 2; ++h) off[h] = (32 * wave + 16 * h + (lane >> 2)) * K + (lane & 3) * 16;
    auto dma = [&](int g) {
        if (g >= G) return;
        const int st = g % S;
        for (int h = 0; h < 2; ++h) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (__attribute__((address_space(3))) void*)(smem + st * 32768 + (32 * wave + 16 * h) * 64), 16, off[h],
                g * 64, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (__attribute__((address_space(3))) void*)(smem + st * 32768 + 16384 + (32 * wave + 16 * h) * 64), 16,
                off[h], g * 64, 0, 0);
        }
    };
    for (int g = 0; g < S - 1; ++g) dma(g);
    for (int g = 0; g < G; ++g) {
        dma(g + S - 1);
        // group g done: 4 (S - 1) operations issued after it, fewer at the tail
        if (g + S - 1 < G) {
            if constexpr (S == 2) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
            if constexpr (S == 3) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
            if constexpr (S == 4) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
            if constexpr (S == 5) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        acc += lds_read(smem, (g % S) * 32768 + tid * 4);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    }
    out[(int64_t)blockIdx.x * 512 + tid] = acc;
}

// four 32 KB stages filled through registers, two groups ahead
__global__ void __launch_bounds__(512) reg_kernel(const uint8_t* A, const uint8_t* B, int K, int tiles_n, float* out) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[4 * 32768];
    const int tid = threadIdx.x;
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
    const int G = K / 64;
    float acc = 0.f;
    // thread t: row t / 2, 32 bytes (two 16-byte chunks) of A and of B; inline-asm loads with
    // explicit waits (the other register set's four loads stay in flight)
    const int r = tid >> 1, c0 = (tid & 1) * 2;
    const int off = r * K + c0 * 16;
    auto desc = [&](const uint8_t* base) {
        const uint64_t p = reinterpret_cast<uint64_t>(base);
        u4v d;
        d.x = __builtin_amdgcn_readfirstlane((uint32_t)p);
        d.y = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32) & 0xffffu);
        d.z = 256u * K;
        d.w = 0x00020000u;
        return d;
    };
    const u4v da = desc(A + (int64_t)tm * 256 * K), db = desc(B + (int64_t)tn * 256 * K);
    u4v va0[2], va1[2], vb0[2], vb1[2];
    auto ld = [&](int g, u4v (&a)[2], u4v (&b)[2]) {
        const int so = (g < G ? g : G - 1) * 64;
        for (int c = 0; c < 2; ++c) {
            asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(a[c]) : "v"(off + c * 16), "s"(da), "s"(so) : "memory");
            asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(b[c]) : "v"(off + c * 16), "s"(db), "s"(so) : "memory");
        }
    };
    auto st = [&](u4v (&a)[2], u4v (&b)[2], int stg) {
        asm volatile("s_waitcnt vmcnt(4)" : "+v"(a[0]), "+v"(a[1]), "+v"(b[0]), "+v"(b[1]) :: "memory");
        for (int c = 0; c < 2; ++c) {
            *reinterpret_cast<u4v*>(smem + stg * 32768 + r * 64 + (c0 + c) * 16) = a[c];
            *reinterpret_cast<u4v*>(smem + stg * 32768 + 16384 + r * 64 + (c0 + c) * 16) = b[c];
        }
    };
    ld(0, va0, vb0); ld(1, va1, vb1);
    for (int g = 0; g < G; g += 2) {
        st(va0, vb0, g & 3); ld(g + 2, va0, vb0);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        acc += lds_read(smem, (g & 3) * 32768 + tid * 4);
        st(va1, vb1, (g + 1) & 3); ld(g + 3, va1, vb1);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        acc += lds_read(smem, ((g + 1) & 3) * 32768 + tid * 4);
    }
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(va0[0]), "+v"(va0[1]), "+v"(vb0[0]), "+v"(vb0[1]), "+v"(va1[0]), "+v"(va1[1]), "+v"(vb1[0]), "+v"(vb1[1]) :: "memory");
    out[(int64_t)blockIdx.x * 512 + tid] = acc;
}

template <typename F>
static float time_us(F f) {
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    for (int i = 0; i < 200; ++i) f();
    std::vector<float> t;
    for (int r = 0; r < 5; ++r) {
        (void)hipEventRecord(e0);
        for (int i = 0; i < 20; ++i) f();
        (void)hipEventRecord(e1);
        (void)hipEventSynchronize(e1);
        float ms;
        (void)hipEventElapsedTime(&ms, e0, e1);
        t.push_back(ms * 1000.f / 20);
    }
    std::sort(t.begin(), t.end());
    return t[2];
}

int main() {
    const int M = 4096, N = 12288, K = 3072, tiles_n = N / 256, wgs = (M / 256) * tiles_n;
    uint8_t *A, *B;
    float* out;
    (void)hipMalloc(&A, (size_t)M * K);
    (void)hipMalloc(&B, (size_t)N * K);
    (void)hipMemset(A, 1, (size_t)M * K);
    (void)hipMemset(B, 1, (size_t)N * K);
    (void)hipMalloc(&out, (size_t)wgs * 512 * 4);
    const double bytes = (double)wgs * (K / 64) * 32768;
    auto report = [&](const char* what, float us) {
        printf("%-44s %7.1f us  %6.0f GB/s into LDS  %5.1f B/clk/CU at 2.1 GHz\n", what, us, bytes / (us * 1e3),
               bytes / (us * 1e-6) / 256 / 2.1e9);
    };
    report("DMA, 2 stages (1 group ahead)", time_us([&] { hipLaunchKernelGGL(dma_kernel<2>, dim3(wgs), dim3(512), 0, 0, A, B, K, tiles_n, out); }));
    report("DMA, 3 stages (2 groups ahead)", time_us([&] { hipLaunchKernelGGL(dma_kernel<3>, dim3(wgs), dim3(512), 0, 0, A, B, K, tiles_n, out); }));
    report("DMA, 4 stages (3 groups ahead, the GEMM's)", time_us([&] { hipLaunchKernelGGL(dma_kernel<4>, dim3(wgs), dim3(512), 0, 0, A, B, K, tiles_n, out); }));
    report("DMA, 5 stages (4 groups ahead)", time_us([&] { hipLaunchKernelGGL(dma_kernel<5>, dim3(wgs), dim3(512), 0, 0, A, B, K, tiles_n, out); }));
    report("registers + ds_write_b128, 2 groups ahead", time_us([&] { hipLaunchKernelGGL(reg_kernel, dim3(wgs), dim3(512), 0, 0, A, B, K, tiles_n, out); }));
    (void)hipFree(A);
    (void)hipFree(B);
    (void)hipFree(out);
    return 0;
}
