// Microbenchmark: operand delivery alone. The W8A8 wide GEMM's per-K-group A and B tiles (256 rows
// x 64 bytes of int8 each, 32 KB per group) go into a 4-stage LDS ring with one barrier per group
// and no math, over the north-star product's 768 tiles (M = 4096, N = 12288, K = 3072: three rounds
// of 48 groups on 256 compute units). MODE 0: buffer_load ... lds, three groups ahead (the
// kernel's DMA); MODE 1: buffer_load_dwordx4 into registers two groups ahead, then ds_write_b128.
// The time is the floor that delivering the operands puts under the GEMM.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <vector>
#include <algorithm>
typedef uint32_t u4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

template <int MODE>
__global__ void __launch_bounds__(512) move_kernel(const uint8_t* A, const uint8_t* B, int M, int N, int K, int tiles_n,
                                                   float* out) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[4 * 32768];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
    const auto ra = rsrc(A + (int64_t)tm * 256 * K, (int64_t)256 * K);
    const auto rb = rsrc(B + (int64_t)tn * 256 * K, (int64_t)256 * K);
    const int G = K / 64;
    float acc = 0.f;
    if constexpr (MODE == 0) {
        int off[2];
        for (int h = 0; h < 2; ++h) {
            const int r = 32 * wave + 16 * h + (lane >> 2);
            off[h] = r * K + (lane & 3) * 16;
        }
        auto dma = [&](int g, int st) {
            if (g >= G) return;
            for (int h = 0; h < 2; ++h) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (__attribute__((address_space(3))) void*)(smem + st * 32768 + (32 * wave + 16 * h) * 64), 16, off[h], g * 64, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (__attribute__((address_space(3))) void*)(smem + st * 32768 + 16384 + (32 * wave + 16 * h) * 64), 16, off[h], g * 64, 0, 0);
            }
        };
        dma(0, 0); dma(1, 1); dma(2, 2);
        for (int g = 0; g < G; ++g) {
            dma(g + 3, (g + 3) & 3);
            // group g's 4 ops done: 12 issued after it (groups g+1..g+3), fewer at the tail
            if (g + 3 < G) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            acc += *reinterpret_cast<const float*>(smem + (g & 3) * 32768 + tid * 4);
            __syncthreads();
        }
    } else {
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
            __syncthreads();
            acc += *reinterpret_cast<const float*>(smem + (g & 3) * 32768 + tid * 4);
            st(va1, vb1, (g + 1) & 3); ld(g + 3, va1, vb1);
            __syncthreads();
            acc += *reinterpret_cast<const float*>(smem + ((g + 1) & 3) * 32768 + tid * 4);
        }
        asm volatile("s_waitcnt vmcnt(0)" : "+v"(va0[0]), "+v"(va0[1]), "+v"(vb0[0]), "+v"(vb0[1]), "+v"(va1[0]), "+v"(va1[1]), "+v"(vb1[0]), "+v"(vb1[1]) :: "memory");
    }
    out[(int64_t)blockIdx.x * 512 + tid] = acc;
}

int main() {
    const int M = 4096, N = 12288, K = 3072;
    uint8_t *A, *B; float* out;
    (void)hipMalloc(&A, (size_t)M * K); (void)hipMalloc(&B, (size_t)N * K);
    (void)hipMemset(A, 1, (size_t)M * K); (void)hipMemset(B, 1, (size_t)N * K);
    const int tiles_m = M / 256, tiles_n = N / 256, wgs = tiles_m * tiles_n;
    (void)hipMalloc(&out, (size_t)wgs * 512 * 4);
    hipEvent_t e0, e1; (void)hipEventCreate(&e0); (void)hipEventCreate(&e1);
    for (int mode = 0; mode < 2; ++mode) {
        auto f = [&]() {
            if (mode == 0) hipLaunchKernelGGL(move_kernel<0>, dim3(wgs), dim3(512), 0, 0, A, B, M, N, K, tiles_n, out);
            else hipLaunchKernelGGL(move_kernel<1>, dim3(wgs), dim3(512), 0, 0, A, B, M, N, K, tiles_n, out);
        };
        for (int i = 0; i < 200; ++i) f();
        std::vector<float> t;
        for (int r = 0; r < 5; ++r) {
            (void)hipEventRecord(e0);
            for (int i = 0; i < 20; ++i) f();
            (void)hipEventRecord(e1); (void)hipEventSynchronize(e1);
            float ms; (void)hipEventElapsedTime(&ms, e0, e1); t.push_back(ms * 1000.f / 20);
        }
        std::sort(t.begin(), t.end());
        const double bytes = (double)wgs * (K / 64) * 32768;
        printf("mode %s: median %.1f us (%.0f GB/s into LDS, %.1f B/clk/CU at 2.1 GHz)\n", mode ? "vgpr+ds_write" : "buffer_load lds",
               t[2], bytes / (t[2] * 1e3), bytes / (t[2] * 1e-6) / 256 / 2.1e9);
    }
    return 0;
}
