// SwiGLU prologue with the eager path's two roundings for fp16 inputs: silu(gate) (from the
// generated table of correctly rounded fp32 results for all 65536 fp16 bit patterns, compiled into
// this translation unit) is rounded to fp16, then silu * up to fp16 again, as the eager
// silu(gate).mul_(up) in fp16 does (patches/comfyui_swiglu_triton_env.patch:16-20).
#include "mq_rotquant_kernel.h"
#include "mq_silu_f16_table.h"

namespace mq {
namespace {

template <>
struct SiluF16Table<1> {
    __device__ static const uint32_t* get() { return kSiluF16Table; }
};

}  // namespace

int launch_swiglu_eager_rotquant_f16(const uint16_t* h, int64_t M, int64_t K, int64_t ldh, int hblock, int bits,
                                     int packed, void* q, int64_t ldq, float* scale, hipStream_t stream) {
    return launch_rotquant_impl<2, 1>(h, M, K, ldh, hblock, bits, packed, q, ldq, scale, stream);
}

}  // namespace mq
