// SwiGLU prologue with the eager path's two roundings, bf16 inputs: silu(gate) is rounded to bf16,
// then silu * up to bf16 again (ComfyUI's silu(gate).mul_(up) in bf16,
// patches/comfyui_swiglu_triton_env.patch:16-20, which comfy-kitchen applies outside its fused
// quantizer's domain, patches/comfy_kitchen_swiglu_w4a4_fused.patch:60-64), then rotated and
// quantized like a plain input (kernel templates in mq_rotquant_kernel.h).
#include "mq_rotquant_kernel.h"

namespace mq {

int launch_swiglu_eager_rotquant_bf16(const uint16_t* h, int64_t M, int64_t K, int64_t ldh, int hblock, int bits,
                                      int packed, void* q, int64_t ldq, float* scale, hipStream_t stream) {
    return launch_rotquant_impl<2, 0>(h, M, K, ldh, hblock, bits, packed, q, ldq, scale, stream);
}

}  // namespace mq
