// SwiGLU prologue fused into rotate + per-token quantize (tools/ck_swiglu/swiglu_quant.cu:23-97),
// bf16 inputs: the input row holds gate | up, the activation silu(gate) * up is formed in fp32
// while loading, rounded once to bf16, then rotated and quantized exactly like a plain input
// (kernel templates in mq_rotquant_kernel.h).
#include "mq_rotquant_kernel.h"

namespace mq {

int launch_swiglu_rotquant_bf16(const uint16_t* h, int64_t M, int64_t K, int64_t ldh, int hblock, int bits,
                                int packed, void* q, int64_t ldq, float* scale, hipStream_t stream) {
    return launch_rotquant_impl<1, 0>(h, M, K, ldh, hblock, bits, packed, q, ldq, scale, stream);
}

}  // namespace mq
