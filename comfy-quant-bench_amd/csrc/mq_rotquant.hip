// Rotate + per-token quantize of plain bf16 activations (the kernel templates and their
// arithmetic are described in mq_rotquant_kernel.h).
#include "mq_rotquant_kernel.h"

namespace mq {

int launch_rotquant_bf16(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int hblock, int bits,
                         int packed, void* q, int64_t ldq, float* scale, hipStream_t stream) {
    return launch_rotquant_impl<0, 0>(x, M, K, ldx, hblock, bits, packed, q, ldq, scale, stream);
}

}  // namespace mq
