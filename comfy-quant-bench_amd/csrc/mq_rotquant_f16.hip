// Rotate + per-token quantize of plain fp16 activations: the bf16 kernels' arithmetic with the
// fp16 values converted exactly to fp32 on load (a translation unit of its own so the two
// instantiation sets compile in parallel).
#include "mq_rotquant_kernel.h"

namespace mq {

int launch_rotquant_f16(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int hblock, int bits,
                        int packed, void* q, int64_t ldq, float* scale, hipStream_t stream) {
    return launch_rotquant_impl<0, 1>(x, M, K, ldx, hblock, bits, packed, q, ldq, scale, stream);
}

}  // namespace mq
