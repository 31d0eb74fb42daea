// Rotate + per-token quantize of plain fp32 activations: the bf16 kernels' arithmetic on fp32
// values loaded as they are (a translation unit of its own so the instantiation sets compile in
// parallel).
#include "mq_rotquant_kernel.h"

namespace mq {

int launch_rotquant_f32(const float* x, int64_t M, int64_t K, int64_t ldx, int hblock, int bits,
                        int packed, void* q, int64_t ldq, float* scale, hipStream_t stream) {
    return launch_rotquant_impl<0, 2>(reinterpret_cast<const uint16_t*>(x), M, K, ldx, hblock, bits, packed, q, ldq,
                                      scale, stream);
}

}  // namespace mq
