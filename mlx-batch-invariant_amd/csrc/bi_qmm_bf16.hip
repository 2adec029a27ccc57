// bi_qmm_bf16.hip — the affine-quantized matmul kernels for bf16 activations
// (one translation unit per element type so the build compiles them in parallel).
#include "bi_matmul_impl.h"

namespace bi {

int qmm_bf16(int bits, int gs, const void* x, int64_t ldx, const uint32_t* w, const void* scales,
             const void* biases, void* out, int M, int N, int K, void* ws, hipStream_t st) {
  return dispatch_quant<bf16>(bits, gs, x, ldx, w, scales, biases, out, M, N, K, ws, st);
}

}  // namespace bi
