// bi_qmm8_f16.hip — the 8-bit affine-quantized matmul kernels for f16
// activations (the 4-bit ones are in bi_qmm_f16.hip; the build compiles the
// two with different scheduler options).
#include "bi_matmul_impl.h"

namespace bi {

int qmm8_f16(int gs, const void* x, int64_t ldx, const uint32_t* w, const void* scales, const void* biases,
             void* out, int M, int N, int K, void* ws, hipStream_t st) {
  return dispatch_quant_bits<f16, 8>(gs, x, ldx, w, scales, biases, out, M, N, K, ws, st);
}

int qmm8_packed_f16(int gs, const void* x, int64_t ldx, const uint32_t* w, const void* scales,
                    const void* biases, const void* packed, void* out, int M, int N, int K, void* ws,
                    hipStream_t st) {
  return run_quant_packed<f16, 8>(gs, x, ldx, w, scales, biases, packed, out, M, N, K, ws, st);
}

}  // namespace bi
