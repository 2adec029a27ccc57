// bi_qmm_f16.hip — the affine-quantized matmul kernels for f16 activations
// (one translation unit per element type so the build compiles them in parallel;
// the 8-bit kernels are in bi_qmm8_f16.hip).
#include "bi_matmul_impl.h"

namespace bi {

int qmm_f16(int bits, int gs, const void* x, int64_t ldx, const uint32_t* w, const void* scales,
            const void* biases, void* out, int M, int N, int K, void* ws, hipStream_t st) {
  if (bits == 8) return qmm8_f16(gs, x, ldx, w, scales, biases, out, M, N, K, ws, st);
  if (bits != 4) return bi_host::fail(BI_E_UNSUPPORTED, "bi_quantized_matmul: bits=%d group_size=%d", bits, gs);
  return dispatch_quant_bits<f16, 4>(gs, x, ldx, w, scales, biases, out, M, N, K, ws, st);
}

int qmm_packed_f16(int bits, int gs, const void* x, int64_t ldx, const uint32_t* w, const void* scales,
                   const void* biases, const void* packed, void* out, int M, int N, int K, void* ws,
                   hipStream_t st) {
  if (bits == 8) return qmm8_packed_f16(gs, x, ldx, w, scales, biases, packed, out, M, N, K, ws, st);
  return run_quant_packed<f16, 4>(gs, x, ldx, w, scales, biases, packed, out, M, N, K, ws, st);
}

}  // namespace bi
