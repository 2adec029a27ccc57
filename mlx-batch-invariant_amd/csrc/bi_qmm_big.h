// bi_qmm_big.h — the large-M launch of the affine-quantized matmul: B is
// dequantized once into a bf16/fp16 workspace, A copied beside it, and the
// dense large-M tile (bi_gemm_big.h) runs on the pair.
//
// The quantized op's k-slot map ("blocked": slot (s, q, e) of a 256-k group
// holds k = 64 q + 8 s + e) differs from the dense tile's ("natural": k' =
// 32 s + 8 q + e) only by a permutation of 8-element chunks within each group:
// chunk c' = 4 s + q of the natural order is chunk c = 8 q + s of the blocked
// one. Writing both operands with that permutation applied makes the dense
// tile put exactly the products a_k * w_k of the quantized order into every
// MFMA slot, so every output bit equals the other quantized launches'. The
// dequantized value is the same T(fmaf(code, scale, bias)) (one rounding).
//
// Workspace: B' [N][K] then A' [M][K], element type T (2-byte types only).
#pragma once

#include "bi_gemm_big.h"

namespace bi {

// Chunk c' (0..31) of a group in natural order -> chunk of the blocked order.
__device__ __forceinline__ int blocked_chunk(int cn) { return 8 * (cn % 4) + cn / 4; }

// One thread per 8-element chunk of B': row n, group g, natural chunk cn.
template <typename T, int BITS, int GS>
__global__ __launch_bounds__(256) void qmm_dequant_rows(const uint32_t* __restrict__ w,
                                                        const T* __restrict__ scales,
                                                        const T* __restrict__ biases,
                                                        T* __restrict__ bq, int N, int K) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int chunks_per_row = K / 8;
  if (idx >= (int64_t)N * chunks_per_row) return;
  const int n = (int)(idx / chunks_per_row);
  const int cr = (int)(idx % chunks_per_row);
  const int g = cr / 32, cn = cr % 32;
  const int k0 = g * kGroupK + 8 * blocked_chunk(cn);          // first k of the chunk's values
  const int gpr = K / GS;
  const float sc = to_f32(scales[(int64_t)n * gpr + k0 / GS]);  // 8 k never straddle a group
  const float bs = to_f32(biases[(int64_t)n * gpr + k0 / GS]);
  const uint32_t* wr = w + (int64_t)n * ((int64_t)K * BITS / 32) + (int64_t)k0 * BITS / 32;
  typedef T vec8 __attribute__((ext_vector_type(8)));
  vec8 out;
  if constexpr (BITS == 4) {
    const uint32_t word = wr[0];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      out[e] = to_store<T>(__builtin_fmaf((float)((word >> (4 * e)) & 0xFu), sc, bs));
  } else {
    const uint32_t w0 = wr[0], w1 = wr[1];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      out[e] = to_store<T>(__builtin_fmaf((float)((w0 >> (8 * e)) & 0xFFu), sc, bs));
      out[4 + e] = to_store<T>(__builtin_fmaf((float)((w1 >> (8 * e)) & 0xFFu), sc, bs));
    }
  }
  *reinterpret_cast<vec8*>(bq + (int64_t)n * K + 8 * cr) = out;
}

// One thread per 8-element chunk of A': A'[m][256 g + 8 cn] = A[m][256 g + 8 blocked_chunk(cn)].
template <typename T>
__global__ __launch_bounds__(256) void qmm_permute_a(const T* __restrict__ a, int64_t lda,
                                                     T* __restrict__ ap, int M, int K) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int chunks_per_row = K / 8;
  if (idx >= (int64_t)M * chunks_per_row) return;
  const int m = (int)(idx / chunks_per_row);
  const int cr = (int)(idx % chunks_per_row);
  const int g = cr / 32, cn = cr % 32;
  *reinterpret_cast<u32x4*>(ap + (int64_t)m * K + 8 * cr) =
      *reinterpret_cast<const u32x4*>(a + (int64_t)m * lda + g * kGroupK + 8 * blocked_chunk(cn));
}

// The shapes that take this launch (qmm_use_big) are defined with the dense
// policy in bi_matmul_impl.h.

inline size_t qmm_big_ws_bytes(int64_t M, int64_t N, int64_t K) { return (size_t)((N + M) * K) * 2; }

}  // namespace bi
