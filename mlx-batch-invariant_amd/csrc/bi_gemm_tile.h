// bi_gemm_tile.h — the one tile body shared by the dense and the quantized
// matmul kernels, and the B-operand sources that feed it.
//
// Canonical reduction order for out[m, n] (follows kernels/matmul.py:1-38 of
// mlx-batch-invariant: fixed K groups, hardware MMA with fp32 accumulate,
// left fold of group partials):
//
//   total = 0
//   for g in 0 .. ceil(K/256)-1:               # fixed 256-wide K groups
//       acc = 0
//       for s in 0 .. 7:                       # 8 MFMA steps per group
//           acc = MFMA_16x16x32(A[m, k(g,s,q,e)], B[k(g,s,q,e), n], acc)
//       total = total + acc                    # plain fp32 add
//   out[m, n] = round_to_T(total)
//
// with the k-slot map  k(g, s, q, e) = 256 g + 64 q + 8 s + e,  where q in
// [0,4) is the lane quarter and e in [0,8) the element of the lane's 8-wide
// fragment. k >= K contributes exact zeros on both operands, and every group
// always runs all 8 steps. The MFMA instruction (v_mfma_f32_16x16x32_bf16 or
// _f16; a chain of eight v_mfma_f32_16x16x4_f32 for fp32) is the same for
// every tile shape. Tile height, tile width, the number of waves and whether
// group partials are folded in registers or by bi_fold_groups are launch
// choices only: an output element always sees exactly the sequence above.
//
// Lane roles for the 16x16x32 MFMA (wave64): lane = 16 q + r. For the A
// operand r is the row, for B the column; both hold the 8 k of quarter q.
// Result register i of lane l is element (row 4 (l/16) + i, column l % 16).
#pragma once

#include "bi_common.h"

namespace bi {

// ---------------------------------------------------------------------------
// Dense B: element b[k, n] at bt[n * ldb + k]; a lane's 64 k of a group are
// contiguous, loaded as 8 fragments.
// ---------------------------------------------------------------------------
template <typename T>
struct DenseB {
  typedef typename Frag<T>::type F;
  struct Raw {
    F f[kSteps];
  };
  const T* bt;
  int64_t ldb;
  int N, K;

  __device__ __forceinline__ void load(Raw& raw, int n, int g, int q) const {
    const int kq = g * kGroupK + 64 * q;
    const bool col_ok = n < N;
    const T* p = bt + (int64_t)(col_ok ? n : 0) * ldb + kq;
#pragma unroll
    for (int s = 0; s < kSteps; ++s)
      raw.f[s] = (col_ok && kq + 8 * s < K) ? frag_load(p + 8 * s) : frag_zero<F>();
  }
  __device__ __forceinline__ F frag(const Raw& raw, int s) const { return raw.f[s]; }
};

// ---------------------------------------------------------------------------
// MLX affine quantized B (kernels/quantized.py:1-22, :44-67 of the reference):
// codes packed low-to-high in uint32 (32/BITS per word), one scale and bias
// per GS consecutive k of a row. Dequantised value for the MFMA:
//     T( fmaf(float(code), float(scale), float(bias)) )      (one RNE rounding)
// and exact zero for k >= K. A lane's 64 k of a group are 64*BITS/32
// consecutive words of row n, fetched as 16-byte loads.
// ---------------------------------------------------------------------------
template <typename T, int BITS, int GS>
struct QuantB {
  typedef typename Frag<T>::type F;
  static constexpr int kWordsPerLane = 64 * BITS / 32;  // 8 (4-bit) or 16 (8-bit)
  static constexpr int kScalesPerLane = GS >= 64 ? 1 : 64 / GS;
  struct Raw {
    uint32_t w[kWordsPerLane];
    float scale[kScalesPerLane];
    float bias[kScalesPerLane];
    int kq;  // first k of this lane's 64-k block
  };
  const uint32_t* w;
  const T* scales;
  const T* biases;
  int N, K;
  int64_t words_per_row, groups_per_row;

  __device__ __forceinline__ void load(Raw& raw, int n, int g, int q) const {
    const int kq = g * kGroupK + 64 * q;
    raw.kq = kq;
    const bool col_ok = n < N;
    const int64_t nn = col_ok ? n : 0;
    const uint32_t* wp = w + nn * words_per_row + (int64_t)kq * BITS / 32;
    // Each 16-byte piece covers 128/BITS consecutive k; K % 32 == 0 makes a
    // piece entirely inside or entirely outside the row.
    constexpr int kPieces = kWordsPerLane / 4;
    constexpr int kPerPiece = 4 * 32 / BITS;
#pragma unroll
    for (int p = 0; p < kPieces; ++p) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (col_ok && kq + p * kPerPiece < K) v = *reinterpret_cast<const u32x4*>(wp + 4 * p);
#pragma unroll
      for (int i = 0; i < 4; ++i) raw.w[4 * p + i] = v[i];
    }
#pragma unroll
    for (int i = 0; i < kScalesPerLane; ++i) {
      const int kk = kq + i * GS;
      const bool ok = col_ok && kk < K;
      const int64_t si = nn * groups_per_row + kk / GS;
      raw.scale[i] = ok ? to_f32(scales[si]) : 0.0f;
      raw.bias[i] = ok ? to_f32(biases[si]) : 0.0f;
    }
  }

  __device__ __forceinline__ F frag(const Raw& raw, int s) const {
    const int si = (GS >= 64) ? 0 : (8 * s) / GS;
    const float sc = raw.scale[si];
    const float bs = raw.bias[si];
    const bool valid = raw.kq + 8 * s < K;
    float d[8];
    if constexpr (BITS == 4) {
      const uint32_t word = raw.w[s];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float c = (float)((word >> (4 * e)) & 0xFu);
        d[e] = __builtin_fmaf(c, sc, bs);
      }
    } else {
      const uint32_t w0 = raw.w[2 * s], w1 = raw.w[2 * s + 1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        d[e] = __builtin_fmaf((float)((w0 >> (8 * e)) & 0xFFu), sc, bs);
        d[4 + e] = __builtin_fmaf((float)((w1 >> (8 * e)) & 0xFFu), sc, bs);
      }
    }
    if constexpr (sizeof(T) == 2) {
      typedef T vec8 __attribute__((ext_vector_type(8)));
      vec8 r;
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = valid ? to_store<T>(d[e]) : (T)0.0f;
      return __builtin_bit_cast(F, r);
    } else {
      f32x8 r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        r.lo[e] = valid ? d[e] : 0.0f;
        r.hi[e] = valid ? d[4 + e] : 0.0f;
      }
      return r;
    }
  }
};

// A fragments straight from global memory: row m, group g, quarter q, step s.
template <typename T>
__device__ __forceinline__ typename Frag<T>::type load_a_frag(const T* a, int64_t lda, int m,
                                                             int M, int K, int g, int q,
                                                             int s) {
  typedef typename Frag<T>::type F;
  const int k0 = g * kGroupK + 64 * q + 8 * s;
  if (m < M && k0 < K) return frag_load(a + (int64_t)m * lda + k0);
  return frag_zero<F>();
}

}  // namespace bi
