// bi_gemm_tile.h — the one arithmetic shared by every matmul tile shape, and
// the B-operand sources that feed it.
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
// with the k-slot map  k(g, s, q, e) = 256 g + 32 s + 8 q + e,  where q in
// [0,4) is the lane quarter and e in [0,8) the element of the lane's 8-wide
// fragment: step s of group g covers k in [256 g + 32 s, 256 g + 32 s + 32).
// k >= K contributes exact zeros on both operands, and every group always
// runs all 8 steps. The MFMA instruction (v_mfma_f32_16x16x32_bf16 or _f16; a
// chain of eight v_mfma_f32_16x16x4_f32 for fp32) is the same for every tile
// shape. Tile height and width, waves per workgroup, staging through LDS or
// straight into registers, and whether group partials are folded in registers
// or by fold_groups are launch choices only: an output element always sees
// exactly the sequence above.
//
// Lane roles for the 16x16x32 MFMA (wave64): lane = 16 q + r. For the A
// operand r is the row, for B the column; both hold the 8 k of quarter q.
// Result register i of lane l is element (row 4 (l/16) + i, column l % 16).
//
// Every global load below is issued unconditionally from a clamped, in-bounds
// address and masked afterwards with a select, so the compiler can put all of
// a group's loads in flight at once instead of branching around each one.
#pragma once

#include "bi_common.h"

namespace bi {

// ---------------------------------------------------------------------------
// Dense B: element b[k, n] at bt[n * ldb + k].
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
    const bool col_ok = n < N;
    const T* p = bt + (int64_t)(col_ok ? n : 0) * ldb;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const int k0 = g * kGroupK + 32 * s + 8 * q;
      const bool ok = col_ok && k0 < K;
      const F v = frag_load(p + (ok ? k0 : 0));
      raw.f[s] = ok ? v : frag_zero<F>();
    }
  }
  __device__ __forceinline__ F frag(const Raw& raw, int s) const { return raw.f[s]; }
};

// ---------------------------------------------------------------------------
// MLX affine quantized B (kernels/quantized.py:1-22, :44-67 of the reference):
// codes packed low-to-high in uint32 (32/BITS per word), one scale and bias
// per GS consecutive k of a row. Dequantised value fed to the MFMA:
//     T( fmaf(float(code), float(scale), float(bias)) )      (one RNE rounding)
// and exact zero for k >= K. Step s of a lane needs the 8 codes of k in
// [256 g + 32 s + 8 q, +8): one word (4-bit) or two (8-bit). The 256/GS
// scales and biases of the group are the same for all four quarters and are
// fetched as one small vector per lane.
// ---------------------------------------------------------------------------
template <typename T, int BITS, int GS>
struct QuantB {
  typedef typename Frag<T>::type F;
  static constexpr int kWordsPerStep = BITS / 4;          // 1 (4-bit) or 2 (8-bit)
  static constexpr int kGroupsPerK = kGroupK / GS;         // scales per 256-k group
  struct Raw {
    uint32_t w[kSteps][kWordsPerStep];
    float scale[kGroupsPerK];
    float bias[kGroupsPerK];
    int kg;  // first k of the group
  };
  const uint32_t* w;
  const T* scales;
  const T* biases;
  int N, K;
  int64_t words_per_row, groups_per_row;

  __device__ __forceinline__ void load(Raw& raw, int n, int g, int q) const {
    const int kg = g * kGroupK;
    raw.kg = kg;
    const bool col_ok = n < N;
    const int64_t nn = col_ok ? n : 0;
    const uint32_t* wp = w + nn * words_per_row;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const int k0 = kg + 32 * s + 8 * q;                  // K % 32 == 0: whole step in or out
      const bool ok = col_ok && kg + 32 * s < K;
      const int64_t wi = ok ? (int64_t)k0 * BITS / 32 : 0;
      if constexpr (BITS == 4) {
        raw.w[s][0] = wp[wi];
      } else {
        const uint2 v = *reinterpret_cast<const uint2*>(wp + wi);
        raw.w[s][0] = v.x;
        raw.w[s][1] = v.y;
      }
    }
    // Scales/biases of the group: up to kGroupsPerK consecutive entries of row
    // n (fewer in a last group cut short by K; those read entry 0 and are
    // never used, since their steps are masked).
#pragma unroll
    for (int i = 0; i < kGroupsPerK; ++i) {
      const bool ok = col_ok && kg + i * GS < K;
      const int64_t si = ok ? nn * groups_per_row + kg / GS + i : 0;
      raw.scale[i] = to_f32(scales[si]);
      raw.bias[i] = to_f32(biases[si]);
    }
  }

  __device__ __forceinline__ F frag(const Raw& raw, int s) const {
    const int gi = (32 * s) / GS;
    const float sc = raw.scale[gi];
    const float bs = raw.bias[gi];
    const bool valid = raw.kg + 32 * s < K;
    float d[8];
    if constexpr (BITS == 4) {
      const uint32_t word = raw.w[s][0];
#pragma unroll
      for (int e = 0; e < 8; ++e) d[e] = __builtin_fmaf((float)((word >> (4 * e)) & 0xFu), sc, bs);
    } else {
      const uint32_t w0 = raw.w[s][0], w1 = raw.w[s][1];
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
      for (int e = 0; e < 8; ++e) r[e] = to_store<T>(d[e]);
      const F f = __builtin_bit_cast(F, r);
      return valid ? f : frag_zero<F>();
    } else {
      f32x8 r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        r.lo[e] = d[e];
        r.hi[e] = d[4 + e];
      }
      return valid ? r : frag_zero<f32x8>();
    }
  }
};

// A fragment straight from global memory: row m, group g, quarter q, step s.
template <typename T>
__device__ __forceinline__ typename Frag<T>::type load_a_frag(const T* a, int64_t lda, int m,
                                                             int M, int K, int g, int q,
                                                             int s) {
  typedef typename Frag<T>::type F;
  const int k0 = g * kGroupK + 32 * s + 8 * q;
  const bool ok = m < M && k0 < K;
  const F v = frag_load(a + (ok ? (int64_t)m * lda + k0 : 0));
  return ok ? v : frag_zero<F>();
}

}  // namespace bi
