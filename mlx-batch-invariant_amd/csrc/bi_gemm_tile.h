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
// Every global load below is issued unconditionally from an in-bounds address,
// so the compiler can put all of a group's loads in flight at once instead of
// branching around each one. Rows of A past M and columns of B past N are
// clamped to the last valid row/column rather than masked: an MFMA output
// element depends only on its own row and column, and the results of those
// padding rows/columns are never stored. Only k past K, in a last group cut
// short, is masked to exact zero on both operands (the FULL = false path).
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

  // n must already be clamped into [0, N). FULL: the whole group lies inside K.
  template <bool FULL>
  __device__ __forceinline__ void load(Raw& raw, int n, int g, int q) const {
    const T* p = bt + (int64_t)n * ldb + g * kGroupK + 8 * q;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      if constexpr (FULL) {
        raw.f[s] = frag_load(p + 32 * s);
      } else {
        const bool ok = g * kGroupK + 32 * s + 8 * q < K;
        const F v = frag_load(ok ? p + 32 * s : bt);
        raw.f[s] = ok ? v : frag_zero<F>();
      }
    }
  }
  template <bool FULL>
  __device__ __forceinline__ F frag(const Raw& raw, int s, int /*kg*/) const { return raw.f[s]; }
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
    T scale[kGroupsPerK];  // kept in storage type: converted where used, so
    T bias[kGroupsPerK];   // issuing the loads never waits for them
  };
  const uint32_t* w;
  const T* scales;
  const T* biases;
  int N, K;
  int64_t words_per_row, groups_per_row;

  // n must already be clamped into [0, N). FULL: the whole group lies inside K
  // (then its kGroupsPerK scales are contiguous and, with K % 256 == 0, aligned).
  template <bool FULL>
  __device__ __forceinline__ void load(Raw& raw, int n, int g, int q) const {
    const int kg = g * kGroupK;
    const uint32_t* wp = w + (int64_t)n * words_per_row + (int64_t)(kg + 8 * q) * BITS / 32;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      // word offset of step s: 32 s codes further along the row
      const bool ok = FULL || kg + 32 * s < K;             // K % 32 == 0: whole step in or out
      const uint32_t* p = ok ? wp + s * (32 * BITS / 32) : w;
      if constexpr (BITS == 4) {
        raw.w[s][0] = *p;
      } else {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        raw.w[s][0] = v.x;
        raw.w[s][1] = v.y;
      }
    }
    const int64_t s0 = (int64_t)n * groups_per_row + kg / GS;
#pragma unroll
    for (int i = 0; i < kGroupsPerK; ++i) {
      const bool ok = FULL || kg + i * GS < K;
      raw.scale[i] = scales[ok ? s0 + i : 0];
      raw.bias[i] = biases[ok ? s0 + i : 0];
    }
  }

  template <bool FULL>
  __device__ __forceinline__ F frag(const Raw& raw, int s, int kg) const {
    const int gi = (32 * s) / GS;
    const float sc = to_f32(raw.scale[gi]);
    const float bs = to_f32(raw.bias[gi]);
    float d[8];
    if constexpr (BITS == 4) {
      // Split the word's nibbles into two registers of four bytes each; the
      // empty asm hides the masks from the optimizer so each code converts
      // with one v_cvt_f32_ubyteN.
      uint32_t lo = raw.w[s][0] & 0x0F0F0F0Fu;
      uint32_t hi = (raw.w[s][0] >> 4) & 0x0F0F0F0Fu;
      asm volatile("" : "+v"(lo), "+v"(hi));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        d[2 * j] = __builtin_fmaf((float)((lo >> (8 * j)) & 0xFFu), sc, bs);
        d[2 * j + 1] = __builtin_fmaf((float)((hi >> (8 * j)) & 0xFFu), sc, bs);
      }
    } else {
      const uint32_t w0 = raw.w[s][0], w1 = raw.w[s][1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        d[e] = __builtin_fmaf((float)((w0 >> (8 * e)) & 0xFFu), sc, bs);
        d[4 + e] = __builtin_fmaf((float)((w1 >> (8 * e)) & 0xFFu), sc, bs);
      }
    }
    F f;
    if constexpr (sizeof(T) == 2) {
      typedef T vec8 __attribute__((ext_vector_type(8)));
      vec8 r;
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = to_store<T>(d[e]);
      f = __builtin_bit_cast(F, r);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f.lo[e] = d[e];
        f.hi[e] = d[4 + e];
      }
    }
    if constexpr (FULL) {
      return f;
    } else {
      return kg + 32 * s < K ? f : frag_zero<F>();
    }
  }
};

// A fragment straight from global memory: row m (already clamped into
// [0, M)), group g, quarter q, step s. FULL: the group lies inside K.
template <typename T, bool FULL>
__device__ __forceinline__ typename Frag<T>::type load_a_frag(const T* a, int64_t lda, int m,
                                                             int K, int g, int q, int s) {
  typedef typename Frag<T>::type F;
  const int k0 = g * kGroupK + 32 * s + 8 * q;
  if constexpr (FULL) {
    return frag_load(a + (int64_t)m * lda + k0);
  } else {
    const bool ok = k0 < K;
    const F v = frag_load(a + (ok ? (int64_t)m * lda + k0 : 0));
    return ok ? v : frag_zero<F>();
  }
}

}  // namespace bi
