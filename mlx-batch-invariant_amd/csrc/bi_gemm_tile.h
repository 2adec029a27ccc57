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
// with a k-slot map k(g, s, q, e) fixed per op, where q in [0,4) is the lane
// quarter and e in [0,8) the element of the lane's 8-wide fragment:
//   dense matmul      k = 256 g + 32 s + 8 q + e   (step s covers 32 consecutive k)
//   quantized matmul  k = 256 g + 64 q + 8 s + e   (quarter q owns 64 consecutive k)
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
  // Per-lane pointer for whole-group loads (row n clamped, quarter q): the
  // group offset is then one wave-uniform add.
  struct Lane {
    const T* b;
  };
  __device__ __forceinline__ Lane lane(int n, int q) const { return Lane{bt + (int64_t)n * ldb + 8 * q}; }
  __device__ __forceinline__ void load_full(Raw& raw, const Lane& l, int g) const {
    const T* p = l.b + g * kGroupK;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) raw.f[s] = frag_load(p + 32 * s);
  }
  // Dense operands carry no per-group metadata.
  static constexpr bool kMeta = false;
  template <bool FULL, bool FAST>
  __device__ __forceinline__ F frag(const Raw& raw, int s, int /*kq*/) const { return raw.f[s]; }
  __device__ __forceinline__ bool huge_scale(const Raw&) const { return false; }

  // Dense op k-slot map: k(g, s, q, e) = 256 g + 32 s + 8 q + e.
  static __device__ __forceinline__ int kbase(int g, int q) { return g * kGroupK + 8 * q; }
  static __device__ __forceinline__ int a_k(int g, int q, int s) { return g * kGroupK + 32 * s + 8 * q; }
  // LDS staging of steps {2p, 2p+1}: LDS chunk kc (columns 8 kc .. 8 kc + 7,
  // read by quarter kc % 4 in step 2p + kc / 4) holds these 8 consecutive k.
  static __device__ __forceinline__ int stage_k(int g, int p, int kc) { return g * kGroupK + 64 * p + 8 * kc; }
};

// A dense 2-byte B repacked once for the decode GEMV: the same elements, so the
// same values reach the MFMA. For 16-row tile t and group g, MFMA lane
// l = r + 16 q's step-s fragment (row 16 t + r, k 256 g + 32 s + 8 q, 8
// elements: the dense k-slot map) is the l-th 16-byte piece of the s-th 1 KB
// run of the (tile, group)'s 8 KB block at (t G + g) 8 KB. A wave's loads then
// read whole 1 KB runs (in the row-major layout each instruction touches 16
// rows, 64 bytes each). tiles = ceil(N / 16), rows past N repeat row N - 1;
// G = ceil(K / 256), elements past K are zero (K % 8 == 0).
template <typename T>
struct DensePacked : DenseB<T> {
  typedef typename DenseB<T>::Raw Raw;
  typedef typename Frag<T>::type F;
  static_assert(sizeof(T) == 2, "DensePacked: 2-byte element types only");
  static constexpr int kBlock = kSteps * 1024;                  // bytes per (tile, group)
  const char* p;
  int G;
  static constexpr int64_t bytes(int64_t N, int64_t K) {
    return (N + 15) / 16 * ((K + kGroupK - 1) / kGroupK) * kBlock;
  }
  struct Lane {
    const char* c;   // the lane's piece of group 0, step 0
  };
  // n must already be clamped into [0, N).
  __device__ __forceinline__ Lane lane(int n, int q) const {
    return Lane{p + (int64_t)(n / 16) * G * kBlock + (n % 16 + 16 * q) * 16};
  }
  __device__ __forceinline__ void load_full(Raw& raw, const Lane& l, int g) const {
    const char* b = l.c + (int64_t)g * kBlock;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) raw.f[s] = __builtin_bit_cast(F, *reinterpret_cast<const u32x4*>(b + 1024 * s));
  }
};

// ---------------------------------------------------------------------------
// MLX affine quantized B (kernels/quantized.py:1-22, :44-67 of the reference):
// codes packed low-to-high in uint32 (32/BITS per word), one scale and bias
// per GS consecutive k of a row. Dequantised value fed to the MFMA:
//     T( fmaf(float(code), float(scale), float(bias)) )      (one RNE rounding)
// and exact zero for k >= K.
//
// The quantized op uses its own k-slot map, the "blocked" map
//     k(g, s, q, e) = 256 g + 64 q + 8 s + e,
// so lane quarter q owns the 64 consecutive codes [256 g + 64 q, +64) of its
// row: two (4-bit) or four (8-bit) 16-byte loads of consecutive words, and for
// group size 64 exactly one scale and bias. (Weight rows are then read as long
// contiguous runs per lane; the dense op's map would read them 16 bytes per
// four lanes, which measured 2.6x slower on the loads alone.) Every launch
// shape of the quantized op uses this map, so the op is consistent with itself
// across batch sizes, as the reference requires of each op
// (kernels/matmul.py:11-12).
// ---------------------------------------------------------------------------
template <typename T, int BITS, int GS>
struct QuantB {
  typedef typename Frag<T>::type F;
  static constexpr int kBits = BITS, kGS = GS;
  static constexpr int kWords = 64 * BITS / 32;            // words per lane per group: 8 or 16
  static constexpr int kScales = GS >= 64 ? 1 : 64 / GS;   // scales per lane per group
  struct Raw {
    u32x4 w[kWords / 4];
    T scale[kScales];  // kept in storage type: converted where used, so
    T bias[kScales];   // issuing the loads never waits for them
  };
  const uint32_t* w;
  const T* scales;
  const T* biases;
  int N, K;
  int64_t words_per_row, groups_per_row;

  static __device__ __forceinline__ int kbase(int g, int q) { return g * kGroupK + 64 * q; }

  // n must already be clamped into [0, N). FULL: the whole group lies inside K.
  template <bool FULL>
  __device__ __forceinline__ void load(Raw& raw, int n, int g, int q) const {
    const int kq = kbase(g, q);
    const uint32_t* wp = w + (int64_t)n * words_per_row + (int64_t)kq * BITS / 32;
    constexpr int kPerPiece = 4 * 32 / BITS;                 // codes per 16-byte piece
#pragma unroll
    for (int p = 0; p < kWords / 4; ++p) {
      const bool ok = FULL || kq + p * kPerPiece < K;        // K % 32 == 0: whole piece in or out
      raw.w[p] = *reinterpret_cast<const u32x4*>(ok ? wp + 4 * p : w);
    }
    const int64_t s0 = (int64_t)n * groups_per_row + kq / GS;
#pragma unroll
    for (int i = 0; i < kScales; ++i) {
      const bool ok = FULL || kq + i * GS < K;
      raw.scale[i] = scales[ok ? s0 + i : 0];
      raw.bias[i] = biases[ok ? s0 + i : 0];
    }
  }

  // Per-lane pointers for whole-group loads (row n clamped, quarter q): the
  // group offset is then one wave-uniform add.
  struct Lane {
    const uint32_t* w;
    const T* s;
    const T* b;
  };
  __device__ __forceinline__ Lane lane(int n, int q) const {
    const int64_t s0 = (int64_t)n * groups_per_row + (64 * q) / GS;
    return Lane{w + (int64_t)n * words_per_row + 64 * q * BITS / 32, scales + s0, biases + s0};
  }
  __device__ __forceinline__ void load_codes(Raw& raw, const Lane& l, int g) const {
    const uint32_t* wp = l.w + g * (kGroupK * BITS / 32);
#pragma unroll
    for (int p = 0; p < kWords / 4; ++p) raw.w[p] = *reinterpret_cast<const u32x4*>(wp + 4 * p);
  }
  __device__ __forceinline__ void load_full(Raw& raw, const Lane& l, int g) const {
    load_codes(raw, l, g);
    const int so = g * (kGroupK / GS);
#pragma unroll
    for (int i = 0; i < kScales; ++i) {
      raw.scale[i] = l.s[so + i];
      raw.bias[i] = l.b[so + i];
    }
  }
  // Per-group metadata (scales, biases) can be staged in LDS for a 16-row
  // tile: scales of rows n0 .. n0 + 15 are the contiguous block
  // scales[n0 * gpr, (n0 + 16) * gpr), likewise biases. LDS layout:
  // [16][gpr] scales, then [16][gpr] biases.
  static constexpr bool kMeta = true;
  // Element i (of the 32 * gpr staged) lives at this global address; indices
  // past the arrays' end read element 0 (those rows are never used).
  __device__ __forceinline__ const T* meta_src(int n0, int64_t i) const {
    const int64_t gpr = groups_per_row, half = 16 * gpr;
    const bool second = i >= half;
    const int64_t e = (int64_t)n0 * gpr + (second ? i - half : i);
    const T* base = second ? biases : scales;
    return e + 8 <= (int64_t)N * gpr ? base + e : base;
  }
  // Scale and bias of group g for lane quarter q of tile row rt from LDS.
  __device__ __forceinline__ void meta_from_lds(Raw& raw, const T* ms, int rt, int g, int q) const {
    const int gpr = (int)groups_per_row;
    const int so = rt * gpr + (g * kGroupK + 64 * q) / GS;
#pragma unroll
    for (int i = 0; i < kScales; ++i) {
      raw.scale[i] = ms[so + i];
      raw.bias[i] = ms[16 * gpr + so + i];
    }
  }

  // A scale this large would overflow scale * 512 in the fp8 conversion path;
  // such a group takes the integer conversion (chosen wave-uniformly).
  __device__ __forceinline__ bool huge_scale(const Raw& raw) const {
    bool big = false;
#pragma unroll
    for (int i = 0; i < kScales; ++i) big |= !(fabsf(to_f32(raw.scale[i])) < 0x1p100f);
    return big;
  }

  // FAST (4-bit only): A byte holding a code c <= 15 read as an OCP FP8 E4M3
  // value is exactly c * 2^-9 (denormal for c < 8, exponent field 1 for
  // c >= 8), so one v_cvt_pk_f32_fp8 converts two codes and
  //     fmaf(c * 2^-9, scale * 2^9, bias) == fmaf(c, scale, bias)
  // bit for bit: both scalings are exact and the product is the same real
  // number. Otherwise each code converts with one v_cvt_f32_ubyteN.
  template <bool FULL, bool FAST>
  __device__ __forceinline__ F frag(const Raw& raw, int s, int kq) const {
    const int si = (GS >= 64) ? 0 : (8 * s) / GS;
    const float sc = to_f32(raw.scale[si]);
    const float bs = to_f32(raw.bias[si]);
    float d[8];
    if constexpr (BITS == 4) {
      // Split the word's nibbles into two registers of four bytes each (even
      // codes, odd codes).
      const uint32_t word = raw.w[s / 4][s % 4];
      uint32_t lo = word & 0x0F0F0F0Fu;
      uint32_t hi = (word >> 4) & 0x0F0F0F0Fu;
      if constexpr (FAST) {
        const float sc_u = sc * 512.0f;
        const auto c02 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
        const auto c46 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
        const auto c13 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
        const auto c57 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
        d[0] = __builtin_fmaf(c02[0], sc_u, bs);
        d[1] = __builtin_fmaf(c13[0], sc_u, bs);
        d[2] = __builtin_fmaf(c02[1], sc_u, bs);
        d[3] = __builtin_fmaf(c13[1], sc_u, bs);
        d[4] = __builtin_fmaf(c46[0], sc_u, bs);
        d[5] = __builtin_fmaf(c57[0], sc_u, bs);
        d[6] = __builtin_fmaf(c46[1], sc_u, bs);
        d[7] = __builtin_fmaf(c57[1], sc_u, bs);
      } else {
        // the empty asm hides the masks so each code is one v_cvt_f32_ubyteN
        asm volatile("" : "+v"(lo), "+v"(hi));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          d[2 * j] = __builtin_fmaf((float)((lo >> (8 * j)) & 0xFFu), sc, bs);
          d[2 * j + 1] = __builtin_fmaf((float)((hi >> (8 * j)) & 0xFFu), sc, bs);
        }
      }
    } else {
      const uint32_t w0 = raw.w[s / 2][2 * (s % 2)], w1 = raw.w[s / 2][2 * (s % 2) + 1];
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
      return kq + 8 * s < K ? f : frag_zero<F>();
    }
  }

  // The A operand must follow the same map: element k of lane quarter q, step s.
  static __device__ __forceinline__ int a_k(int g, int q, int s) { return g * kGroupK + 64 * q + 8 * s; }
  // LDS staging of steps {2p, 2p+1}: LDS chunk kc (read by quarter kc % 4 in
  // step 2p + kc / 4) holds these 8 consecutive k.
  static __device__ __forceinline__ int stage_k(int g, int p, int kc) {
    return g * kGroupK + 64 * (kc % 4) + 16 * p + 8 * (kc / 4);
  }
};

// ---------------------------------------------------------------------------
// An affine quantized B repacked once for the decode GEMV: the same codes,
// scales and biases as QuantB<T, BITS, GS>, so the same values reach the MFMA.
// For 16-row tile t and group g, MFMA lane l = r + 16 q holds row 16 t + r, k
// [256 g + 64 q, +64) (the blocked map): its kWords words are the l-th 16-byte
// pieces of kPieces consecutive 1 KB runs, followed by a run of the block's
// (scale, bias) pairs, 4 bytes each, every pair once: for groups of 32 and 64
// lane l's kScales pairs at 4 kScales l; for groups of 128 (two lanes of a row
// share a pair) row r's pair of half h at 4 (16 h + r). A wave's code loads then read whole 1 KB runs
// (in the MLX layout each instruction touches 16 weight rows 2 KB apart), and
// each lane's scales and biases arrive with its codes instead of being staged
// per tile. Block (t, g) starts at byte (t G + g) kBlock; tiles = ceil(N / 16),
// rows past N repeat row N - 1. 2-byte T only (a pair is two 16-bit values).
// ---------------------------------------------------------------------------
template <typename T, int BITS, int GS>
struct QuantPacked : QuantB<T, BITS, GS> {
  typedef QuantB<T, BITS, GS> Base;
  typedef typename Base::Raw Raw;
  static constexpr int kScales = Base::kScales;
  static constexpr int kPieces = Base::kWords / 4;               // 16-byte pieces per lane and group
  static constexpr int kMetaBytes = 16 * (kGroupK / GS) * 4;     // the block's pairs, each once
  static constexpr int kBlock = kPieces * 1024 + kMetaBytes;     // bytes per (tile, group)
  // Byte offset of lane (r, q)'s first pair within the metadata run.
  static __host__ __device__ constexpr int meta_off(int r, int q) {
    return GS >= 128 ? 4 * (16 * (q * 64 / GS) + r) : 4 * kScales * (r + 16 * q);
  }
  static_assert(sizeof(T) == 2, "QuantPacked: 2-byte element types only");
  static_assert(kScales == 1 || kScales == 2, "QuantPacked: one or two scales per lane");
  const char* p;
  int G;
  static constexpr int64_t bytes(int64_t N, int64_t K) { return (N + 15) / 16 * (K / kGroupK) * kBlock; }
  struct Lane {
    const char* c;   // the lane's first code piece of group 0
    const char* m;   // the lane's (scale, bias) pairs of group 0
  };
  // n must already be clamped into [0, N).
  __device__ __forceinline__ Lane lane(int n, int q) const {
    const char* b = p + (int64_t)(n / 16) * G * kBlock;
    const int l = n % 16 + 16 * q;
    return Lane{b + 16 * l, b + kPieces * 1024 + meta_off(n % 16, q)};
  }
  __device__ __forceinline__ void load_full(Raw& raw, const Lane& l, int g) const {
    const int64_t o = (int64_t)g * kBlock;
#pragma unroll
    for (int i = 0; i < kPieces; ++i) raw.w[i] = *reinterpret_cast<const u32x4*>(l.c + o + 1024 * i);
    uint32_t m[kScales];
    if constexpr (kScales == 1) {
      m[0] = *reinterpret_cast<const uint32_t*>(l.m + o);
    } else {
      const u32x2 v = *reinterpret_cast<const u32x2*>(l.m + o);
      m[0] = v[0];
      m[1] = v[1];
    }
#pragma unroll
    for (int i = 0; i < kScales; ++i) {
      raw.scale[i] = __builtin_bit_cast(T, (uint16_t)(m[i] & 0xffffu));
      raw.bias[i] = __builtin_bit_cast(T, (uint16_t)(m[i] >> 16));
    }
  }
};

// A fragment straight from global memory: row m (already clamped into
// [0, M)), first k of the fragment k0 (from the op's k-slot map). FULL: the
// group lies inside K.
template <typename T, bool FULL>
__device__ __forceinline__ typename Frag<T>::type load_a_frag(const T* a, int64_t lda, int m,
                                                             int K, int k0) {
  typedef typename Frag<T>::type F;
  if constexpr (FULL) {
    return frag_load(a + (int64_t)m * lda + k0);
  } else {
    const bool ok = k0 < K;
    const F v = frag_load(a + (ok ? (int64_t)m * lda + k0 : 0));
    return ok ? v : frag_zero<F>();
  }
}

}  // namespace bi
