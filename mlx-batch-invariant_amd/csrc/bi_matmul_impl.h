// bi_matmul_impl.h — matmul kernels, launch policy and the quantized
// dispatch, shared by the translation units that instantiate them
// (bi_matmul.hip: dense; bi_qmm_<dtype>.hip: one quantized element type each,
// so the build compiles them in parallel).
//
// Kernels (all run the arithmetic of bi_gemm_tile.h):
//   gemm_direct  M <= 32. Each wave owns 16 columns x MT 16-row tiles; its A
//                and B fragments go straight from global memory into
//                registers (quantized B is dequantized in registers). With
//                more than one K group it runs one workgroup per (column
//                tile, group) and writes the raw fp32 group partial.
//   fold_groups  out = T(((0 + part[0]) + part[1]) + ...), the split fold.
//   gemm_big     dense 2-byte types, M > 128, K % 64 == 0, enough 256 x 128
//                tiles to fill the chip: 8 waves, operands copied straight
//                into swizzled LDS rows through buffer resources, copies and
//                fragment reads interleaved with the MFMAs (bi_gemm_big.h).
//   gemm_tall    dense 2-byte types, 16 < M <= 256 where gemm_big is not
//                used: one weight stream through a ring-capped LDS ring, 1-3
//                workgroups per CU (bi_gemm_tall.h).
//   gemv_stream, gemv_wg, gemm_mid, gemm_mid2
//                the quantized decode and mid-M launches (bi_gemv_stream.h,
//                bi_gemm_mid.h) and the workgroup-fold GEMV.
//   gemm_lds     other M > 32. A BM x BN tile per 256-thread workgroup, K
//                staged 64 at a time through double-buffered LDS (quantized B
//                is dequantized while it is staged), all groups folded in
//                registers.
// Reference launchers: kernels/matmul.py:279-314 (launch_tiled: split for
// M <= SPLIT_M_MAX and more than one group, fused otherwise), the combine
// kernel kernels/matmul.py:226-234, and kernels/quantized.py:106-125.
#pragma once

#include <type_traits>

#include <algorithm>

#include "bi_gemm_big.h"
#include "bi_gemv_stream.h"
#include "bi_gemm_mid.h"
#include "bi_gemm_tall.h"
#include "bi_qmm_big.h"
#include "bi_gemm_tile.h"

namespace bi {

constexpr int kSplitMMax = 32;
constexpr int kStreamMMax = 16;   // rows of x the streaming GEMV takes (8-bit codes: 8 with A staged in LDS)
// gemv_wg with A staged in LDS: at most kGemvAChunks / W 16-byte chunks of A
// per thread (M * K <= kGemvAChunks * 64 * 8).
constexpr int kGemvAChunks = 32;
// gemv_wg META: at most kGemvMetaChunks / W 16-byte chunks of scales and
// biases per thread (4 * K / group_size <= kGemvMetaChunks * 64).
constexpr int kGemvMetaChunks = 16;

// ---------------------------------------------------------------------------
// gemm_direct: MT m-tiles x 1 n-tile per wave, WAVES waves per workgroup
// along n. SPLIT: one group per workgroup (blockIdx.z), raw partial out.
// ---------------------------------------------------------------------------
// The eight MFMA steps of one group from acc = 0, B fragments dequantized (or
// taken) on the fly. The fast/slow B conversion is chosen once per group for
// the whole wave, so the step loop has no divergent branch.
template <typename T, class BSrc, int MT, bool FULL>
__device__ __forceinline__ void mma_group(const BSrc& bsrc, const typename BSrc::Raw& braw,
                                          const typename Frag<T>::type (&af)[MT][kSteps], int g,
                                          int q, f32x4 (&acc)[MT]) {
  typedef typename Frag<T>::type F;
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (!__any(bsrc.huge_scale(braw))) {
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const F bf = bsrc.template frag<FULL, true>(braw, s, BSrc::kbase(g, q));
#pragma unroll
      for (int i = 0; i < MT; ++i) acc[i] = mfma_step(af[i][s], bf, acc[i]);
    }
  } else {
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const F bf = bsrc.template frag<FULL, false>(braw, s, BSrc::kbase(g, q));
#pragma unroll
      for (int i = 0; i < MT; ++i) acc[i] = mfma_step(af[i][s], bf, acc[i]);
    }
  }
}

template <typename T, class BSrc, int MT, bool FULL>
__device__ __forceinline__ void direct_group(const T* a, int64_t lda, const BSrc& bsrc, int n,
                                             const int (&rows)[MT], int K, int g, int q,
                                             f32x4 (&acc)[MT]) {
  typedef typename Frag<T>::type F;
  // Load phase: every fragment of the group is requested before any is used.
  typename BSrc::Raw braw;
  bsrc.template load<FULL>(braw, n, g, q);
  F af[MT][kSteps];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int s = 0; s < kSteps; ++s) af[i][s] = load_a_frag<T, FULL>(a, lda, rows[i], K, BSrc::a_k(g, q, s));
  // Compute phase.
  mma_group<T, BSrc, MT, FULL>(bsrc, braw, af, g, q, acc);
}

template <typename T, class BSrc, int MT, int WAVES, bool SPLIT>
__global__ __launch_bounds__(kWave* WAVES) void gemm_direct(const T* __restrict__ a, int64_t lda,
                                                            BSrc bsrc, T* __restrict__ out,
                                                            float* __restrict__ part, int M,
                                                            int N, int K, int G) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int r = lane % 16, q = lane / 16;
  const int n_base = (blockIdx.x * WAVES + wave) * 16;
  const int m_base = blockIdx.y * 16 * MT;
  if (n_base >= N) return;  // wave-uniform; the kernel has no block barrier
  const int n = min(n_base + r, N - 1);          // clamped: padding columns are not stored
  int rows[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) rows[i] = min(m_base + 16 * i + r, M - 1);
  const int g0 = SPLIT ? (int)blockIdx.z : 0;
  const int g1 = SPLIT ? g0 + 1 : G;

  f32x4 total[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) total[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int g = g0; g < g1; ++g) {
    f32x4 acc[MT];
    if ((g + 1) * kGroupK <= K) direct_group<T, BSrc, MT, true>(a, lda, bsrc, n, rows, K, g, q, acc);
    else direct_group<T, BSrc, MT, false>(a, lda, bsrc, n, rows, K, g, q, acc);
    if constexpr (SPLIT) {
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = m_base + 16 * i + 4 * q + e;
          if (m < M && n_base + r < N) part[((int64_t)g * M + m) * N + n] = acc[i][e];
        }
    } else {
#pragma unroll
      for (int i = 0; i < MT; ++i) total[i] = total[i] + acc[i];
    }
  }
  if constexpr (!SPLIT) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m_base + 16 * i + 4 * q + e;
        if (m < M && n_base + r < N) out[(int64_t)m * N + n] = to_store<T>(total[i][e]);
      }
  }
}

// ---------------------------------------------------------------------------
// gemv_wg: M <= 32, the decode-shaped launch. One workgroup of W waves per 16
// columns covers every K group: wave w computes groups w, w + W, w + 2W, ...,
// and writes each raw fp32 group partial to LDS; after a barrier the
// workgroup folds the partials in group order, ((0 + p0) + p1) + ..., exactly
// the fold of the other launches. A wave issues the B-operand loads of up to
// NB of its groups before computing any of them (all unconditional, so the
// wait counters only ever wait for the group being computed). With ALDS the
// M rows of A are staged once per workgroup into LDS (while the first weight
// loads are in flight) and A fragments are read from there; with META (a
// quantized B) the tile's scales and biases are staged alongside, so a wave's
// memory instructions per group are just its two 16-byte code loads.
// Dynamic LDS: G * MT * 64 f32x4 partials, then (ALDS) M rows of K + 8
// elements, then (META) 32 * groups_per_row elements of scales and biases.
// ---------------------------------------------------------------------------
template <typename T, class BSrc, int MT, int W, int NB, bool ALDS, bool META = false, int AC = 0>
// `a` is deliberately not __restrict__: a restrict-const operand's loads count
// as invariant, and the compiler then re-issues A loads after the weight
// loads instead of keeping them in registers, turning the LDS staging wait
// into a wait for every weight load.
__global__ __launch_bounds__(kWave* W) void gemv_wg(const T* a, int64_t lda, BSrc bsrc,
                                                    T* __restrict__ out, int M, int N, int K,
                                                    int G) {
  static_assert(!META || (ALDS && BSrc::kMeta), "META needs ALDS and a quantized B");
  typedef typename Frag<T>::type F;
  extern __shared__ __attribute__((aligned(16))) f32x4 smem[];
  f32x4* part = smem;                                        // [G][MT][64]
  T* As = reinterpret_cast<T*>(smem + (size_t)G * MT * kWave);  // [M][K + 8]
  const int lds_row = K + 8;
  T* Ms = As + (size_t)M * lds_row;                          // META: [2][16][gpr]
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int r = lane % 16, q = lane / 16;
  const int n_base = blockIdx.x * 16;
  const int m_base = blockIdx.y * 16 * MT;
  const int n = min(n_base + r, N - 1);          // clamped: padding columns are not stored
  int rows[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) rows[i] = min(m_base + 16 * i + r, M - 1);

  const int gfull = K / kGroupK;                 // groups lying entirely inside K
  const int nw = gfull > wave ? (gfull - 1 - wave) / W + 1 : 0;   // this wave's full groups
  const int last = wave + (nw - 1) * W;

  // A fragments of group g: from LDS (ALDS) or from global memory.
  auto load_af = [&](F (&af)[MT][kSteps], int g) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int s = 0; s < kSteps; ++s) {
        const int k0 = BSrc::a_k(g, q, s);
        if constexpr (ALDS)
          af[i][s] = *reinterpret_cast<const F*>(As + (size_t)(rows[i] - m_base) * lds_row + k0);
        else
          af[i][s] = load_a_frag<T, true>(a, lda, rows[i], K, k0);
      }
  };
  auto compute = [&](typename BSrc::Raw& braw, int g, f32x4 (&acc)[MT]) {
    if constexpr (META) bsrc.meta_from_lds(braw, Ms, n - n_base, g, q);
    F af[MT][kSteps];
    load_af(af, g);
    mma_group<T, BSrc, MT, true>(bsrc, braw, af, g, q, acc);
  };
  auto load_group = [&](typename BSrc::Raw& braw, const typename BSrc::Lane& bl, int g) {
    if constexpr (META) bsrc.load_codes(braw, bl, g);
    else bsrc.load_full(braw, bl, g);
  };

  typename BSrc::Raw braw[NB];
  const typename BSrc::Lane blane = bsrc.lane(n, q);
  const int lastc = nw > 0 ? last : 0;                 // clamp target (any valid group)
  if constexpr (ALDS) {
    // Issue order: A (and META: scales/biases), then the first NB groups of
    // codes, then the LDS writes (which wait for the first batch only: vmcnt
    // retires in order) and the barrier. K / 8 is a multiple of the thread
    // count and this workgroup's rows of A are exactly AC chunks per thread
    // (both checked on the host), so chunk j of every thread lies in row
    // j * threads / (K / 8): row and column base are wave-uniform, and every
    // load is unconditional (conditional loads make the wait counts
    // conservative).
    static_assert(AC >= 1, "ALDS needs the A chunk count");
    const int kch = K / 8;
    constexpr int kThreads = kWave * W;
    const T* abase = a + (int64_t)m_base * lda;
    F av[AC];
    {
      int row = 0, colb = 0;
#pragma unroll
      for (int j = 0; j < AC; ++j) {
        av[j] = frag_load(abase + (int64_t)row * lda + 8 * (colb + (int)threadIdx.x));
        colb += kThreads;
        if (colb == kch) {
          colb = 0;
          ++row;
        }
      }
    }
    // META: the tile's scales then biases, 32 * gpr elements, in 8-element
    // chunks; chunk c of the 4 * gpr reads element 8 c of its half. Chunks
    // of rows past N (last tile only) read the array's first chunk instead.
    constexpr int kMetaMax = META ? kGemvMetaChunks / W : 1;
    F mv[kMetaMax];
    int nmeta = 0;
    if constexpr (META) {
      const int gpr = (int)bsrc.groups_per_row;
      nmeta = 4 * gpr;
      const int limit = (N - n_base) * gpr;          // valid elements from the tile's first row
      const T* sbase = bsrc.scales + (int64_t)n_base * gpr;
      const T* bbase = bsrc.biases + (int64_t)n_base * gpr;
#pragma unroll
      for (int j = 0; j < kMetaMax; ++j) {
        const int c = (int)threadIdx.x + j * kThreads;
        const bool second = c >= 2 * gpr;
        int e = 8 * (second ? c - 2 * gpr : c);
        e = (e + 8 <= limit) ? e : 0;
        mv[j] = frag_load((second ? bbase : sbase) + e);
      }
    }
    // Keep the loads above ahead of the weight loads in issue order.
    asm volatile("" ::: "memory");
#pragma unroll
    for (int j = 0; j < NB; ++j) load_group(braw[j], blane, min(wave + j * W, lastc));
    {
      int row = 0, colb = 0;
#pragma unroll
      for (int j = 0; j < AC; ++j) {
        *reinterpret_cast<F*>(As + (size_t)row * lds_row + 8 * (colb + threadIdx.x)) = av[j];
        colb += kThreads;
        if (colb == kch) {
          colb = 0;
          ++row;
        }
      }
    }
    if constexpr (META) {
#pragma unroll
      for (int j = 0; j < kMetaMax; ++j) {
        const int c = (int)threadIdx.x + j * kThreads;
        if (c < nmeta) *reinterpret_cast<F*>(Ms + 8 * c) = mv[j];
      }
    }
    __syncthreads();
  } else {
#pragma unroll
    for (int j = 0; j < NB; ++j) load_group(braw[j], blane, min(wave + j * W, lastc));
  }
  // Dense B without ALDS: the A fragments of the batch's NB groups are
  // requested right after their rows of B (clamped group indices, as for B:
  // every load is unconditional). bf16 [4096, 14336] M = 5 / 8 / 16 28.5 /
  // 30.0 / 35.7 -> 26.9 / 28.3 / 34.5 us; a quantized B measured slower with
  // it (M = 5 17.5 -> 20.6 us), so it and ALDS read A per group.
  constexpr bool kPre = !ALDS && !BSrc::kMeta;
  constexpr int kAB = kPre ? NB : 1;
  F afb[kAB][MT][kSteps];
  if constexpr (kPre) {
#pragma unroll
    for (int j = 0; j < NB; ++j) load_af(afb[j], min(wave + j * W, lastc));
  }
  for (int c0 = 0; c0 < nw; c0 += NB) {
    if (c0 > 0) {
#pragma unroll
      for (int j = 0; j < NB; ++j) load_group(braw[j], blane, min(wave + (c0 + j) * W, last));
      if constexpr (kPre) {
#pragma unroll
        for (int j = 0; j < NB; ++j) load_af(afb[j], min(wave + (c0 + j) * W, last));
      }
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if (c0 + j < nw) {
        const int g = wave + (c0 + j) * W;
        f32x4 acc[MT];
        if constexpr (kPre) mma_group<T, BSrc, MT, true>(bsrc, braw[j], afb[j], g, q, acc);
        else compute(braw[j], g, acc);
#pragma unroll
        for (int i = 0; i < MT; ++i) part[(g * MT + i) * kWave + lane] = acc[i];
      }
    }
  }
  // A last group cut short by K (zero-padded past K), A from global memory.
  if (gfull < G && wave == gfull % W) {
    f32x4 acc[MT];
    direct_group<T, BSrc, MT, false>(a, lda, bsrc, n, rows, K, gfull, q, acc);
#pragma unroll
    for (int i = 0; i < MT; ++i) part[(gfull * MT + i) * kWave + lane] = acc[i];
  }
  __syncthreads();
  // Ordered fold: one thread per output element (m-tile i, lane l, register
  // e of the MFMA result layout), so every wave takes a share.
  const float* partf = reinterpret_cast<const float*>(part);
  for (int idx = threadIdx.x; idx < MT * kWave * 4; idx += kWave * W) {
    const int i = idx / (4 * kWave), e = (idx / kWave) % 4, l = idx % kWave;
    // Loads eight groups at a time so the LDS latency is paid once per eight;
    // the adds stay in group order.
    const float* pp = partf + (i * kWave + l) * 4 + e;
    const int gstride = MT * kWave * 4;
    float total = 0.f;
    int gg = 0;
    for (; gg + 8 <= G; gg += 8) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = pp[(gg + j) * gstride];
#pragma unroll
      for (int j = 0; j < 8; ++j) total = total + v[j];
    }
    for (; gg < G; ++gg) total = total + pp[gg * gstride];
    const int col = n_base + l % 16;
    const int m = m_base + 16 * i + 4 * (l / 16) + e;
    if (m < M && col < N) out[(int64_t)m * N + col] = to_store<T>(total);
  }
}

// Left fold of the group partials, exactly the fused kernels' fold:
// total = 0; total = total + part[g] for g = 0 .. G-1; out = T(total).
// Loads are issued eight groups at a time; the adds stay in group order.
template <typename T>
__global__ __launch_bounds__(256) void fold_groups(const float* __restrict__ part,
                                                   T* __restrict__ out, int64_t MN, int G) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= MN) return;
  float total = 0.0f;
  int g = 0;
  for (; g + 8 <= G; g += 8) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = part[(int64_t)(g + j) * MN + idx];
#pragma unroll
    for (int j = 0; j < 8; ++j) total = total + v[j];
  }
  for (; g < G; ++g) total = total + part[(int64_t)g * MN + idx];
  out[idx] = to_store<T>(total);
}

// ---------------------------------------------------------------------------
// gemm_lds: BM x BN tile, 4 waves in 2 x 2, each wave (BM/2) x (BN/2).
// K stage = two MFMA steps {2p, 2p+1} of group g (64 k, which k is the op's
// k-slot map); group g = stages 4g .. 4g+3.
// ---------------------------------------------------------------------------
constexpr int kStageK = 64;
constexpr int kLdsPad = 8;                      // elements; rows 16 B apart in banks
constexpr int kLdsRow = kStageK + kLdsPad;      // LDS row length (elements)

// Stages the two MFMA steps {2p, 2p+1} of group g for ROWS rows into LDS as
// 8-element chunks; MAP (the B source type) says which k each LDS chunk holds.
template <typename T, int ROWS, class MAP>
struct StageA {
  static constexpr int kChunks = ROWS * (kStageK / 8) / 256;  // per thread
  typedef typename Frag<T>::type F;
  F v[kChunks];
  __device__ __forceinline__ void load(const T* a, int64_t lda, int M, int K, int m0, int g, int p) {
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int c = threadIdx.x + 256 * i;
      const int row = c / 8, kc = c % 8;
      const int m = m0 + row, k = MAP::stage_k(g, p, kc);
      const bool ok = m < M && k < K;
      const F x = frag_load(a + (ok ? (int64_t)m * lda + k : 0));
      v[i] = ok ? x : frag_zero<F>();
    }
  }
  __device__ __forceinline__ void store(T* lds) const {
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int c = threadIdx.x + 256 * i;
      const int row = c / 8, kc = c % 8;
      *reinterpret_cast<F*>(lds + row * kLdsRow + 8 * kc) = v[i];
    }
  }
};

// B stage for dense operands: same chunking as A over bt rows (columns n).
template <typename T, int ROWS>
struct StageDenseB {
  StageA<T, ROWS, DenseB<T>> s;
  __device__ __forceinline__ void load(const DenseB<T>& b, int n0, int g, int p) {
    s.load(b.bt, b.ldb, b.N, b.K, n0, g, p);
  }
  __device__ __forceinline__ void store(T* lds) const { s.store(lds); }
};

// B stage for quantized operands: each chunk is 8 consecutive codes of one
// row, dequantized with the row's scale/bias for that k and rounded to T.
template <typename T, int BITS, int GS, int ROWS>
struct StageQuantB {
  static constexpr int kChunks = ROWS * (kStageK / 8) / 256;
  static constexpr int kWords = BITS / 4;
  typedef typename Frag<T>::type F;
  typedef QuantB<T, BITS, GS> Src;
  uint32_t w[kChunks][kWords];
  T sc[kChunks], bs[kChunks];
  bool ok[kChunks];
  __device__ __forceinline__ void load(const Src& b, int n0, int g, int p) {
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int c = threadIdx.x + 256 * i;
      const int row = c / 8, kc = c % 8;
      const int n = n0 + row, k = Src::stage_k(g, p, kc);
      const bool good = n < b.N && k < b.K;
      const int64_t nn = good ? n : 0;
      const int kk = good ? k : 0;
      const uint32_t* wp = b.w + nn * b.words_per_row + (int64_t)kk * BITS / 32;
      if constexpr (BITS == 4) {
        w[i][0] = wp[0];
      } else {
        const uint2 x = *reinterpret_cast<const uint2*>(wp);
        w[i][0] = x.x;
        w[i][1] = x.y;
      }
      const int64_t si = nn * b.groups_per_row + kk / GS;
      sc[i] = b.scales[si];
      bs[i] = b.biases[si];
      ok[i] = good;
    }
  }
  __device__ __forceinline__ void store(T* lds) const {
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int c = threadIdx.x + 256 * i;
      const int row = c / 8, kc = c % 8;
      const float s = to_f32(sc[i]), bb = to_f32(bs[i]);
      float d[8];
      if constexpr (BITS == 4) {
#pragma unroll
        for (int e = 0; e < 8; ++e) d[e] = __builtin_fmaf((float)((w[i][0] >> (4 * e)) & 0xFu), s, bb);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          d[e] = __builtin_fmaf((float)((w[i][0] >> (8 * e)) & 0xFFu), s, bb);
          d[4 + e] = __builtin_fmaf((float)((w[i][1] >> (8 * e)) & 0xFFu), s, bb);
        }
      }
      F f;
      if constexpr (sizeof(T) == 2) {
        typedef T vec8 __attribute__((ext_vector_type(8)));
        vec8 rr;
#pragma unroll
        for (int e = 0; e < 8; ++e) rr[e] = to_store<T>(d[e]);
        f = __builtin_bit_cast(F, rr);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          f.lo[e] = d[e];
          f.hi[e] = d[4 + e];
        }
      }
      *reinterpret_cast<F*>(lds + row * kLdsRow + 8 * kc) = ok[i] ? f : frag_zero<F>();
    }
  }
};

template <class BSrc, typename T, int ROWS> struct StageFor;
template <typename T, int ROWS> struct StageFor<DenseB<T>, T, ROWS> { typedef StageDenseB<T, ROWS> type; };
template <typename T, int BITS, int GS, int ROWS> struct StageFor<QuantB<T, BITS, GS>, T, ROWS> {
  typedef StageQuantB<T, BITS, GS, ROWS> type;
};

template <typename T, class BSrc, int BM, int BN>
__global__ __launch_bounds__(256) void gemm_lds(const T* __restrict__ a, int64_t lda, BSrc bsrc,
                                                T* __restrict__ out, int M, int N, int K, int G,
                                                int tiles_n, int tiles_total) {
  typedef typename Frag<T>::type F;
  constexpr int TM = BM / 32, TN = BN / 32;  // 16x16 tiles per wave along m and n
  __shared__ __attribute__((aligned(16))) T As[2][BM * kLdsRow];
  __shared__ __attribute__((aligned(16))) T Bs[2][BN * kLdsRow];

  // XCD-aware tile order: consecutive workgroup ids are dealt round-robin to
  // the 8 XCDs; give each XCD a contiguous run of tiles so neighbouring tiles
  // share that XCD's L2. Launch order only.
  const int bid = blockIdx.x;
  const int per_xcd = (tiles_total + 7) / 8;
  const int tile = (bid % 8) * per_xcd + bid / 8;
  if (tile >= tiles_total) return;  // uniform per workgroup, before any barrier
  const int tm = tile / tiles_n, tn = tile % tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int wm = wave / 2, wn = wave % 2;
  const int r = lane % 16, q = lane / 16;

  f32x4 total[TM][TN], acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      total[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      acc[i][j] = total[i][j];
    }

  StageA<T, BM, BSrc> sa;
  typename StageFor<BSrc, T, BN>::type sb;
  const int nstages = 4 * G;
  sa.load(a, lda, M, K, m0, 0, 0);
  sb.load(bsrc, n0, 0, 0);
  sa.store(As[0]);
  sb.store(Bs[0]);
  __syncthreads();

  for (int st = 0; st < nstages; ++st) {
    const int buf = st & 1;
    if (st + 1 < nstages) {
      sa.load(a, lda, M, K, m0, (st + 1) >> 2, (st + 1) & 3);
      sb.load(bsrc, n0, (st + 1) >> 2, (st + 1) & 3);
    }
    const T* Ab = As[buf] + (wm * TM * 16 + r) * kLdsRow + 8 * q;
    const T* Bb = Bs[buf] + (wn * TN * 16 + r) * kLdsRow + 8 * q;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      F af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const F*>(Ab + 16 * i * kLdsRow + 32 * s2);
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = *reinterpret_cast<const F*>(Bb + 16 * j * kLdsRow + 32 * s2);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma_step(af[i], bf[j], acc[i][j]);
    }
    if ((st & 3) == 3) {  // end of a 256-k group: fold and restart from zero
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          total[i][j] = total[i][j] + acc[i][j];
          acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    if (st + 1 < nstages) {
      sa.store(As[buf ^ 1]);
      sb.store(Bs[buf ^ 1]);
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn * TN * 16 + 16 * j + r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + wm * TM * 16 + 16 * i + 4 * q + e;
        if (m < M && n < N) out[(int64_t)m * N + n] = to_store<T>(total[i][j][e]);
      }
    }
}

static inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// Launch-shape policy (kernels/matmul.py:279-314): M <= 32 with more than one
// group -> split partials + fold; otherwise fused. Bits never depend on it.
static inline bool use_split(int64_t M, int G) { return M <= kSplitMMax && G > 1; }
// The in-workgroup fold keeps every group partial in LDS (1 KB per group and
// 16-row tile); up to 64 KB of it. Larger K takes the split + fold launch.
static inline bool use_wg(int64_t M, int G) { return M <= kSplitMMax && G * (M <= 16 ? 1 : 2) <= 64; }

// Dense large tile (bi_gemm_big.h) for 2-byte types, K % 64 == 0, M > 64, in
// three forms: 256 x 128 (8 waves), 128 x 128 (4 waves, one per SIMD) and
// 128 x 64 (4 waves, two workgroups per CU). The policy, a function of the
// shape only (so the workspace query and the launch agree; bits never depend
// on it):
//   1. 128 x 64 when it has kBigNarrowMinTiles..kBigFitTiles tiles (at most one
//      per CU) and K >= 768;
//   2. else 128 x 128 when its tiles fit one per CU and either the 256 x 128
//      rule below holds or 64 < M <= 256 with kBigHalfMinTiles tiles (K >=
//      768, and not K < 1024 with a part-filled last row tile);
//   3. else 256 x 128 from M = 129 with kBigMinTiles tiles, or M > 256 with
//      kBigShortKMinTiles tiles and at most 4 groups of K.
// Other shapes take the tall tile or the small-M launches. A tile's time is
// nearly flat in the number of tiles up to one per CU, so the smallest form
// that still fits the chip in one round wins. Measured on one MI355X, bf16
// us, old policy -> this one (stock hipBLASLt):
//   [4096, 4096]  M = 192 / 256 / 512 / 1024: 33.2 / 37.2 / 90.0 / 39.6 ->
//                 25.7 / 27.1 / 27.5 / 38.1 (- / - / 31.4 / 41.6);
//   [4096, 14336] M = 192 / 512 / 1024: 109.3 / 310.1 / 139.5 -> 82.2 / 94.7 /
//                 135.2 (- / 89.0 / 130.4);
//   [14336, 4096] M = 80 / 128 / 256: 38.5 / 44.0 / 43.7 -> 30.6 / 32.6 / 42.9;
//   [6144, 4096]  M = 128 / 256 / 512: 38.7 / 38.0 / 39.4 -> 27.9 / 27.8 / 38.6;
//   [4864, 896]   M = 128 / 192 / 256: 10.3 / 10.8 / 13.6 -> 9.3 / 8.9 / 9.4;
//   [1024, 4096]  M = 768 / 1024 / 2048: 68.6 / 68.6 / 88.2 -> 26.1 / 25.7 / 26.5
//                 (20.5 / 21.1 / -).
// With 64 tiles of 128 x 64 or fewer the tall tile (with K chunks) is faster
// ([4096, 4096] M = 128: 25.0 against 27.0; [1024, 4096] M = 384: 23.5
// against 25.9), and a 128 x 64 tiling with more tiles than CUs is slower than
// the 128 x 128 one ([14336, 4096] M = 192: 47.8 against 40.8).
constexpr int kBigFromM = 129;
constexpr int kBigShortKMinTiles = 32;
constexpr int kTallMaxM = 256;
constexpr int kBigFitTiles = 256;
constexpr int kBigNarrowMinTiles = 72;
constexpr int kBigHalfMinTiles = 48;
enum BigForm { kBig256x128 = 0, kBig128x128 = 1, kBig128x64 = 2 };
constexpr int kBigFormRows[3] = {256, 128, 128};
constexpr int kBigFormCols[3] = {128, 128, 64};
static inline int64_t big_form_tiles(int64_t M, int64_t N, int form) {
  return (int64_t)ceil_div(M, kBigFormRows[form]) * ceil_div(N, kBigFormCols[form]);
}
struct BigPlan {
  bool use = false;
  int form = kBig256x128;
  int tiles_m = 0, tiles_n = 0;
};
static inline BigPlan big_plan(int64_t M, int64_t N, int64_t K) {
  BigPlan p;
  if (M <= 64 || N <= 0 || K <= 0 || K % 64) return p;
  const int64_t t256 = big_form_tiles(M, N, kBig256x128), t128 = big_form_tiles(M, N, kBig128x128),
                t64 = big_form_tiles(M, N, kBig128x64);
  const bool full = M >= kBigFromM &&
                    (t256 >= kBigMinTiles || (M > kTallMaxM && K <= 4 * kGroupK && t256 >= kBigShortKMinTiles));
  const bool half_mid = M <= kTallMaxM && t128 >= kBigHalfMinTiles && K >= 768 &&
                        !(K < 1024 && M % kBigFormRows[kBig128x128] != 0);
  if (t64 >= kBigNarrowMinTiles && t64 <= kBigFitTiles && K >= 768) p.form = kBig128x64;
  else if (t128 <= kBigFitTiles && (full || half_mid)) p.form = kBig128x128;
  else if (full) p.form = kBig256x128;
  else return p;
  p.use = true;
  p.tiles_m = ceil_div(M, kBigFormRows[p.form]);
  p.tiles_n = ceil_div(N, kBigFormCols[p.form]);
  return p;
}

// Launch of a planned large-tile call (tile index order: bi_gemm_big.h).
template <typename T>
static void launch_big(const BigPlan& bp, const T* a, int64_t lda, const T* bt, int64_t ldb, T* out, int M, int N,
                       int K, hipStream_t st) {
  const int work = bp.tiles_m * bp.tiles_n, grid = ((work + 7) / 8) * 8;
  if (bp.form == kBig128x64)
    gemm_big<T, 2, 64><<<grid, big_threads<2, 64>(), 0, st>>>(a, lda, bt, ldb, out, M, N, K, bp.tiles_m,
                                                              bp.tiles_n);
  else if (bp.form == kBig128x128)
    gemm_big<T, 2><<<grid, big_threads<2, kBigBN>(), 0, st>>>(a, lda, bt, ldb, out, M, N, K, bp.tiles_m,
                                                              bp.tiles_n);
  else
    gemm_big<T><<<grid, big_threads<4, kBigBN>(), 0, st>>>(a, lda, bt, ldb, out, M, N, K, bp.tiles_m, bp.tiles_n);
}

// Dense mid-M launch (bi_gemm_tall.h) for 2-byte types: 16 < M <= 1024,
// K % 64 == 0, where the large tile is not used. Tile configurations (rows
// x columns, k per stage, ring cap): a ring of 3-6 stages leaves LDS for 1-3
// workgroups per CU, which measured faster than one workgroup with the
// deepest ring at every shape tried (4 waves per workgroup; more workgroups
// per CU overlap one's waits with another's MFMAs).
enum TallTile { kT64x64s64, kT64x32, kT64x32s64, kT32x64, kT32x32, kT32x64s64, kT32x32s64, kTallTiles };
struct TallShape {
  int bm, bn, sk, ring;
};
constexpr TallShape kTallShapes[kTallTiles] = {
    {64, 64, 64, 4}, {64, 32, 128, 3}, {64, 32, 64, 4}, {32, 64, 128, 4},
    {32, 32, 128, 4}, {32, 64, 64, 5}, {32, 32, 64, 6}};
// Workgroups of a configuration one CU holds at once (LDS-bound: the ring of
// stages of BM + BN rows, A rows in whole copy slots of 4 waves).
constexpr int tall_occupancy(const TallShape& t) {
  const int slot_rows = 4 * (64 / (t.sk / 8));
  const int rows = (t.bm / slot_rows + (t.bn + slot_rows - 1) / slot_rows) * slot_rows;
  const int stage = rows * t.sk * 2;
  const int ring = t.ring < 160 * 1024 / stage ? t.ring : 160 * 1024 / stage;  // as TallCfg::kRing
  const int per_cu = 160 * 1024 / (ring * stage);
  return per_cu < 8 ? per_cu : 8;
}
static_assert(tall_occupancy(TallShape{64, 32, 64, 4}) == 3 && tall_occupancy(TallShape{32, 64, 128, 4}) == 1,
              "tall_occupancy: LDS per workgroup as TallCfg lays it out");

struct TallPlan {
  bool use = false;
  int tile = 0, chunks = 1, cg = 0;
};
// The choice (a function of the shape only, so the workspace query and the
// launch agree):
//   * M <= 32: 32-row tiles, the widest column tile (64, else 32) that gives
//     kTallMinTiles workgroups (kTallMinTilesShortK for at most 4 groups of
//     K); with too few even at 32 columns, K is split into chunks of groups.
//   * 32 < M <= 256: the configuration that comes closest to filling the
//     chip's workgroup slots (256 CUs x its occupancy) without needing a
//     second round; ties go to the higher occupancy. When even the best one
//     fills less than half the slots and K has at least 8 groups, K is split
//     into 2 or 4 chunks by the same measure.
// Measured over Llama-3-8B and Qwen2-0.5B dense shapes (M = 32..256): within
// 2% of the best configuration tried on average, 10-30% faster than one
// workgroup per CU with the deepest ring.
constexpr int kTallMinTiles = 200;
// Up to this M the tall tile also serves the shapes the large tile leaves out
// (few output columns: [1024, 4096] M = 384 / 512 23.5 / 24.9 us, [896, 4864]
// 24.8 / 29.1 us, where the generic LDS tile took 68-80 us).
constexpr int kTallPlanMaxM = 1024;
constexpr int kTallMinTilesShortK = 100;
static inline TallPlan tall_plan(int64_t M, int64_t N, int64_t K) {
  TallPlan p;
  if (M <= 16 || M > kTallPlanMaxM || N <= 0 || K <= 0 || K % 64) return p;
  if (big_plan(M, N, K).use) return p;
  const int G = ceil_div(K, kGroupK);
  const bool k128 = K % 128 == 0;
  auto split = [&](int want) {
    p.cg = ceil_div(G, want);
    p.chunks = ceil_div(G, p.cg);
  };
  p.use = true;
  p.cg = G;
  if (M <= 32) {
    const int min_tiles = G <= 4 ? kTallMinTilesShortK : kTallMinTiles;
    const bool wide = ceil_div(N, 64) >= min_tiles;
    p.tile = wide ? (k128 ? kT32x64 : kT32x64s64) : (k128 ? kT32x32 : kT32x32s64);
    const int64_t t = ceil_div(N, wide ? 64 : 32);
    if (t < min_tiles && G > 1) split((int)std::min<int64_t>(G, ceil_div(min_tiles, t)));
    return p;
  }
  // Fill of a configuration: workgroups / (256 x occupancy); best = the
  // largest fill <= 1, else the smallest fill above 1; ties: occupancy, then
  // table order, then fewer chunks.
  double best_f = -1.0;
  int best_t = -1, best_c = 1;
  auto better = [&](double f, int t) {
    if (best_t < 0) return true;
    const bool in = f <= 1.0, bin = best_f <= 1.0;
    if (in != bin) return in;
    if (f != best_f) return in ? f > best_f : f < best_f;
    const int occ = tall_occupancy(kTallShapes[t]), bocc = tall_occupancy(kTallShapes[best_t]);
    if (occ != bocc) return occ > bocc;
    return t < best_t;
  };
  for (int chunks : {1, 2, 4}) {
    // K is split only when no unsplit configuration fills half the slots.
    if (chunks > 1 && (G < 8 || G < 2 * chunks || (best_c == 1 && best_f >= 0.5))) break;
    for (int t = 0; t < kTallTiles; ++t) {
      const TallShape& s = kTallShapes[t];
      if (K % s.sk || (s.sk == 64 && k128 && s.bm == 32)) continue;  // 32-row tiles: 64-k stages only for K % 128 != 0
      const double f = (double)(ceil_div(M, s.bm) * ceil_div(N, s.bn) * chunks) / (256.0 * tall_occupancy(s));
      if (better(f, t)) {
        best_f = f;
        best_t = t;
        best_c = chunks;
      }
    }
  }
  p.tile = best_t;
  if (best_c > 1) split(best_c);
  return p;
}

// Large-M quantized launch (bi_qmm_big.h), 2-byte T, K % 256 == 0, M >=
// kBigMinM: whenever the dense policy runs the shape on a large-tile form or
// on the tall tile without K chunks. The dequantized weight is then read by
// one tiled GEMM; the dequantization costs one pass over the codes and one
// write of the weight ([4096, 4096] 4-bit: 8.4 MB read, 33.6 MB written).
inline bool qmm_use_big(int64_t M, int64_t N, int64_t K, int elem_bytes) {
  if (elem_bytes != 2 || M < kBigMinM || K % kGroupK || K >= kBigMaxLd) return false;
  if (big_plan(M, N, K).use) return true;
  const TallPlan tp = tall_plan(M, N, K);
  return tp.use && tp.chunks == 1;
}

template <typename T, int TI, int WM, int WN, int SK, int R>
static void launch_tall2(const T* a, int64_t lda, const DenseB<T>& b, T* out, float* ws, int M, int N, int K,
                         int G, const TallPlan& p, hipStream_t st) {
  dim3 grid(ceil_div(N, 16 * WN), ceil_div(M, 16 * TI * WM), p.chunks);
  if (p.chunks > 1) {
    gemm_tall<T, TI, WM, WN, SK, true, R><<<grid, 256, 0, st>>>(a, lda, b.bt, b.ldb, out, ws, M, N, K, G, p.cg);
    const int64_t MN = (int64_t)M * N;
    fold_groups<T><<<(unsigned)((MN + 255) / 256), 256, 0, st>>>(ws, out, MN, G);
  } else {
    gemm_tall<T, TI, WM, WN, SK, false, R><<<grid, 256, 0, st>>>(a, lda, b.bt, b.ldb, out, ws, M, N, K, G, G);
  }
}

template <typename T>
static void launch_tall(const T* a, int64_t lda, const DenseB<T>& b, T* out, float* ws, int M, int N, int K,
                        int G, const TallPlan& p, hipStream_t st) {
  // Template arguments per configuration: TI x WM row blocks of 16, WN
  // column blocks of 16 (4 waves), SK, ring cap (kTallShapes).
  switch (p.tile) {
    case kT64x64s64: launch_tall2<T, 4, 1, 4, 64, 4>(a, lda, b, out, ws, M, N, K, G, p, st); break;
    case kT64x32: launch_tall2<T, 2, 2, 2, 128, 3>(a, lda, b, out, ws, M, N, K, G, p, st); break;
    case kT64x32s64: launch_tall2<T, 2, 2, 2, 64, 4>(a, lda, b, out, ws, M, N, K, G, p, st); break;
    case kT32x64: launch_tall2<T, 2, 1, 4, 128, 4>(a, lda, b, out, ws, M, N, K, G, p, st); break;
    case kT32x32: launch_tall2<T, 1, 2, 2, 128, 4>(a, lda, b, out, ws, M, N, K, G, p, st); break;
    case kT32x64s64: launch_tall2<T, 2, 1, 4, 64, 5>(a, lda, b, out, ws, M, N, K, G, p, st); break;
    default: launch_tall2<T, 1, 2, 2, 64, 6>(a, lda, b, out, ws, M, N, K, G, p, st); break;  // 32 x 32, 64-k
  }
}

template <typename T, class BSrc, int BM, int BN>
static void launch_lds(const T* a, int64_t lda, const BSrc& bsrc, T* out, int M, int N, int K,
                       int G, hipStream_t st) {
  const int tn = ceil_div(N, BN), tmm = ceil_div(M, BM);
  const int total = tn * tmm;
  const int grid = ((total + 7) / 8) * 8;
  gemm_lds<T, BSrc, BM, BN><<<grid, 256, 0, st>>>(a, lda, bsrc, out, M, N, K, G, tn, total);
}

template <typename T, class BSrc, int W, int NB, bool ALDS, bool META, int AC>
static void launch_wg1(const T* a, int64_t lda, const BSrc& bsrc, T* out, int M, int N, int K, int G,
                       size_t lds, hipStream_t st) {
  gemv_wg<T, BSrc, 1, W, NB, ALDS, META, AC><<<dim3(ceil_div(N, 16)), kWave * W, lds, st>>>(a, lda, bsrc, out,
                                                                                         M, N, K, G);
}

// ALDS launches, by per-wave group count: A chunks per thread 2 (one row of
// K = 4096 with 4 waves, the decode case) or the maximum.
template <typename T, class BSrc, int W, bool META, int AC>
static void launch_wg_alds(const T* a, int64_t lda, const BSrc& bsrc, T* out, int M, int N, int K, int G,
                           size_t lds, int per_wave, hipStream_t st) {
  if (per_wave <= 1) launch_wg1<T, BSrc, W, 1, true, META, AC>(a, lda, bsrc, out, M, N, K, G, lds, st);
  else if (per_wave <= 2) launch_wg1<T, BSrc, W, 2, true, META, AC>(a, lda, bsrc, out, M, N, K, G, lds, st);
  else launch_wg1<T, BSrc, W, 4, true, META, AC>(a, lda, bsrc, out, M, N, K, G, lds, st);
}

// The barrier-free decode GEMV (bi_gemv_stream.h) for a quantized or a dense
// B: W waves of NB = G / W consecutive groups, M <= MR rows of A staged per
// wave (AG: read per group from global memory instead), CT column tiles per
// wave, B loads PD groups ahead. Returns false when the shape does not
// qualify.
template <typename T, class BSrc, int W, int NB, int MR, int PD, int CT = 1, bool AG = false>
static bool launch_stream1(const T* a, int64_t lda, const BSrc& b, T* out, int M, int N, int K, int G,
                           hipStream_t st) {
  constexpr int kCE = 16 / (int)sizeof(T);
  constexpr int GS = StreamMeta<BSrc>::kGS;
  constexpr int kSPR = GS > 0 ? NB * kGroupK / (GS > 0 ? GS : 1) : 0;
  // 2-byte T only: the kernel's 16-byte staging pieces are whole 8-element
  // fragments only there.
  // LDS of the configuration (GemvStreamCfg::kLdsBytes, computed here so an
  // unsupported configuration is never instantiated): MR rows x K of A do not
  // fit for every shape; the caller then falls back.
  constexpr size_t kElemBytes = (size_t)((AG ? 0 : MR * NB * kGroupK) + 2 * 16 * CT * kSPR) * sizeof(T);
  constexpr size_t kLds = (size_t)W * std::max<size_t>(kElemBytes, (size_t)NB * CT * kWave * 16);
  if constexpr (sizeof(T) != 2 || kSPR % kCE != 0 || (MR * NB * kGroupK) % (kCE * kWave) != 0 ||
                kLds > 160 * 1024) {
    return false;
  } else {
    typedef GemvStreamCfg<T, GS, W, NB, MR, CT, AG> C;
    static_assert(C::kLdsBytes == kLds, "launch_stream1: LDS size");
    if (G != W * NB) return false;
    // More than 64 KB of dynamic LDS (8 or 16 rows of A) is allowed
    // explicitly, once per instantiation (a failure leaves the default limit
    // and no error state behind; the launch then reports its own status).
    static const bool lds_raised = [] {
      if (C::lds_bytes(16) <= 65536) return true;
      const bool ok = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_stream<T, BSrc, W, NB, MR, PD, CT, AG>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
      if (!ok) (void)hipGetLastError();
      return ok;
    }();
    (void)lds_raised;
    gemv_stream<T, BSrc, W, NB, MR, PD, CT, AG><<<dim3(ceil_div(N, 16 * CT)), kWave * W, C::lds_bytes(G), st>>>(
        a, lda, b, out, M, N, K, G);
    return true;
  }
}

// Column tiles per wave of the streaming GEMV: the fewest (1, 2, 4) that bring
// the grid within one round of resident workgroups (LDS: four per CU at MR <= 4,
// two at MR = 8, one at MR = 16: A's MR rows x K of every workgroup sit in
// LDS). Each further tile reuses every A fragment the wave reads. Measured,
// 4-bit g64 [14336, 4096] (896 column tiles): M = 5 / 8 11.2 / 12.1 ->
// 10.1 / 10.5 us at MR = 8, CT = 2; M = 12 / 16 16.7 / 16.9 (the mid-M
// launch) -> 12.3 / 12.9 us at MR = 16, CT = 4; M = 1 keeps CT = 1 (9.2
// against 10.3 us).
constexpr int kStreamCUs = 256;   // MI355X compute units
inline int stream_ct(int MR, int N) {
  const int64_t cap = (int64_t)kStreamCUs * (MR >= 16 ? 1 : MR >= 8 ? 2 : 4);
  int ct = 1;
  while (ct < 4 && ceil_div(N, 16 * ct) > cap) ct *= 2;
  return ct;
}

// The streaming GEMV with A read per group from global memory (AG), for M <=
// 16 rows whose MR rows x K of A do not fit in LDS beside the other resident
// workgroups (K = 8192 at M > 8, K = 14336 at M > 4), with at least one column
// tile per CU (fewer tiles take the split-K mid-M launch). A's fragments of a
// group then come from L2 with the group's codes: each workgroup rereads A
// (M x K, a few hundred KB) from L2, which costs less than the workgroup-fold
// GEMV's per-group reads. Measured against the launches they replace (same
// box, bits equal), 4-bit g64 [4096, 14336] M = 5 / 8 / 12 / 16: 17.6 / 19.0
// / 20.7 / 23.1 -> 13.5 / 15.1 / 17.4 / 20.7 us (7 waves of 8 groups; 14 of 4
// equal); [4096, 8192] M = 12 / 16 12.7 / 14.0 -> 10.8 / 12.6 us, [8192,
// 8192] 23.9 / 25.6 -> 18.8 / 22.2 (4 waves of 8); 8-bit g128 [4096, 14336]
// M = 5 / 16 21.7 / 28.8 -> 16.7 / 23.8 us; dense bf16 [4096, 8192] M = 12 /
// 16 19.9 / 20.4 -> 15.1 / 16.4 us (8 waves of 4), [4096, 14336] M = 5 / 8
// 21.3 / 23.1 -> 20.6 / 22.3 us. Where A fits in LDS the staged launches are
// faster (K = 4096 M = 16: 12.8 against 14.2 us), so they keep those shapes.
template <typename T, class BSrc, int W, int NB>
static bool launch_stream_ag(const T* a, int64_t lda, const BSrc& b, T* out, int M, int N, int K, int G,
                             hipStream_t st) {
  if (M > 16 || ceil_div(N, 16) < kStreamCUs) return false;
  return launch_stream1<T, BSrc, W, NB, 16, 1, 1, true>(a, lda, b, out, M, N, K, G, st);
}

template <typename T, class QB, int W, int NB, int PD>
static bool launch_stream_m(const T* a, int64_t lda, const QB& b, T* out, int M, int N, int K, int G,
                            hipStream_t st) {
  constexpr int BITS = QB::kBits;
  if (M == 1) return launch_stream1<T, QB, W, NB, 1, PD>(a, lda, b, out, M, N, K, G, st);
  // 2-4 rows share the 4-row A slice: a 2-row slice measured no faster
  // ([14336, 4096] M = 2 9.28-9.38 against 9.20-9.50 us, same box).
  if (M <= 4) return launch_stream1<T, QB, W, NB, 4, PD>(a, lda, b, out, M, N, K, G, st);
  if constexpr (BITS == 4) {
    // Column tiles only for 4-bit codes (8-bit codes of four tiles do not fit
    // the register file next to A).
    if (M <= 8) {
      if (stream_ct(8, N) > 1) return launch_stream1<T, QB, W, NB, 8, PD, 2>(a, lda, b, out, M, N, K, G, st);
      return launch_stream1<T, QB, W, NB, 8, PD>(a, lda, b, out, M, N, K, G, st);
    }
    switch (stream_ct(16, N)) {
      case 4: return launch_stream1<T, QB, W, NB, 16, PD, 4>(a, lda, b, out, M, N, K, G, st);
      case 2: return launch_stream1<T, QB, W, NB, 16, PD, 2>(a, lda, b, out, M, N, K, G, st);
      default: return launch_stream1<T, QB, W, NB, 16, PD>(a, lda, b, out, M, N, K, G, st);
    }
  } else {
    if (M > 8) return false;
    return launch_stream1<T, QB, W, NB, 8, PD>(a, lda, b, out, M, N, K, G, st);
  }
}

// Launch shapes in order of preference (measured, Llama MLP shape, M = 1):
// two groups per wave with one group of codes in flight beyond the one being
// computed, else four groups per wave one ahead (8-bit g128, whose two-group
// scale slice is not a whole 16-byte load: 13.7 us against 14.1 two ahead). A
// shape whose scale slice or A slice is not whole 16-byte loads is skipped.
// 32 and 56 groups (K = 8192, 14336) run 8 and 14 waves of four groups:
// [4096, 8192] M = 1 / 4 / 8 8.7 / 10.7 / 11.4 -> 6.6 / 7.2 / 8.1 us, the
// Llama MLP down projection [4096, 14336] M = 1 / 4 16.7 / 17.5 -> 9.7 /
// 11.0 us (A's rows x K must fit in LDS: M <= 8 and M <= 4 there).
template <typename T, int BITS, int GS>
static bool launch_stream(const T* a, int64_t lda, const QuantB<T, BITS, GS>& b, T* out, int M, int N, int K,
                          int G, hipStream_t st) {
  typedef QuantB<T, BITS, GS> QB;
  if (M > kStreamMMax || K % kGroupK) return false;
  if (b.groups_per_row % (16 / (int)sizeof(T)) || !bi_host::aligned16(b.scales) || !bi_host::aligned16(b.biases) ||
      lda % (16 / (int)sizeof(T)) || !bi_host::aligned16(a))
    return false;
  switch (G) {
    case 16:
      return launch_stream_m<T, QB, 8, 2, 1>(a, lda, b, out, M, N, K, G, st) ||
             launch_stream_m<T, QB, 4, 4, 1>(a, lda, b, out, M, N, K, G, st);
    case 8:
      return launch_stream_m<T, QB, 4, 2, 1>(a, lda, b, out, M, N, K, G, st) ||
             launch_stream_m<T, QB, 2, 4, 2>(a, lda, b, out, M, N, K, G, st);
    case 4:
      return launch_stream_m<T, QB, 4, 1, 1>(a, lda, b, out, M, N, K, G, st) ||
             launch_stream_m<T, QB, 2, 2, 1>(a, lda, b, out, M, N, K, G, st) ||
             launch_stream_m<T, QB, 1, 4, 2>(a, lda, b, out, M, N, K, G, st);
    case 32:
      return launch_stream_m<T, QB, 8, 4, 1>(a, lda, b, out, M, N, K, G, st) ||
             launch_stream_ag<T, QB, 4, 8>(a, lda, b, out, M, N, K, G, st);
    case 56:
      return launch_stream_m<T, QB, 14, 4, 1>(a, lda, b, out, M, N, K, G, st) ||
             launch_stream_ag<T, QB, 7, 8>(a, lda, b, out, M, N, K, G, st);
    default:
      return false;
  }
}

// The streaming GEMV on a repacked B (QuantPacked: group size 64, the codes'
// and metadata's layout made for it): the launch shapes of launch_stream, with
// no staged metadata (so no scale-slice constraint). False when the shape does
// not qualify; the caller then runs the launch the MLX-layout B would take.
// Measured against the MLX layout (same box, bits equal), 4-bit [14336, 4096]
// M = 1 / 4 / 8 / 16: 9.68 / 10.52 / 10.98 / 13.31 -> 9.30-9.53 / 10.10 /
// 10.32 / 11.95 us; [4096, 14336] M = 4 / 8 / 16 11.20 / 15.59 / 20.84 ->
// 10.84 / 14.13 / 18.99 us.
template <typename T, int BITS, int GS>
static bool launch_stream_packed(const T* a, int64_t lda, const QuantPacked<T, BITS, GS>& b, T* out, int M, int N,
                                 int K, int G, hipStream_t st) {
  typedef QuantPacked<T, BITS, GS> QB;
  if (M > kStreamMMax || K % kGroupK || lda % (16 / (int)sizeof(T)) || !bi_host::aligned16(a)) return false;
  switch (G) {
    case 16:
      // 16 waves of one group (twice the waves per CU of 8 x 2 at the LDS A
      // takes) for 9-16 rows, and for 5-8 rows with one column tile per wave:
      // [14336, 4096] M = 12 / 16 11.2 / 11.5 -> 10.4 / 10.8 us, [4096, 4096]
      // M = 8 / 16 5.12 / 5.52 -> 4.67 / 5.48 us; 8 x 2 stays where 5-8 rows
      // take two column tiles (9.9 against 10.5 us at M = 8). For 1-4 rows
      // 16 x 1 (a 4-row A slice) wins only at 256 to 512 column tiles:
      // [4096, 4096] M = 1 / 2 / 4 4.36-4.44 / 4.55-4.68 / 4.62-4.70 ->
      // 4.15-4.33 / 4.20-4.40 / 4.26-4.34 us; with more tiles 8 x 2 stays
      // (896 tiles, M = 1: 9.3-9.7 against 10.1-10.7 us). 4-bit codes only:
      // 8-bit ones keep 8 x 2 (g128 [14336, 4096] M = 1 / 4 12.6-12.7 /
      // 13.4-13.7 against 16.6-17.0 / 17.2 us for 16 x 1, [4096, 4096] 5.3-5.6
      // / 5.7-5.9 against 5.6-5.8 / 5.9-6.0 us).
      if (BITS == 4 && M <= 4 && ceil_div(N, 16) >= 256 && ceil_div(N, 16) <= 512)
        return launch_stream1<T, QB, 16, 1, 4, 1>(a, lda, b, out, M, N, K, G, st);
      if (BITS == 4 && (M > 8 || (M > 4 && stream_ct(8, N) == 1)))
        return launch_stream_m<T, QB, 16, 1, 1>(a, lda, b, out, M, N, K, G, st);
      return launch_stream_m<T, QB, 8, 2, 1>(a, lda, b, out, M, N, K, G, st);
    case 8: return launch_stream_m<T, QB, 4, 2, 1>(a, lda, b, out, M, N, K, G, st);
    case 4:
      return M <= 2 && (launch_stream_m<T, QB, 4, 1, 1>(a, lda, b, out, M, N, K, G, st) ||
                        launch_stream_m<T, QB, 2, 2, 1>(a, lda, b, out, M, N, K, G, st) ||
                        launch_stream_m<T, QB, 1, 4, 2>(a, lda, b, out, M, N, K, G, st));
    case 32:
      return launch_stream_m<T, QB, 8, 4, 1>(a, lda, b, out, M, N, K, G, st) ||
             launch_stream_ag<T, QB, 4, 8>(a, lda, b, out, M, N, K, G, st);
    case 56:
      return launch_stream_m<T, QB, 14, 4, 1>(a, lda, b, out, M, N, K, G, st) ||
             launch_stream_ag<T, QB, 7, 8>(a, lda, b, out, M, N, K, G, st);
    default: return false;
  }
}

// The streaming GEMV for a dense 2-byte B, M <= 16: one column tile per wave
// (a dense tile is eight 16-byte loads per group and lane; two tiles measured
// slower), A's MR rows of the wave's groups staged in LDS. G = 16: 8 waves of
// 2 groups, 8: 4 of 2, 32: 8 of 4, 56: 14 of 4. Measured against the
// workgroup-fold GEMV it replaces (bf16, same-box probe, bits equal):
// [14336, 4096] M = 1 / 4 / 8 / 16 22.0 / 26.8 / 29.3 / 34.6 -> 21.5 / 22.0 /
// 23.8 / 28.6 us; [4096, 4096] 9.1 / 9.0 / 10.0 / 11.3 -> 7.7 / 8.0 / 8.3 /
// 9.1 us; [4096, 14336] M = 1 / 4 26.9 / 28.0 -> 21.5 / 22.4 us.
template <typename T, int W, int NB, class DB = DenseB<T>>
static bool launch_stream_dense_m(const T* a, int64_t lda, const DB& b, T* out, int M, int N, int K, int G,
                                  hipStream_t st) {
  if (M == 1) return launch_stream1<T, DB, W, NB, 1, 1>(a, lda, b, out, M, N, K, G, st);
  if (M <= 4) return launch_stream1<T, DB, W, NB, 4, 1>(a, lda, b, out, M, N, K, G, st);
  if (M <= 8) return launch_stream1<T, DB, W, NB, 8, 1>(a, lda, b, out, M, N, K, G, st);
  return launch_stream1<T, DB, W, NB, 16, 1>(a, lda, b, out, M, N, K, G, st);
}

template <typename T>
static bool launch_stream_dense(const T* a, int64_t lda, const DenseB<T>& b, T* out, int M, int N, int K, int G,
                                hipStream_t st) {
  if (M > kStreamMMax || K % kGroupK || b.ldb % (16 / (int)sizeof(T)) || !bi_host::aligned16(b.bt) ||
      lda % (16 / (int)sizeof(T)) || !bi_host::aligned16(a))
    return false;
  switch (G) {
    case 16: return launch_stream_dense_m<T, 8, 2>(a, lda, b, out, M, N, K, G, st);
    case 8: return launch_stream_dense_m<T, 4, 2>(a, lda, b, out, M, N, K, G, st);
    case 32:
      return launch_stream_dense_m<T, 8, 4>(a, lda, b, out, M, N, K, G, st) ||
             launch_stream_ag<T, DenseB<T>, 8, 4>(a, lda, b, out, M, N, K, G, st);
    case 56:
      return launch_stream_dense_m<T, 14, 4>(a, lda, b, out, M, N, K, G, st) ||
             launch_stream_ag<T, DenseB<T>, 7, 8>(a, lda, b, out, M, N, K, G, st);
    default: return false;
  }
}

// The dense streaming GEMV on a repacked B (DensePacked): the launch shapes of
// launch_stream_dense. False when the shape does not qualify; the caller then
// runs the launch the row-major B would take. Measured against the row-major
// layout (same box, bits equal), bf16 [14336, 4096] M = 1 / 8 / 16 21.50 /
// 23.89 / 28.51 -> 20.96 / 21.86 / 27.23 us; [4096, 14336] M = 4 23.60 ->
// 21.94; [4096, 4096] M = 1 / 8 7.99 / 8.75 -> 7.63 / 8.11; [1024, 4096]
// M = 1 / 16 5.81 / 7.11 -> 4.57 / 5.70 us.
// G = ceil(K / 256): the copy is zero past K, so K need only be a multiple of
// 8; 4 groups (K = 769 .. 1024, the Qwen2-0.5B projections' K = 896) run 4
// waves of one group, A's rows staged in LDS (config-1 linear [4864, 896]
// M = 1 / 4 / 16: 4.86 / 5.13 / 5.84 -> 4.12 / 4.15 / 4.70 us against the
// workgroup-fold GEMV on the row-major weight).
template <typename T>
static bool launch_stream_dense_packed(const T* a, int64_t lda, const DensePacked<T>& b, T* out, int M, int N,
                                       int K, int G, hipStream_t st) {
  typedef DensePacked<T> DB;
  if (M > kStreamMMax || K % 8 || lda % (16 / (int)sizeof(T)) || !bi_host::aligned16(a)) return false;
  switch (G) {
    case 4:
      if (M <= 4) return launch_stream1<T, DB, 4, 1, 4, 1>(a, lda, b, out, M, N, K, G, st);
      if (M <= 8) return launch_stream1<T, DB, 4, 1, 8, 1>(a, lda, b, out, M, N, K, G, st);
      return launch_stream1<T, DB, 4, 1, 16, 1>(a, lda, b, out, M, N, K, G, st);
    case 16: return launch_stream_dense_m<T, 8, 2, DB>(a, lda, b, out, M, N, K, G, st);
    case 8: return launch_stream_dense_m<T, 4, 2, DB>(a, lda, b, out, M, N, K, G, st);
    case 32:
      return launch_stream_dense_m<T, 8, 4, DB>(a, lda, b, out, M, N, K, G, st) ||
             launch_stream_ag<T, DB, 8, 4>(a, lda, b, out, M, N, K, G, st);
    case 56:
      return launch_stream_dense_m<T, 14, 4, DB>(a, lda, b, out, M, N, K, G, st) ||
             launch_stream_ag<T, DB, 7, 8>(a, lda, b, out, M, N, K, G, st);
    default: return false;
  }
}

// One thread per (16-row tile, group, MFMA lane): the lane's eight fragments
// copied into the DensePacked layout, zero past K (K % 8 == 0).
template <typename T>
__global__ __launch_bounds__(256) void dense_pack_rows(const T* __restrict__ bt, int64_t ldb,
                                                       char* __restrict__ packed, int N, int K) {
  typedef DensePacked<T> P;
  const int G = (K + kGroupK - 1) / kGroupK;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)((N + 15) / 16) * G * kWave) return;
  const int l = (int)(idx % kWave);
  const int64_t tg = idx / kWave;                  // tile * G + group
  const int g = (int)(tg % G);
  const int n = (int)min<int64_t>(tg / G * 16 + l % 16, N - 1);
  const int k0 = g * kGroupK + 8 * (l / 16);
  const T* src = bt + (int64_t)n * ldb + k0;
  char* blk = packed + tg * P::kBlock;
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const u32x4 v = k0 + 32 * s < K ? *reinterpret_cast<const u32x4*>(src + 32 * s) : u32x4{0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4*>(blk + 1024 * s + 16 * l) = v;
  }
}

template <typename T, class BSrc, int W>
static void launch_wg(const T* a, int64_t lda, const BSrc& bsrc, T* out, int M, int N, int K, int G,
                      hipStream_t st) {
  dim3 grid(ceil_div(N, 16), 1, 1);
  const int mt = M <= 16 ? 1 : 2;
  const size_t part_bytes = (size_t)G * mt * kWave * sizeof(f32x4);
  const size_t a_bytes = (size_t)M * (K + 8) * sizeof(T);
  constexpr int kThreads = kWave * W;
  // A staged in LDS: M <= 16 rows, K / 8 a multiple of the thread count, at
  // most kGemvAChunks / W chunks per thread.
  bool alds = M <= 16 && K % kGroupK == 0 && (K / 8) % kThreads == 0 &&
              (int64_t)M * K <= kGemvAChunks * kWave * 8 && part_bytes + a_bytes <= 65536;
  size_t meta_bytes = 0;
  if constexpr (BSrc::kMeta) {
    // A quantized B takes the ALDS path only with its scales and biases in LDS.
    meta_bytes = (size_t)32 * bsrc.groups_per_row * sizeof(T);
    alds = alds && 4 * bsrc.groups_per_row <= kGemvMetaChunks * kWave && bi_host::aligned16(bsrc.scales) &&
           bi_host::aligned16(bsrc.biases) && part_bytes + a_bytes + meta_bytes <= 65536;
  }
  const size_t lds = part_bytes + (alds ? a_bytes + meta_bytes : 0);
  const int per_wave = ceil_div(K / kGroupK, W);       // full groups per wave
  if (alds) {
    constexpr bool kM = BSrc::kMeta;
    const int64_t nA = (int64_t)M * (K / 8) / kThreads;   // exact: A chunks per thread
    if (nA == 2) launch_wg_alds<T, BSrc, W, kM, 2>(a, lda, bsrc, out, M, N, K, G, lds, per_wave, st);
    else if (nA == 1) launch_wg_alds<T, BSrc, W, kM, 1>(a, lda, bsrc, out, M, N, K, G, lds, per_wave, st);
    else if (nA <= 4 && (nA & (nA - 1)) == 0)
      launch_wg_alds<T, BSrc, W, kM, 4>(a, lda, bsrc, out, M, N, K, G, lds, per_wave, st);
    else alds = false;
    if (alds) return;
  }
  if (M <= 16) {
    // A quantized B with 5..16 rows and 32 or more groups (the Llama MLP down
    // projection at M = 5 .. 16, where A's rows x K do not fit in LDS):
    // codes of four groups requested ahead instead of two. 4-bit g64
    // [4096, 14336] M = 8 / 12 / 16 19.4 / 22.4 / 25.3 -> 18.4 / 20.8 / 23.3
    // us, [4096, 8192] M = 12 / 16 13.0 / 15.0 -> 12.7 / 14.0; a dense B
    // measured slower with it, and so did 16 waves either way.
    if (BSrc::kMeta && M > 4 && G >= 32)
      launch_wg1<T, BSrc, W, 4, false, false, 0>(a, lda, bsrc, out, M, N, K, G, part_bytes, st);
    else launch_wg1<T, BSrc, W, 2, false, false, 0>(a, lda, bsrc, out, M, N, K, G, part_bytes, st);
  } else {
    gemv_wg<T, BSrc, 2, W, 2, false><<<grid, kWave * W, part_bytes, st>>>(a, lda, bsrc, out, M, N, K, G);
  }
}

// Mid-M launch (bi_gemm_mid.h) for a quantized B, 2-byte T, K % 256 == 0:
// 16 < M < kBigMinM at any N, and 4 < M <= 16 with >= 128 blocks of 64
// columns. Row blocks of 16 MT rows (MT = 1 for M <= 16, 4 for 32 < M <= 64,
// else 2: M > 64 takes several);
// when the (column block, row block) tiles are fewer than kMidMinTiles, K is
// split into chunks of cg groups (per-group fp32 partials in the workspace,
// then fold_groups) so that about kMidTargetWG workgroups run.
constexpr int kMidMinTiles = 160;
constexpr int kMidTargetWG = 512;
struct MidPlan {
  bool use = false;
  int mt = 1, mtiles = 1, chunks = 1, cg = 0;
};
// 5 <= M <= 16 with at most 2048 columns and 32 or more groups, where the
// streaming GEMV (tried first) does not take the shape: the workgroup-fold
// GEMV would run one workgroup per 16 columns (at most 128, half the CUs) and
// read A's rows from L2 for every group; the split mid-M launch runs chunks of
// 4 groups on every CU and folds the per-group partials in order. Same-box
// probe, bits equal: 4-bit g64 [1024, 14336] M = 5 / 8 / 16 16.4 / 18.6 /
// 24.7 -> 11.8 / 12.2 / 12.6 us, [2048, 14336] 16.6 / 18.8 / 24.6 -> 14.7 /
// 15.1 / 17.0, [1024, 16384] 17.2 / 19.2 / 25.8 -> 12.3 / 12.6 / 13.0,
// [2048, 8192] M = 16 14.0 -> 12.0 (M <= 8 streams there); dense bf16
// [1024, 14336] 24.4 / 26.5 / 31.9 -> 14.0 / 14.1 / 14.2, [2048, 14336]
// 25.6 / 27.4 / 33.3 -> 21.0 / 21.0 / 22.3. With 20 groups, or 3072 columns
// and more, the workgroup-fold GEMV measured as fast or faster.
static inline MidPlan few_columns_plan(int64_t M, int64_t N, int64_t K) {
  MidPlan p;
  if (M <= 4 || M > 16 || N <= 0 || N > 2048 || K <= 0 || K % kGroupK || K / kGroupK < 32) return p;
  const int G = (int)(K / kGroupK);
  p.mt = 1;
  p.mtiles = (int)ceil_div(M, 16);
  p.cg = 4;
  p.chunks = ceil_div(G, p.cg);
  p.use = true;
  return p;
}

static inline MidPlan mid_plan(int64_t M, int64_t N, int64_t K) {
  MidPlan p;
  if (M <= 4 || M >= kBigMinM || N <= 0 || K <= 0 || K % kGroupK) return p;
  const int G = (int)(K / kGroupK);
  if (M <= 16 && ceil_div(N, 64) < 128) return few_columns_plan(M, N, K);
  // 64-row blocks only for 32 < M <= 64; larger M runs several 32-row blocks
  // (measured faster: more workgroups per CU, each a shallower register file).
  p.mt = M <= 16 ? 1 : (M <= 32 || M > 64) ? 2 : 4;
  p.mtiles = (int)ceil_div(M, 16 * p.mt);
  const int64_t t = ceil_div(N, 64) * p.mtiles;
  p.cg = G;
  if (t < kMidMinTiles && G > 1) {
    const int want = (int)std::min<int64_t>(G, ceil_div(kMidTargetWG, t));
    p.cg = ceil_div(G, want);
    p.chunks = ceil_div(G, p.cg);
  }
  p.use = true;
  return p;
}

template <typename T, class BSrc>
static bool use_mid(const MidPlan& p, int64_t lda, const T* a) {
  if constexpr (sizeof(T) != 2 || !BSrc::kMeta) {
    return false;
  } else {
    return p.use && lda % 8 == 0 && bi_host::aligned16(a);
  }
}

// Unsplit: an 8-group A ring for 16-row blocks, 4 for 32- and 64-row blocks
// (a deeper ring for 32 rows measured 7% slower), B loads 8 groups ahead. Split K: short chunks and several workgroups
// per CU, so a shallow ring and B loads kMidSplitPD groups ahead (a chunk runs
// in whole rounds of that many groups; the padding groups are not folded).
constexpr int kMidSplitPD = 2;
// Unsplit launches of at most this many workgroups (about one per CU) run the
// K-interleaved eight-wave kernel (two waves per SIMD); larger grids already
// put several four-wave workgroups on each CU, where it measured slower.
constexpr int kMidInterleaveMaxTiles = 320;
// B loads 4 stages ahead, 2 for 64-row blocks (measured at the Llama MLP
// shape, M = 64: 24.3 against 25.5 us; M = 16 / 32 prefer 4).
template <int MT> constexpr int mid_interleave_pd() { return MT == 4 ? 2 : 4; }
template <typename T, class BSrc, int MT, int NA_ONE, int NA_SPLIT>
static void launch_mid2(const T* a, int64_t lda, const BSrc& bsrc, T* out, float* ws, int M, int N, int K,
                        int G, const MidPlan& p, hipStream_t st) {
  constexpr int PD = 8;
  const dim3 grid(ceil_div(N, 64), p.mtiles, p.chunks);
  if (p.chunks == 1 && G >= 2 && (int64_t)grid.x * grid.y <= kMidInterleaveMaxTiles) {
    constexpr int NA2 = MT == 4 ? 2 : 4;
    gemm_mid2<T, BSrc, MT, mid_interleave_pd<MT>(), NA2, false><<<grid, 512, 0, st>>>(a, lda, bsrc, out, ws, M, N,
                                                                                      K, G, G);
    return;
  }
  if (p.chunks > 1) {
    gemm_mid<T, BSrc, MT, kMidSplitPD, NA_SPLIT, true><<<grid, 256, 0, st>>>(a, lda, bsrc, out, ws, M, N, K, G,
                                                                             p.cg);
    const int64_t MN = (int64_t)M * N;
    fold_groups<T><<<(unsigned)((MN + 255) / 256), 256, 0, st>>>(ws, out, MN, G);
  } else {
    gemm_mid<T, BSrc, MT, PD, NA_ONE, false><<<grid, 256, 0, st>>>(a, lda, bsrc, out, ws, M, N, K, G, G);
  }
}

template <typename T, class BSrc>
static void launch_mid(const T* a, int64_t lda, const BSrc& bsrc, T* out, float* ws, int M, int N, int K,
                       int G, const MidPlan& p, hipStream_t st) {
  if constexpr (sizeof(T) == 2 && BSrc::kMeta) {
    if (p.mt == 1) launch_mid2<T, BSrc, 1, 8, 4>(a, lda, bsrc, out, ws, M, N, K, G, p, st);
    else if (p.mt == 2) launch_mid2<T, BSrc, 2, 4, 4>(a, lda, bsrc, out, ws, M, N, K, G, p, st);
    else launch_mid2<T, BSrc, 4, 4, 2>(a, lda, bsrc, out, ws, M, N, K, G, p, st);
  }
}

template <typename T, class BSrc>
static int run_gemm(const T* a, int64_t lda, const BSrc& bsrc, T* out, int M, int N, int K,
                    float* ws, hipStream_t st, const char* what) {
  const int G = ceil_div(K, kGroupK);
  constexpr int WAVES = 4;
  if constexpr (BSrc::kMeta) {
    // The streaming GEMV wherever it takes the shape (M <= 16, 4-bit; M <= 8,
    // 8-bit, or up to 16 with A read from global memory at 32 or 56 groups),
    // at any number of column tiles, with 8 or more groups, or with 4
    // groups at M <= 2 and groups of up to 64 (4 groups of 128: 2.99 -> 3.82 us
    // at N = 256, M = 1). Measured against the workgroup-fold GEMV and the mid-M
    // launch it replaces (4-bit g64, bits equal): K = 4096 N = 4096 M = 1 / 4 /
    // 8 / 16 5.7 / 5.9 / 6.8 / 8.0 -> 4.5 / 4.8 / 5.3 / 6.0 us; N = 1024 (64
    // tiles) 4.6 / 4.8 / 6.2 / 7.5 -> 3.8 / 4.1 / 4.3 / 4.9 us; N = 16 (one
    // tile) 5.5 / 4.3 / 5.7 / 6.9 -> 3.7 / 3.7 / 3.9 / 4.3 us; K = 14336 N = 1024
    // M = 1 / 4 15.7 / 16.1 -> 8.1 / 9.6 us; 8-bit g64 K = 2048 N = 1024 M = 1 /
    // 8 5.6 / 5.9 -> 3.5 / 3.9 us.
    if ((G >= 8 || (M <= 2 && BSrc::kGS <= 64)) &&
        launch_stream<T, BSrc::kBits, BSrc::kGS>(a, lda, bsrc, out, M, N, K, G, st))
      return bi_host::launch_status(what);
  } else if constexpr (sizeof(T) == 2) {
    // Dense 2-byte B at any number of column tiles (bf16, bits equal): K =
    // 4096 N = 1024 M = 1 / 8 / 16 6.1 / 8.8 / 10.5 -> 5.8 / 6.6 / 7.2 us, N =
    // 16 M = 16 8.8 -> 6.2 us; K = 14336 N = 1024 M = 1 / 4 22.0 / 24.1 -> 15.0
    // / 16.8 us; K = 2048 N = 1024 M = 16 5.6 -> 4.3 us.
    if (launch_stream_dense<T>(a, lda, bsrc, out, M, N, K, G, st))
      return bi_host::launch_status(what);
    const MidPlan fp = few_columns_plan(M, N, K);
    if (fp.use && lda % 8 == 0 && bi_host::aligned16(a) && bsrc.ldb % 8 == 0 && bi_host::aligned16(bsrc.bt)) {
      launch_mid2<T, BSrc, 1, 8, 4>(a, lda, bsrc, out, ws, M, N, K, G, fp, st);
      return bi_host::launch_status(what);
    }
  }
  if constexpr (BSrc::kMeta) {
    const MidPlan mp = mid_plan(M, N, K);
    if (use_mid<T, BSrc>(mp, lda, a)) {
      launch_mid<T, BSrc>(a, lda, bsrc, out, ws, M, N, K, G, mp, st);
      return bi_host::launch_status(what);
    }
  }
  if constexpr (sizeof(T) == 2 && std::is_same<BSrc, DenseB<T>>::value) {
    const BigPlan bp = big_plan(M, N, K);
    if (bp.use && lda < kBigMaxLd && bsrc.ldb < kBigMaxLd) {
      launch_big<T>(bp, a, lda, bsrc.bt, bsrc.ldb, out, M, N, K, st);
      return bi_host::launch_status(what);
    }
    const TallPlan tp = tall_plan(M, N, K);
    if (tp.use && lda < kBigMaxLd && bsrc.ldb < kBigMaxLd) {
      launch_tall<T>(a, lda, bsrc, out, ws, M, N, K, G, tp, st);
      return bi_host::launch_status(what);
    }
  }
  if (M <= kSplitMMax && use_wg(M, G)) {
    // 4 waves per workgroup when there are enough column tiles for every
    // workgroup to be resident at once (4 per CU at <= 128 VGPRs), so the whole
    // weight stream is requested up front; 8 waves otherwise, to spread K.
    if (ceil_div(N, 16) >= 512 && G >= 8) launch_wg<T, BSrc, 4>(a, lda, bsrc, out, M, N, K, G, st);
    else launch_wg<T, BSrc, 8>(a, lda, bsrc, out, M, N, K, G, st);
    return bi_host::launch_status(what);
  }
  if (M <= kSplitMMax) {
    const bool split = use_split(M, G);
    dim3 grid(ceil_div(N, 16 * WAVES), 1, split ? G : 1);
    if (M <= 16) {
      if (split) gemm_direct<T, BSrc, 1, WAVES, true><<<grid, kWave * WAVES, 0, st>>>(a, lda, bsrc, out, ws, M, N, K, G);
      else gemm_direct<T, BSrc, 1, WAVES, false><<<grid, kWave * WAVES, 0, st>>>(a, lda, bsrc, out, ws, M, N, K, G);
    } else {
      if (split) gemm_direct<T, BSrc, 2, WAVES, true><<<grid, kWave * WAVES, 0, st>>>(a, lda, bsrc, out, ws, M, N, K, G);
      else gemm_direct<T, BSrc, 2, WAVES, false><<<grid, kWave * WAVES, 0, st>>>(a, lda, bsrc, out, ws, M, N, K, G);
    }
    int rc = bi_host::launch_status(what);
    if (rc || !split) return rc;
    const int64_t MN = (int64_t)M * N;
    fold_groups<T><<<(unsigned)((MN + 255) / 256), 256, 0, st>>>(ws, out, MN, G);
    return bi_host::launch_status(what);
  }
  // M > 32: LDS-tiled; the largest tile that still gives the chip >= 256 tiles.
  auto tiles = [&](int bm, int bn) { return (int64_t)ceil_div(M, bm) * ceil_div(N, bn); };
  if constexpr (sizeof(T) == 4) {
    if (tiles(64, 128) >= 256) launch_lds<T, BSrc, 64, 128>(a, lda, bsrc, out, M, N, K, G, st);
    else launch_lds<T, BSrc, 64, 64>(a, lda, bsrc, out, M, N, K, G, st);
  } else {
    if (tiles(128, 128) >= 256) launch_lds<T, BSrc, 128, 128>(a, lda, bsrc, out, M, N, K, G, st);
    else if (tiles(64, 128) >= 256) launch_lds<T, BSrc, 64, 128>(a, lda, bsrc, out, M, N, K, G, st);
    else launch_lds<T, BSrc, 64, 64>(a, lda, bsrc, out, M, N, K, G, st);
  }
  return bi_host::launch_status(what);
}

template <typename T, int BITS, int GS>
int run_quant(const void* x, int64_t ldx, const uint32_t* w, const void* scales,
              const void* biases, void* out, int M, int N, int K, void* ws, hipStream_t st) {
  if constexpr (sizeof(T) == 2) {
    if (bi::qmm_use_big(M, N, K, 2)) {
      // Large M (bi_qmm_big.h): B dequantized and A copied, both in the dense
      // tile's k order, into the caller's workspace; then the dense launch
      // the dense policy picks for the shape (a large-tile form or the
      // unsplit tall tile: qmm_use_big admits no launch that needs more
      // workspace).
      T* bq = static_cast<T*>(ws);
      T* ap = bq + (size_t)N * K;
      const int64_t nb = (int64_t)N * (K / 8), na = (int64_t)M * (K / 8);
      bi::qmm_dequant_rows<T, BITS, GS><<<(unsigned)((nb + 255) / 256), 256, 0, st>>>(
          w, static_cast<const T*>(scales), static_cast<const T*>(biases), bq, N, K);
      bi::qmm_permute_a<T><<<(unsigned)((na + 255) / 256), 256, 0, st>>>(static_cast<const T*>(x), ldx, ap, M, K);
      bi::DenseB<T> db;
      db.bt = bq;
      db.ldb = K;
      db.N = N;
      db.K = K;
      return bi::run_gemm<T, bi::DenseB<T>>(ap, K, db, static_cast<T*>(out), M, N, K, nullptr, st,
                                            "bi_quantized_matmul");
    }
  }
  bi::QuantB<T, BITS, GS> b;
  b.w = w;
  b.scales = static_cast<const T*>(scales);
  b.biases = static_cast<const T*>(biases);
  b.N = N;
  b.K = K;
  b.words_per_row = (int64_t)K * BITS / 32;
  b.groups_per_row = K / GS;
  return bi::run_gemm(static_cast<const T*>(x), ldx, b, static_cast<T*>(out), M, N, K,
                      static_cast<float*>(ws), st, "bi_quantized_matmul");
}

// One thread per (16-row tile, group, MFMA lane): the lane's kWords code
// words and its (scale, bias) pairs copied into the QuantPacked layout.
template <typename T, int BITS, int GS>
__global__ __launch_bounds__(256) void qmm_pack_rows(const uint32_t* __restrict__ w,
                                                     const T* __restrict__ scales,
                                                     const T* __restrict__ biases, char* __restrict__ packed,
                                                     int N, int K) {
  typedef QuantPacked<T, BITS, GS> P;
  const int G = K / kGroupK;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)((N + 15) / 16) * G * kWave) return;
  const int l = (int)(idx % kWave);
  const int64_t tg = idx / kWave;                  // tile * G + group
  const int g = (int)(tg % G);
  const int n = (int)min<int64_t>(tg / G * 16 + l % 16, N - 1);
  const int k0 = g * kGroupK + 64 * (l / 16);
  const uint32_t* src = w + (int64_t)n * ((int64_t)K * BITS / 32) + (int64_t)k0 * BITS / 32;
  char* blk = packed + tg * P::kBlock;
#pragma unroll
  for (int i = 0; i < P::kPieces; ++i)
    *reinterpret_cast<u32x4*>(blk + 1024 * i + 16 * l) = *reinterpret_cast<const u32x4*>(src + 4 * i);
  // Groups of 128: the two lanes of a row that share a pair both write it
  // (the same value).
#pragma unroll
  for (int i = 0; i < P::kScales; ++i) {
    const int64_t si = (int64_t)n * (K / GS) + k0 / GS + i;
    const uint32_t m = (uint32_t)__builtin_bit_cast(uint16_t, scales[si]) |
                       ((uint32_t)__builtin_bit_cast(uint16_t, biases[si]) << 16);
    *reinterpret_cast<uint32_t*>(blk + P::kPieces * 1024 + P::meta_off(l % 16, l / 16) + 4 * i) = m;
  }
}

// The quantized op with an optional repacked copy of B: the streaming GEMV
// reads the copy wherever it takes the shape, every other launch the
// MLX-layout operands, so the bits equal run_quant's at every M.
template <typename T, int BITS, int GS>
int run_quant_packed_gs(const void* x, int64_t ldx, const uint32_t* w, const void* scales, const void* biases,
                        const void* packed, void* out, int M, int N, int K, void* ws, hipStream_t st) {
  if (packed && K % kGroupK == 0 && M > 0) {
    QuantPacked<T, BITS, GS> b;
    b.w = w;
    b.scales = static_cast<const T*>(scales);
    b.biases = static_cast<const T*>(biases);
    b.N = N;
    b.K = K;
    b.words_per_row = (int64_t)K * BITS / 32;
    b.groups_per_row = K / GS;
    b.p = static_cast<const char*>(packed);
    b.G = K / kGroupK;
    const T* a = static_cast<const T*>(x);
    if (launch_stream_packed<T, BITS, GS>(a, ldx, b, static_cast<T*>(out), M, N, K, b.G, st))
      return bi_host::launch_status("bi_quantized_matmul_packed");
    // The mid-M launches read B through the same per-lane interface, so they
    // take the copy too: Llama MLP up [14336, 4096] M = 17 / 32 / 64 17.9-19.2
    // / 18.8-19.8 / 22.2 -> 13.6-14.6 / 14.2-14.9 / 17.8 us, down [4096,
    // 14336] M = 32 / 64 30.4-31.1 / 43.1 -> 24.1-24.3 / 36.1 us, [4096,
    // 4096] M = 32 / 64 15.8-16.1 / 17.8 -> 14.0-14.2 / 16.7 us (same box,
    // bits equal): their per-CU load rate, not the arithmetic, bounds them.
    MidPlan mp = mid_plan(M, N, K);
    // 33-64 rows that the plan splits over K (64-row blocks, fewer than
    // kMidMinTiles of them) run unsplit on the copy as 32-row blocks when that
    // gives at least 128 workgroups: [4096, 4096] / [4096, 8192] / [4096,
    // 14336] M = 64 17.1 / 22.5 / 37.0 -> 12.5 / 19.8 / 31.0 us, M = 48 14.7
    // / 20.0 / 33.0 -> 12.8 / 20.5 / 32.2 us (same box, bits equal: the same
    // group partials, folded in the same order).
    if (mp.use && mp.mt == 4 && mp.chunks > 1 && (int64_t)ceil_div(N, 64) * ceil_div(M, 32) >= 128 &&
        (int64_t)ceil_div(N, 64) * ceil_div(M, 32) <= kMidInterleaveMaxTiles) {
      mp.mt = 2;
      mp.mtiles = ceil_div(M, 32);
      mp.cg = b.G;
      mp.chunks = 1;
    }
    if (use_mid<T, QuantPacked<T, BITS, GS>>(mp, ldx, a)) {
      launch_mid<T, QuantPacked<T, BITS, GS>>(a, ldx, b, static_cast<T*>(out), static_cast<float*>(ws), M, N, K,
                                              b.G, mp, st);
      return bi_host::launch_status("bi_quantized_matmul_packed");
    }
  }
  return run_quant<T, BITS, GS>(x, ldx, w, scales, biases, out, M, N, K, ws, st);
}

template <typename T, int BITS>
int run_quant_packed(int gs, const void* x, int64_t ldx, const uint32_t* w, const void* scales,
                     const void* biases, const void* packed, void* out, int M, int N, int K, void* ws,
                     hipStream_t st) {
  if (gs == 32) return run_quant_packed_gs<T, BITS, 32>(x, ldx, w, scales, biases, packed, out, M, N, K, ws, st);
  if (gs == 64) return run_quant_packed_gs<T, BITS, 64>(x, ldx, w, scales, biases, packed, out, M, N, K, ws, st);
  if (gs == 128) return run_quant_packed_gs<T, BITS, 128>(x, ldx, w, scales, biases, packed, out, M, N, K, ws, st);
  return bi_host::fail(BI_E_UNSUPPORTED, "bi_quantized_matmul_packed: bits=%d group_size=%d", BITS, gs);
}

template <typename T, int BITS, int GS>
int pack_quant(const uint32_t* w, const void* scales, const void* biases, void* packed, int N, int K,
               hipStream_t st) {
  const int64_t n = (int64_t)ceil_div(N, 16) * (K / kGroupK) * kWave;
  qmm_pack_rows<T, BITS, GS><<<(unsigned)((n + 255) / 256), 256, 0, st>>>(
      w, static_cast<const T*>(scales), static_cast<const T*>(biases), static_cast<char*>(packed), N, K);
  return bi_host::launch_status("bi_quantized_pack");
}

template <typename T>
int dispatch_quant(int bits, int gs, const void* x, int64_t ldx, const uint32_t* w,
                   const void* scales, const void* biases, void* out, int M, int N, int K,
                   void* ws, hipStream_t st) {
#define BI_Q(B, G)                                                                       \
  if (bits == B && gs == G)                                                              \
    return run_quant<T, B, G>(x, ldx, w, scales, biases, out, M, N, K, ws, st);
  BI_Q(4, 32) BI_Q(4, 64) BI_Q(4, 128) BI_Q(8, 32) BI_Q(8, 64) BI_Q(8, 128)
#undef BI_Q
  return bi_host::fail(BI_E_UNSUPPORTED, "bi_quantized_matmul: bits=%d group_size=%d", bits, gs);
}

// The same for one bit width (the 2-byte types compile their 4-bit and 8-bit
// kernels in separate translation units, which the build compiles with
// different scheduler options).
template <typename T, int BITS>
int dispatch_quant_bits(int gs, const void* x, int64_t ldx, const uint32_t* w, const void* scales,
                        const void* biases, void* out, int M, int N, int K, void* ws, hipStream_t st) {
  if (gs == 32) return run_quant<T, BITS, 32>(x, ldx, w, scales, biases, out, M, N, K, ws, st);
  if (gs == 64) return run_quant<T, BITS, 64>(x, ldx, w, scales, biases, out, M, N, K, ws, st);
  if (gs == 128) return run_quant<T, BITS, 128>(x, ldx, w, scales, biases, out, M, N, K, ws, st);
  return bi_host::fail(BI_E_UNSUPPORTED, "bi_quantized_matmul: bits=%d group_size=%d", BITS, gs);
}

// Per-element-type entry points of the quantized op (bi_qmm_<dtype>.hip; the
// 8-bit kernels of the 2-byte types in bi_qmm8_<dtype>.hip).
int qmm_bf16(int bits, int gs, const void* x, int64_t ldx, const uint32_t* w, const void* scales,
             const void* biases, void* out, int M, int N, int K, void* ws, hipStream_t st);
int qmm_f16(int bits, int gs, const void* x, int64_t ldx, const uint32_t* w, const void* scales,
            const void* biases, void* out, int M, int N, int K, void* ws, hipStream_t st);
int qmm8_bf16(int gs, const void* x, int64_t ldx, const uint32_t* w, const void* scales, const void* biases,
              void* out, int M, int N, int K, void* ws, hipStream_t st);
int qmm8_f16(int gs, const void* x, int64_t ldx, const uint32_t* w, const void* scales, const void* biases,
             void* out, int M, int N, int K, void* ws, hipStream_t st);
int qmm_f32(int bits, int gs, const void* x, int64_t ldx, const uint32_t* w, const void* scales,
            const void* biases, void* out, int M, int N, int K, void* ws, hipStream_t st);
// The op with a repacked copy (run_quant_packed; bi_qmm_<dtype>.hip, the
// 8-bit kernels in bi_qmm8_<dtype>.hip) and the packing (pack_quant).
int qmm_packed_bf16(int bits, int gs, const void* x, int64_t ldx, const uint32_t* w, const void* scales,
                    const void* biases, const void* packed, void* out, int M, int N, int K, void* ws,
                    hipStream_t st);
int qmm_packed_f16(int bits, int gs, const void* x, int64_t ldx, const uint32_t* w, const void* scales,
                   const void* biases, const void* packed, void* out, int M, int N, int K, void* ws,
                   hipStream_t st);
int qmm8_packed_bf16(int gs, const void* x, int64_t ldx, const uint32_t* w, const void* scales,
                     const void* biases, const void* packed, void* out, int M, int N, int K, void* ws,
                     hipStream_t st);
int qmm8_packed_f16(int gs, const void* x, int64_t ldx, const uint32_t* w, const void* scales,
                    const void* biases, const void* packed, void* out, int M, int N, int K, void* ws,
                    hipStream_t st);

}  // namespace bi
