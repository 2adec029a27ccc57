// bi_gemm_mid.h — the mid-M launch (4 < M <= 64): every weight element is
// read from HBM once and (for a quantized B) dequantized once, then used for
// all M rows.
//
// Same arithmetic as every other launch (bi_gemm_tile.h: the B source's k-slot
// map, eight MFMA steps per 256-k group from zero, total = total + acc in group
// order).
//
// One 256-thread workgroup per 64 output columns and up to 16 MT rows; wave w
// owns columns 16 w .. 16 w + 15 of the block for the whole of K, so the group
// fold stays in registers. Per group g:
//   * A rows [m0, m0 + 16 MT) x k [256 g, 256 g + 256) sit in a ring of NA LDS
//     buffers (8 groups for MT <= 2, 4 for MT = 4), copied by the
//     load unit (global_load_lds_dwordx4, two 512-byte rows per instruction;
//     16-byte chunk c of row r in slot c ^ (r & 15), so the 16 rows of a
//     fragment read hit 16 distinct slots). Group g + NA - 1 is requested
//     right after the barrier that opens group g.
//   * each wave's B operand (codes + scale/bias for a quantized B, the bf16/
//     fp16 rows for a dense one) goes global -> registers PD groups ahead and
//     is converted once per step, then multiplied with the MT A fragments.
// Requirements (host policy): 2-byte T, K % 256 == 0, lda % 8 == 0, a 16-byte
// aligned. Rows past M are clamped to row M - 1 (never stored); columns past N
// to column N - 1 (never stored).
#pragma once

#include "bi_gemm_tile.h"

namespace bi {

template <typename T, int MT>
struct MidCfg {
  static constexpr int kRows = 16 * MT;
  static constexpr int kRowBytes = kGroupK * (int)sizeof(T);      // 512
  static constexpr int kRowsPerCopy = 1024 / kRowBytes;            // 2
  static constexpr int kCopies = kRows / kRowsPerCopy;             // per group
  static constexpr int kCopiesPerWave = kCopies / 4;
  static constexpr int kBufBytes = kRows * kRowBytes;
  static constexpr int kRing = (128 * 1024 / kBufBytes) < 8 ? (128 * 1024 / kBufBytes) : 8;  // A groups in LDS
  static_assert(sizeof(T) == 2, "gemm_mid: 2-byte element types only");
  static_assert(kCopies % 4 == 0, "gemm_mid: copies must split over 4 waves");
  static_assert(kRing >= 2, "gemm_mid: at least two A buffers");
  static __device__ __forceinline__ int off(int r, int c) { return r * kRowBytes + ((c ^ (r & 15)) << 4); }
};

// Lower bound on the vector-memory instructions one load_full issues (each
// 16-byte piece of codes or dense rows is its own instruction; scales and
// biases are at least one each).
template <class BSrc> struct MidLoads;
template <typename T> struct MidLoads<DenseB<T>> { static constexpr int kMin = kSteps; };
template <typename T, int BITS, int GS> struct MidLoads<QuantB<T, BITS, GS>> {
  static constexpr int kMin = QuantB<T, BITS, GS>::kWords / 4 + 2;
};

template <typename T, class BSrc, int MT, int PD>
__global__ __launch_bounds__(256) void gemm_mid(const T* a, int64_t lda, BSrc bsrc, T* __restrict__ out,
                                                int M, int N, int K, int G) {
  typedef MidCfg<T, MT> C;
  typedef typename Frag<T>::type F;
  constexpr int NA = C::kRing;
  // Outstanding vector-memory instructions that are certainly issued after
  // the copies of group g when its barrier is reached (copies of NA - 2 later
  // groups and at least min(PD, NA - 1) groups of B loads): waiting down to
  // this count lands group g (they complete in issue order). Every copy and
  // load below is issued unconditionally (past the last group they repeat
  // it), so the count holds at every group. Capped at the counter's 63: a
  // smaller count only waits longer.
  constexpr int kAfter = (NA - 2) * C::kCopiesPerWave + (PD < NA - 1 ? PD : NA - 1) * MidLoads<BSrc>::kMin;
  constexpr int kWaitA = kAfter < 63 ? kAfter : 63;
  __shared__ __attribute__((aligned(1024))) char As[NA][C::kBufBytes];

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int r = lane % 16, q = lane / 16;
  const int m0 = blockIdx.y * C::kRows;
  const int n_out = blockIdx.x * 64 + 16 * wave + r;
  const int n = min(n_out, N - 1);
  const typename BSrc::Lane bl = bsrc.lane(n, q);

  auto copy_a = [&](int g) {  // group min(g, G - 1) into buffer g % NA
    char* buf = As[g % NA];
    const int gg = min(g, G - 1);
#pragma unroll
    for (int i = 0; i < C::kCopiesPerWave; ++i) {
      const int ci = wave * C::kCopiesPerWave + i;
      const int row = ci * C::kRowsPerCopy + lane / (C::kRowBytes / 16);
      const int ch = (lane % (C::kRowBytes / 16)) ^ (row & 15);
      copy_to_lds16(a + (int64_t)min(m0 + row, M - 1) * lda + gg * kGroupK + 8 * ch, buf + 1024 * ci);
    }
  };

  f32x4 total[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) total[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  typename BSrc::Raw raw[PD];
  // Prologue: A of groups 0 .. NA - 2, then B of groups 0 .. PD - 1.
#pragma unroll
  for (int g = 0; g < NA - 1; ++g) copy_a(g);
  // One fence per group keeps the loads in group order: the scheduler would
  // otherwise batch all codes before all scales, leaving group 0's last, and
  // the wait counts at the loop head would collapse to zero.
#pragma unroll
  for (int j = 0; j < PD; ++j) {
    asm volatile("" ::: "memory");
    bsrc.load_full(raw[j], bl, min(j, G - 1));
  }
  asm volatile("" ::: "memory");

  // One group: wait for its A, request A of group g + NA - 1, compute, fold,
  // request B of group g + PD into the registers it released.
  auto group = [&](int g, int j) {
    // Group g's A landed for every wave; every wave is past group g - 1,
    // whose buffer now takes group g + NA - 1.
    stage_barrier<kWaitA>();
    copy_a(g + NA - 1);
    asm volatile("" ::: "memory");
    const char* buf = As[g % NA];
    f32x4 acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int gc = min(g, G - 1);
    const int kq = BSrc::kbase(gc, q);
    auto steps = [&](auto fast) {
#pragma unroll
      for (int s = 0; s < kSteps; ++s) {
        const int ch = (BSrc::a_k(gc, q, s) - gc * kGroupK) / 8;
        const F bf = bsrc.template frag<true, decltype(fast)::value>(raw[j], s, kq);
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          const F af = *reinterpret_cast<const F*>(buf + C::off(16 * i + r, ch));
          acc[i] = mfma_step(af, bf, acc[i]);
        }
      }
    };
    if (!__any(bsrc.huge_scale(raw[j]))) steps(std::true_type());
    else steps(std::false_type());
    const bool live = g < G;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const f32x4 t = total[i] + acc[i];
      total[i] = live ? t : total[i];
    }
    asm volatile("" ::: "memory");
    bsrc.load_full(raw[j], bl, min(g + PD, G - 1));
    asm volatile("" ::: "memory");
  };
  // A whole number of PD-group rounds (padding groups recompute the last group
  // and are not folded), the first one peeled: the loop body then has no
  // branch around memory instructions and the loop is entered from a state
  // shaped like its own back edge, so the compiler's wait counts stay exact.
  const int Gp = (G + PD - 1) / PD * PD;
#pragma unroll
  for (int j = 0; j < PD; ++j) group(j, j);
  for (int g0 = PD; g0 < Gp; g0 += PD) {
#pragma unroll
    for (int j = 0; j < PD; ++j) group(g0 + j, j);
  }

  if (n_out < N) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 16 * i + 4 * q + e;
        if (m < M) out[(int64_t)m * N + n_out] = to_store<T>(total[i][e]);
      }
  }
}

}  // namespace bi
