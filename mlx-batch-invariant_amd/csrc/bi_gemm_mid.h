// bi_gemm_mid.h — the mid-M launch (4 < M < 256, quantized B): every weight
// element of a workgroup's column block and K chunk is read from HBM once and
// dequantized once, then used for all of the block's rows.
//
// Same arithmetic as every other launch (bi_gemm_tile.h: the B source's k-slot
// map, eight MFMA steps per 256-k group from zero, total = total + acc in group
// order).
//
// One 256-thread workgroup per 64 output columns, 16 MT rows and a chunk of CG
// consecutive 256-k groups; wave w owns columns 16 w .. 16 w + 15 of the block.
// Per group g of the chunk:
//   * A rows [m0, m0 + 16 MT) x k [256 g, 256 g + 256) sit in a ring of NA LDS
//     buffers, copied by the load unit (global_load_lds_dwordx4, two 512-byte
//     rows per instruction; 16-byte chunk c of row r in slot c ^ (r & 15), so
//     the 16 rows of a fragment read hit 16 distinct slots). Group g + NA - 1
//     is requested right after the barrier that opens group g.
//   * each wave's B operand (codes + scale/bias for a quantized B, the bf16/
//     fp16 rows for a dense one) goes global -> registers PD groups ahead and
//     is converted once per step, then multiplied with the MT A fragments.
// With one chunk (CG = G) the group fold stays in registers and the kernel
// writes the output; with several (SPLIT) every group's raw fp32 partial goes
// to part[g][M][N] and fold_groups adds them in group order afterwards, so the
// bits are the same either way. Splitting K only adds workgroups: it is the
// launch's answer to too few column blocks (N <= 4096) to fill the chip.
// Requirements (host policy): 2-byte T, K % 256 == 0, lda % 8 == 0, a 16-byte
// aligned. Rows past M are clamped to row M - 1 (never stored); columns past N
// to column N - 1 (never stored).
#pragma once

#include "bi_gemm_tile.h"

namespace bi {

template <typename T, int MT, int NA>
struct MidCfg {
  static constexpr int kRows = 16 * MT;
  static constexpr int kRowBytes = kGroupK * (int)sizeof(T);      // 512
  static constexpr int kRowsPerCopy = 1024 / kRowBytes;            // 2
  static constexpr int kCopies = kRows / kRowsPerCopy;             // per group
  static constexpr int kCopiesPerWave = kCopies / 4;
  static constexpr int kBufBytes = kRows * kRowBytes;
  static constexpr int kRing = NA;                                 // A groups in LDS
  static_assert(sizeof(T) == 2, "gemm_mid: 2-byte element types only");
  static_assert(kCopies % 4 == 0, "gemm_mid: copies must split over 4 waves");
  static_assert(kRing >= 2 && kRing * kBufBytes <= 160 * 1024, "gemm_mid: 2 or more A buffers within LDS");
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
// The repacked B: its code pieces and one load of the lane's (scale, bias) pairs.
template <typename T, int BITS, int GS> struct MidLoads<QuantPacked<T, BITS, GS>> {
  static constexpr int kMin = QuantPacked<T, BITS, GS>::kPieces + 1;
};

// The A ring lives in one __shared__ array per slot, and every access names
// its slot by a compile-time index: a DS read of one slot then provably does
// not alias the LDS copies still landing in the others, so the compiler waits
// only for the counts the kernel asks for (one array indexed by a run-time
// slot made it wait for every outstanding copy and B load before each
// group's first read, which serialised the prefetch with the compute).
#define BI_MID_SLOT(i, BYTES) __shared__ __attribute__((aligned(1024))) char ring##i[NA > i ? (BYTES) : 16];
#define BI_MID_SLOTS(BYTES)                                                                              \
  BI_MID_SLOT(0, BYTES) BI_MID_SLOT(1, BYTES) BI_MID_SLOT(2, BYTES) BI_MID_SLOT(3, BYTES)            \
  BI_MID_SLOT(4, BYTES) BI_MID_SLOT(5, BYTES) BI_MID_SLOT(6, BYTES) BI_MID_SLOT(7, BYTES)            \
  auto slot = [&](int s_) -> char* {                                                                     \
    switch (s_) {                                                                                        \
      case 0: return ring0; case 1: return ring1; case 2: return ring2; case 3: return ring3;            \
      case 4: return ring4; case 5: return ring5; case 6: return ring6; default: return ring7;           \
    }                                                                                                    \
  };

// The eight MFMA steps of one group for the MT row blocks: the B fragment of
// step s dequantized from the raw registers, the A fragments read from LDS one
// step ahead of their MFMAs, so the reads of step s + 1 are in flight while
// step s multiplies (Llama MLP shape, 4-bit g64, M = 64: 24.2 -> 22.7 us).
template <class C, int MT, bool FAST, class BSrc>
__device__ __forceinline__ void mid_group_steps(const BSrc& bsrc, const typename BSrc::Raw& raw, const char* buf,
                                                int gc, int q, int kq, int r, f32x4 (&acc)[MT]) {
  typedef typename BSrc::F F;
  F af[2][MT];
  auto read_a = [&](int s, F (&dst)[MT]) {
    const int ch = (BSrc::a_k(gc, q, s) - gc * kGroupK) / 8;
#pragma unroll
    for (int i = 0; i < MT; ++i) dst[i] = *reinterpret_cast<const F*>(buf + C::off(16 * i + r, ch));
  };
  read_a(0, af[0]);
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const F bf = bsrc.template frag<true, FAST>(raw, s, kq);
    if (s + 1 < kSteps) read_a(s + 1, af[(s + 1) & 1]);
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = mfma_step(af[s & 1][i], bf, acc[i]);
  }
}

template <typename T, class BSrc, int MT, int PD, int NA, bool SPLIT>
__global__ __launch_bounds__(256) void gemm_mid(const T* a, int64_t lda, BSrc bsrc, T* __restrict__ out,
                                                float* __restrict__ part, int M, int N, int K, int G, int CG) {
  typedef MidCfg<T, MT, NA> C;
  // Outstanding vector-memory instructions that are certainly issued after
  // the copies of group g when its barrier is reached (copies of NA - 2 later
  // groups and at least min(PD, NA - 1) groups of B loads): waiting down to
  // this count lands group g (they complete in issue order). Every copy and
  // load below is issued unconditionally (past the last group they repeat
  // it), so the count holds at every group. Capped at the counter's 63: a
  // smaller count only waits longer.
  constexpr int kAfter = (NA - 2) * C::kCopiesPerWave + (PD < NA - 1 ? PD : NA - 1) * MidLoads<BSrc>::kMin;
  constexpr int kWaitA = kAfter < 63 ? kAfter : 63;
  // Groups run in unrolled rounds of U: slot (group mod NA) and B registers
  // (group mod PD) are then compile-time indices.
  constexpr int U = PD > NA ? PD : NA;
  static_assert(NA <= 8 && U % PD == 0 && U % NA == 0, "gemm_mid: PD and NA powers of two, NA <= 8");
  BI_MID_SLOTS(C::kBufBytes)

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int r = lane % 16, q = lane / 16;
  const int m0 = blockIdx.y * C::kRows;
  const int n_out = blockIdx.x * 64 + 16 * wave + r;
  const int n = min(n_out, N - 1);
  const typename BSrc::Lane bl = bsrc.lane(n, q);
  const int gb = blockIdx.z * CG;             // the chunk's first group
  const int gn = min(CG, G - gb);             // and its group count (>= 1)

  auto copy_a = [&](int j, int sl) {  // chunk group min(j, gn - 1) into slot sl = j % NA
    char* buf = slot(sl);
    const int gg = gb + min(j, gn - 1);
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
  for (int g = 0; g < NA - 1; ++g) copy_a(g, g);
  // One fence per group keeps the loads in group order: the scheduler would
  // otherwise batch all codes before all scales, leaving group 0's last, and
  // the wait counts at the loop head would collapse to zero.
#pragma unroll
  for (int j = 0; j < PD; ++j) {
    asm volatile("" ::: "memory");
    bsrc.load_full(raw[j], bl, gb + min(j, gn - 1));
  }
  asm volatile("" ::: "memory");

  // One chunk group l (u = l mod U): wait for its A, request A of group
  // l + NA - 1, compute, fold (or store the partial), request B of group
  // l + PD into the registers it released.
  auto group = [&](int l, int u) {
    const int j = u % PD;
    // Group l's A landed for every wave; every wave is past group l - 1,
    // whose buffer now takes group l + NA - 1.
    stage_barrier<kWaitA>();
    copy_a(l + NA - 1, (u + NA - 1) % NA);
    asm volatile("" ::: "memory");
    const char* buf = slot(u % NA);
    f32x4 acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int gc = gb + min(l, gn - 1);
    const int kq = BSrc::kbase(gc, q);
    auto steps = [&](auto fast) {
      mid_group_steps<C, MT, decltype(fast)::value>(bsrc, raw[j], buf, gc, q, kq, r, acc);
    };
    if (!__any(bsrc.huge_scale(raw[j]))) steps(std::true_type());
    else steps(std::false_type());
    const bool live = l < gn;
    if constexpr (SPLIT) {
      if (live && n_out < N) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int m = m0 + 16 * i + 4 * q + e;
            if (m < M) part[((int64_t)gc * M + m) * N + n_out] = acc[i][e];
          }
      }
    } else {
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const f32x4 t = total[i] + acc[i];
        total[i] = live ? t : total[i];
      }
    }
    asm volatile("" ::: "memory");
    bsrc.load_full(raw[j], bl, gb + min(l + PD, gn - 1));
    asm volatile("" ::: "memory");
  };
  // A whole number of U-group rounds (padding groups recompute the last group
  // and are not folded), the first one peeled: the loop body then has no
  // branch around memory instructions and the loop is entered from a state
  // shaped like its own back edge, so the compiler's wait counts stay exact.
  const int Gp = (gn + U - 1) / U * U;
#pragma unroll
  for (int u = 0; u < U; ++u) group(u, u);
  for (int l0 = U; l0 < Gp; l0 += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) group(l0 + u, u);
  }
  // The ring's last requests (past the chunk they repeat its last group) are
  // still in flight: drain them before the workgroup's LDS can be reused.
  wait_vm_lgkm0<0>();

  if (!SPLIT && n_out < N) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 16 * i + 4 * q + e;
        if (m < M) out[(int64_t)m * N + n_out] = to_store<T>(total[i][e]);
      }
  }
}


// K-interleaved variant (512 threads): wave w owns columns 16 (w % 4) .. + 15
// of the block and the chunk's groups of parity w / 4, so two waves share each
// SIMD and one's dequantisation overlaps the other's MFMAs. Ring stage t holds
// A of groups 2t and 2t + 1; the odd wave's raw fp32 partial of stage t goes
// to a double-buffered LDS slot and the even wave folds the stage at the next
// barrier: total = (total + acc_2t) + acc_2t+1, the same left fold in group
// order as gemm_mid (SPLIT: every wave stores its own partials).
template <typename T, class BSrc, int MT, int PD, int NA, bool SPLIT>
__global__ __launch_bounds__(512) void gemm_mid2(const T* a, int64_t lda, BSrc bsrc, T* __restrict__ out,
                                                 float* __restrict__ part, int M, int N, int K, int G, int CG) {
  typedef MidCfg<T, MT, NA> C;  // one group's A buffer; a stage holds two
  constexpr int kCopiesPerWave = C::kCopies / 4;  // two groups' copies over eight waves
  // As in gemm_mid: vector-memory instructions certainly issued after a
  // stage's copies when its barrier is reached (copies of NA - 2 later stages
  // and at least min(PD, NA - 1) stages of this wave's B loads).
  constexpr int kAfter = (NA - 2) * kCopiesPerWave + (PD < NA - 1 ? PD : NA - 1) * MidLoads<BSrc>::kMin;
  constexpr int kWaitA = kAfter < 63 ? kAfter : 63;
  constexpr int U = PD > NA ? PD : NA;  // stages per unrolled round
  static_assert(NA <= 8 && U % PD == 0 && U % NA == 0, "gemm_mid2: PD and NA powers of two, NA <= 8");
  BI_MID_SLOTS(2 * C::kBufBytes)        // slot s: groups 2t, 2t + 1 of a stage t = s mod NA
  __shared__ __attribute__((aligned(16))) f32x4 xbuf[2][4][MT][kWave];
  static_assert(NA * 2 * C::kBufBytes + sizeof(xbuf) <= 160 * 1024, "gemm_mid2: LDS");

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int cw = wave & 3, par = wave >> 2;
  const int r = lane % 16, q = lane / 16;
  const int m0 = blockIdx.y * C::kRows;
  const int n_out = blockIdx.x * 64 + 16 * cw + r;
  const int n = min(n_out, N - 1);
  const typename BSrc::Lane bl = bsrc.lane(n, q);
  const int gb = blockIdx.z * CG;           // the chunk's first group
  const int gn = min(CG, G - gb);           // its group count (>= 1)
  const int ns = (gn + 1) / 2;              // stages

  auto copy_stage = [&](int t, int sl) {  // groups 2t, 2t + 1 (clamped to the chunk) into slot sl = t % NA
#pragma unroll
    for (int i = 0; i < kCopiesPerWave; ++i) {
      const int ci = wave * kCopiesPerWave + i;
      const int h = ci / C::kCopies, cl = ci % C::kCopies;
      const int gg = gb + min(2 * t + h, gn - 1);
      const int row = cl * C::kRowsPerCopy + lane / (C::kRowBytes / 16);
      const int ch = (lane % (C::kRowBytes / 16)) ^ (row & 15);
      copy_to_lds16(a + (int64_t)min(m0 + row, M - 1) * lda + gg * kGroupK + 8 * ch,
                    slot(sl) + h * C::kBufBytes + 1024 * cl);
    }
  };

  f32x4 total[MT], held[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) total[i] = held[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  typename BSrc::Raw raw[PD];
#pragma unroll
  for (int t = 0; t < NA - 1; ++t) copy_stage(t, t);
#pragma unroll
  for (int j = 0; j < PD; ++j) {
    asm volatile("" ::: "memory");
    bsrc.load_full(raw[j], bl, gb + min(2 * j + par, gn - 1));
  }
  asm volatile("" ::: "memory");

  // Even waves: fold stage tp (its own partial, kept in `held`, then the odd
  // wave's from LDS). Runs after a barrier that follows the odd wave's write.
  auto fold_stage = [&](int tp) {
    if constexpr (!SPLIT) {
      if (par == 0 && tp >= 0 && tp < ns) {
#pragma unroll
        for (int i = 0; i < MT; ++i) total[i] = total[i] + held[i];
        if (2 * tp + 1 < gn) {
#pragma unroll
          for (int i = 0; i < MT; ++i) total[i] = total[i] + xbuf[tp & 1][cw][i][lane];
        }
      }
    }
  };

  auto stage = [&](int t, int u) {  // u = t mod U
    const int j = u % PD;
    stage_barrier<kWaitA>();
    fold_stage(t - 1);
    copy_stage(t + NA - 1, (u + NA - 1) % NA);
    asm volatile("" ::: "memory");
    const char* buf = slot(u % NA) + par * C::kBufBytes;
    f32x4 acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int gl = min(2 * t + par, gn - 1);
    const int gc = gb + gl;
    const int kq = BSrc::kbase(gc, q);
    auto steps = [&](auto fast) {
      mid_group_steps<C, MT, decltype(fast)::value>(bsrc, raw[j], buf, gc, q, kq, r, acc);
    };
    if (!__any(bsrc.huge_scale(raw[j]))) steps(std::true_type());
    else steps(std::false_type());
    if constexpr (SPLIT) {
      if (2 * t + par < gn && n_out < N) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int m = m0 + 16 * i + 4 * q + e;
            if (m < M) part[((int64_t)gc * M + m) * N + n_out] = acc[i][e];
          }
      }
    } else {
      if (par == 0) {
#pragma unroll
        for (int i = 0; i < MT; ++i) held[i] = acc[i];
      } else {
#pragma unroll
        for (int i = 0; i < MT; ++i) xbuf[t & 1][cw][i][lane] = acc[i];
      }
    }
    asm volatile("" ::: "memory");
    bsrc.load_full(raw[j], bl, gb + min(2 * (t + PD) + par, gn - 1));
    asm volatile("" ::: "memory");
  };
  const int Sp = (ns + U - 1) / U * U;
#pragma unroll
  for (int u = 0; u < U; ++u) stage(u, u);
  for (int t0 = U; t0 < Sp; t0 += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) stage(t0 + u, u);
  }
  wait_vm_lgkm0<0>();   // every copy landed and the odd waves' last partials are written
  __syncthreads();
  // Stages 0 .. Sp - 2 were folded at the start of the next stage; the last
  // one here (a padding stage folds nothing: its predecessor ns - 1 < Sp - 1
  // was folded inside the loop).
  fold_stage(Sp - 1);

  if (!SPLIT && par == 0 && n_out < N) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 16 * i + 4 * q + e;
        if (m < M) out[(int64_t)m * N + n_out] = to_store<T>(total[i][e]);
      }
  }
}

#undef BI_MID_SLOTS
#undef BI_MID_SLOT

}  // namespace bi
