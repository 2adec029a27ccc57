// bi_gemv_stream.h — the decode GEMV for an affine-quantized B with no
// workgroup-wide staging barrier before compute.
//
// Same arithmetic as every other quantized launch (bi_gemm_tile.h, blocked
// k-slot map; each group's raw fp32 partial, then the ordered fold).
//
// One workgroup of W waves per 16 output columns; wave w owns the NB
// consecutive groups [w NB, w NB + NB). Each wave requests, in this order:
//   * its slice of A (MR rows x NB * 256 k, 16-byte loads),
//   * its slice of the scales and biases (16 rows x NB * 256 / GS each;
//     consecutive groups make every row's slice contiguous),
//   * the codes of its NB groups (two 16-byte loads per group and lane for
//     4-bit),
// then writes A and the scales/biases into a wave-private LDS region (DS
// operations of one wave complete in order, so no barrier is needed to read
// them back) and computes its groups as their codes arrive. Code loads run at
// most PD groups ahead of compute: with every group requested up front, a
// wave's loads arrive scattered over the whole weight stream and its compute
// only starts near the end; a bounded depth keeps each wave's requests close
// together in the memory queues. Issuing the code loads only after A and the
// metadata have landed measured slower (the weight stream starts later). The
// only barrier is the one before the fold.
// A workgroup-wide staging barrier made every wave wait for the slowest of
// its workgroup's metadata loads, which arrive among the whole weight stream;
// here a wave waits only for its own.
//
// LDS (dynamic), per wave: A [MR][NB * 256], scales [16][SPR], biases
// [16][SPR] (SPR = NB * 256 / GS); once the wave has computed its groups, the
// same region holds its NB raw fp32 partials (64 lanes x f32x4 each), which
// the fold reads after the barrier. A's 8-element
// chunk c of row r sits in slot c ^ (r & 15) of its row, so the 16 rows of a
// fragment read (same chunk, row stride a multiple of 256 bytes) hit 16
// distinct bank groups instead of one.
//
// AG (A from global memory): for rows x K of A too large for LDS, no A slice
// is staged; each group's eight A fragments are loaded into registers with
// the group's codes (PD groups ahead), so the LDS holds only the metadata and
// the partials and several workgroups share a CU. Same values in the same
// MFMA steps, so the same bits.
#pragma once

#include <type_traits>

#include "bi_gemm_tile.h"

namespace bi {

// Group size of a B source's per-group metadata staged in LDS; 0 for a dense B
// (none) and for a repacked quantized B, whose metadata arrive with its codes
// (kRegMeta: then checked for huge scales in registers). kPadK: B is zero past
// K within its last group (a repacked dense B, zero-filled to whole groups), so
// K need not be a multiple of 256; A's elements past K are then loaded as zero,
// as every other launch's partial last group has them.
template <class BSrc> struct StreamMeta {
  static constexpr int kGS = 0;
  static constexpr bool kRegMeta = false;
  static constexpr bool kPadK = false;
};
template <typename T, int BITS, int GS> struct StreamMeta<QuantB<T, BITS, GS>> {
  static constexpr int kGS = GS;
  static constexpr bool kRegMeta = false;
  static constexpr bool kPadK = false;
};
template <typename T, int BITS, int GS> struct StreamMeta<QuantPacked<T, BITS, GS>> {
  static constexpr int kGS = 0;
  static constexpr bool kRegMeta = true;
  static constexpr bool kPadK = false;
};
template <typename T> struct StreamMeta<DensePacked<T>> {
  static constexpr int kGS = 0;
  static constexpr bool kRegMeta = false;
  static constexpr bool kPadK = true;
};

template <typename T, int GS, int W, int NB, int MR, int CT = 1, bool AG = false>
struct GemvStreamCfg {
  static constexpr int kCE = 16 / (int)sizeof(T);            // elements per 16-byte load
  static constexpr int kSPR = GS > 0 ? NB * kGroupK / GS : 0; // scales per row per wave (GS = 0: dense B)
  static constexpr int kRows = 16 * CT;                       // weight rows (output columns) per workgroup
  static constexpr int kAElems = AG ? 0 : MR * NB * kGroupK;  // A elements per wave staged in LDS
  static constexpr int kALoads = kAElems / kCE / kWave;       // A loads per lane
  static constexpr int kMChunks = 2 * kRows * kSPR / kCE;     // meta chunks per wave
  static constexpr int kMLoads = (kMChunks + kWave - 1) / kWave;
  static constexpr int kWaveElems = kAElems + 2 * kRows * kSPR;  // A + metadata elements per wave
  // Bytes per wave region: A and metadata, or later the NB x CT partials.
  static constexpr int kWaveBytes = (kWaveElems * (int)sizeof(T) > NB * CT * kWave * 16)
                                        ? kWaveElems * (int)sizeof(T) : NB * CT * kWave * 16;
  static constexpr int kRowElems = NB * kGroupK;               // A row of the wave's slice
  // LDS element offset of A element k (0 <= k < kRowElems) of slice row ar.
  static __device__ __forceinline__ int a_off(int ar, int k) {
    return ar * kRowElems + ((((k >> 3) ^ (ar & 15))) << 3) + (k & 7);
  }
  static_assert(sizeof(T) == 2, "gemv_stream: 2-byte element types only (16-byte pieces = one fragment)");
  static_assert(kAElems % (kCE * kWave) == 0, "A slice must be whole 16-byte loads per lane");
  static_assert(kSPR % kCE == 0, "scale rows must be whole 16-byte chunks");
  static constexpr size_t kLdsBytes = (size_t)W * kWaveBytes;
  static size_t lds_bytes(int /*G*/) { return kLdsBytes; }
};

template <typename T, class BSrc, int W, int NB, int MR, int PD, int CT = 1, bool AG = false>
__global__ __launch_bounds__(kWave* W) void gemv_stream(const T* a, int64_t lda, BSrc bsrc,
                                                        T* __restrict__ out, int M, int N, int K,
                                                        int G) {
  constexpr int GS = StreamMeta<BSrc>::kGS;
  typedef GemvStreamCfg<T, GS, W, NB, MR, CT, AG> C;
  typedef BSrc QB;
  typedef typename Frag<T>::type F;
  extern __shared__ __attribute__((aligned(16))) f32x4 smem[];
  char* regions = reinterpret_cast<char*>(smem);                   // W x kWaveBytes
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  T* As = reinterpret_cast<T*>(regions + (size_t)wave * C::kWaveBytes);
  T* Ms = As + C::kAElems;                                          // [2][kRows][SPR]
  const int r = lane % 16, q = lane / 16;
  const int n_base = blockIdx.x * C::kRows;
  const int g0 = wave * NB;                      // G == W * NB (checked on the host)

  // 1. A slice: row ar, elements [g0 * 256 + ac, +kCE) of the wave's slice.
  F av[C::kALoads > 0 ? C::kALoads : 1];
#pragma unroll
  for (int i = 0; i < C::kALoads; ++i) {
    const int c = lane + kWave * i;
    const int ar = c / (NB * kGroupK / C::kCE), ac = (c % (NB * kGroupK / C::kCE)) * C::kCE;
    const int kk = g0 * kGroupK + ac;
    if constexpr (StreamMeta<BSrc>::kPadK) {
      const bool ok = kk < K;                      // K % 8 == 0: a chunk lies wholly before or past K
      const F v = frag_load(a + (ok ? (int64_t)min(ar, M - 1) * lda + kk : 0));
      av[i] = ok ? v : frag_zero<F>();
    } else {
      av[i] = frag_load(a + (int64_t)min(ar, M - 1) * lda + kk);
    }
  }
  // 2. Scales then biases of rows n_base .. n_base + kRows - 1 for the wave's
  // groups (a quantized B; a dense one has none).
  F mv[C::kMLoads > 0 ? C::kMLoads : 1];
  if constexpr (GS > 0) {
    const int gpr = (int)bsrc.groups_per_row;
#pragma unroll
    for (int i = 0; i < C::kMLoads; ++i) {
      const int c0 = lane + kWave * i;
      const int c = c0 < C::kMChunks ? c0 : 0;
      const int kind = c / (C::kRows * C::kSPR / C::kCE);
      const int within = c % (C::kRows * C::kSPR / C::kCE);
      const int row = within / (C::kSPR / C::kCE), col = (within % (C::kSPR / C::kCE)) * C::kCE;
      const T* base = kind ? bsrc.biases : bsrc.scales;
      mv[i] = frag_load(base + (int64_t)min(n_base + row, N - 1) * gpr + g0 * (kGroupK / GS) + col);
    }
  }
  // 3. Codes of the wave's first PD groups (CT column tiles: weight rows
  // n_base + 16 c + r, clamped; padding columns are not stored), after
  // everything above in issue order; group j + PD is requested when group j
  // starts.
  asm volatile("" ::: "memory");
  // A group's B operand: the codes of a quantized B (its scales and biases
  // come from LDS), all eight fragments of a dense one.
  auto load_b = [&](typename QB::Raw& raw, const typename QB::Lane& l, int g) {
    if constexpr (GS > 0) bsrc.load_codes(raw, l, g);
    else bsrc.load_full(raw, l, g);
  };
  // AG: A's fragments of a group go straight from global memory (L2) to
  // registers, requested with the group's codes (PD groups ahead), instead of
  // the MR rows x K of A staged in LDS.
  constexpr int kAR = AG ? (PD < NB ? PD + 1 : NB) : 1;
  F areg[kAR][AG ? kSteps : 1];
  const T* arowp = a + (int64_t)min(r, M - 1) * lda;
  auto load_a = [&](int j) {
    if constexpr (AG) {
#pragma unroll
      for (int s = 0; s < kSteps; ++s) {
        const int kk = QB::a_k(g0 + j, q, s);
        if constexpr (StreamMeta<BSrc>::kPadK) {
          const bool ok = kk < K;
          const F v = frag_load(ok ? arowp + kk : a);
          areg[j % kAR][s] = ok ? v : frag_zero<F>();
        } else {
          areg[j % kAR][s] = frag_load(arowp + kk);
        }
      }
    }
  };
  typename QB::Raw braw[NB][CT];
  typename QB::Lane bl[CT];
  int rt[CT];                                     // the lanes' rows of the staged metadata
#pragma unroll
  for (int c = 0; c < CT; ++c) {
    const int n = min(n_base + 16 * c + r, N - 1);
    bl[c] = bsrc.lane(n, q);
    rt[c] = n - n_base;
  }
#pragma unroll
  for (int j = 0; j < PD && j < NB; ++j) {
    load_a(j);
#pragma unroll
    for (int c = 0; c < CT; ++c) load_b(braw[j][c], bl[c], g0 + j);
  }
  // Wave-private LDS: written and read back by this wave only.
#pragma unroll
  for (int i = 0; i < C::kALoads; ++i) {
    const int c = lane + kWave * i;
    const int ar = c / (NB * kGroupK / C::kCE), ac = (c % (NB * kGroupK / C::kCE)) * C::kCE;
    *reinterpret_cast<F*>(As + C::a_off(ar, ac)) = av[i];
  }
#pragma unroll
  for (int i = 0; i < C::kMLoads; ++i) {
    const int c = lane + kWave * i;
    if (c < C::kMChunks) *reinterpret_cast<F*>(Ms + c * C::kCE) = mv[i];
  }
  asm volatile("" ::: "memory");

  const int arow = min(r, MR - 1);                // A rows past MR alias a loaded row (never stored)
  f32x4 accs[NB][CT];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int g = g0 + j;
    if (j + PD < NB) {
      asm volatile("" ::: "memory");
      load_a(j + PD);
#pragma unroll
      for (int c = 0; c < CT; ++c) load_b(braw[j + PD][c], bl[c], g0 + j + PD);
      asm volatile("" ::: "memory");
    }
    bool huge = false;
    if constexpr (GS > 0) {
#pragma unroll
      for (int c = 0; c < CT; ++c) {
#pragma unroll
        for (int i = 0; i < QB::kScales; ++i) {
          const int v = j * (kGroupK / GS) + (64 * q) / GS + i;
          braw[j][c].scale[i] = Ms[rt[c] * C::kSPR + v];
          braw[j][c].bias[i] = Ms[C::kRows * C::kSPR + rt[c] * C::kSPR + v];
        }
        huge |= bsrc.huge_scale(braw[j][c]);
      }
    } else if constexpr (StreamMeta<BSrc>::kRegMeta) {
#pragma unroll
      for (int c = 0; c < CT; ++c) huge |= bsrc.huge_scale(braw[j][c]);
    }
    // A fragments are read from LDS one step ahead of their MFMA (not all
    // eight up front): 24 fewer live registers, which lets a CU hold every
    // workgroup of the decode grid at once.
    auto afrag = [&](int s) {
      if constexpr (AG) return areg[j % kAR][s];
      else return *reinterpret_cast<const F*>(As + C::a_off(arow, QB::a_k(j, q, s)));
    };
    f32x4 acc[CT];
#pragma unroll
    for (int c = 0; c < CT; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto steps = [&](auto fast) {
      F a_cur = afrag(0);
#pragma unroll
      for (int s = 0; s < kSteps; ++s) {
        const F a_nxt = afrag(s + 1 < kSteps ? s + 1 : s);
#pragma unroll
        for (int c = 0; c < CT; ++c) {
          const F bf = bsrc.template frag<true, decltype(fast)::value>(braw[j][c], s, QB::kbase(g, q));
          acc[c] = mfma_step(a_cur, bf, acc[c]);
        }
        a_cur = a_nxt;
      }
    };
    if (!__any(huge)) steps(std::true_type());
    else steps(std::false_type());
#pragma unroll
    for (int c = 0; c < CT; ++c) accs[j][c] = acc[c];
  }
  // The wave's A and metadata are dead now (its DS reads complete in order):
  // its partials take their place, slot j CT + c.
  asm volatile("" ::: "memory");
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int c = 0; c < CT; ++c)
      *reinterpret_cast<f32x4*>(regions + (size_t)wave * C::kWaveBytes + (j * CT + c) * kWave * 16 + lane * 16) =
          accs[j][c];
  __syncthreads();
  // Ordered fold: one thread per stored output element (column tile c, lane
  // l, register e of the MFMA result layout), eight LDS loads in flight, adds
  // in group order. Partial of group g: wave g / NB's region, slot
  // (g % NB) CT + c.
  auto pptr = [&](int g, int c, int l, int e) {
    return reinterpret_cast<const float*>(regions + (size_t)(g / NB) * C::kWaveBytes +
                                          ((g % NB) * CT + c) * kWave * 16 + l * 16) + e;
  };
  for (int idx = threadIdx.x; idx < CT * kWave * 4; idx += kWave * W) {
    const int c = idx / (kWave * 4), e = (idx / kWave) % 4, l = idx % kWave;
    const int m = 4 * (l / 16) + e;
    const int col = n_base + 16 * c + l % 16;
    if (m >= M || col >= N) continue;           // tile rows past M, columns past N are never stored
    float total = 0.f;
    int gg = 0;
    for (; gg + 8 <= G; gg += 8) {
      float v[8];
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) v[jj] = *pptr(gg + jj, c, l, e);
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) total = total + v[jj];
    }
    for (; gg < G; ++gg) total = total + *pptr(gg, c, l, e);
    out[(int64_t)m * N + col] = to_store<T>(total);
  }
}

}  // namespace bi
