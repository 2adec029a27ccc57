// bi_gemm_big.h — the large-M dense tile: 256 x 128 outputs per workgroup of
// 8 waves, operands copied global -> LDS by the load unit
// (global_load_lds_dwordx4, no VGPR staging), three stage buffers.
//
// Same arithmetic as every other matmul launch (bi_gemm_tile.h, dense k-slot
// map k = 256 g + 32 s + 8 q + e): per 256-k group eight MFMA steps from zero,
// then total = total + acc. Only the staging differs.
//
// Stage = 64 k of 256 A rows and 128 B rows (48 KB). In LDS each of the 384
// rows is 128 bytes (8 chunks of 8 elements) with chunk c of row r stored in
// slot c ^ (r & 7). One copy instruction moves 8 whole rows: lane l fetches
// row 8b + l/8, chunk (l % 8) ^ (l / 8), and lands at 16 l, which is exactly
// that chunk's swizzled slot. Each row is thus read as one full 128-byte line
// (16 rows x 64 bytes per instruction measured half the L2 throughput), and
// the MFMA fragment reads (lane 16 q + r: row r, chunk 4 s + q) hit 8
// distinct slots in every 8-lane group: no LDS bank conflicts.
//
// Wave roles: 8 waves in 4 x 2, each 64 x 64 outputs (4 x 4 MFMA tiles; fp32
// acc + total = 128 registers, so two waves share a SIMD). Wave w copies rows
// 48 w .. 48 w + 47 of each stage (6 instructions). Stage st + 2 is requested
// right after the barrier that opens stage st, so copies have two stages of
// MFMA work to land.
//
// Tile order: workgroup ids are dealt round-robin to the 8 XCDs; each XCD
// takes a contiguous run of tile indices, and the run walks groups of 4 tile
// rows column by column, so the ~32 tiles an XCD runs at once share 4 rows of
// A and 8 columns of B in its L2.
//
// Requirements (checked by the host policy): 2-byte T, K % 256 == 0, rows of
// A and B 16-byte aligned (lda, ldb % 8 == 0). Rows past M / columns past N
// are clamped to the last valid one (never stored).
#pragma once

#include "bi_gemm_tile.h"

namespace bi {

constexpr int kBigBM = 256, kBigBN = 128;
constexpr int kBigWaves = 8;
constexpr int kBigRows = kBigBM + kBigBN;                      // 384 rows per stage
constexpr int kBigStage = kBigRows * 64;                       // elements (48 KB)
constexpr int kBigBufs = 3;
constexpr int kBigCopiesPerWave = kBigRows / 8 / kBigWaves;    // 6
constexpr int kBigGroupM = 4;
// The large tile is taken from M = 256 with at least this many tiles (fewer
// tiles than CUs still beat the smaller LDS tiles at these shapes).
constexpr int kBigMinM = 256;
constexpr int kBigMinTiles = 96;

template <typename T>
__global__ __launch_bounds__(64 * kBigWaves) void gemm_big(const T* __restrict__ a, int64_t lda,
                                                           const T* __restrict__ bt, int64_t ldb,
                                                           T* __restrict__ out, int M, int N, int K,
                                                           int tiles_m, int tiles_n) {
  static_assert(sizeof(T) == 2, "gemm_big: 2-byte element types only");
  typedef typename Frag<T>::type F;
  __shared__ __attribute__((aligned(1024))) T lds[kBigBufs * kBigStage];

  const int tiles_total = tiles_m * tiles_n;
  const int bid = blockIdx.x;
  const int per_xcd = (tiles_total + 7) / 8;
  const int t = (bid % 8) * per_xcd + bid / 8;
  if (t >= tiles_total) return;  // uniform per workgroup, before any barrier
  const int span = kBigGroupM * tiles_n;
  const int first_m = (t / span) * kBigGroupM;
  const int gm = min(tiles_m - first_m, kBigGroupM);
  const int tm = first_m + (t % span) % gm, tn = (t % span) / gm;
  const int m0 = tm * kBigBM, n0 = tn * kBigBN;

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int r = lane % 16, q = lane / 16;
  const int wm = wave / 2, wn = wave % 2;

  // Copy sources: instruction c of this wave moves stage rows 8 b .. 8 b + 7,
  // b = 6 wave + c (rows 0..255 are A, 256..383 are B).
  const T* src[kBigCopiesPerWave];
  {
    const int rr = lane / 8, ch = (lane % 8) ^ rr;
#pragma unroll
    for (int c = 0; c < kBigCopiesPerWave; ++c) {
      const int row = 8 * (wave * kBigCopiesPerWave + c) + rr;
      src[c] = row < kBigBM ? a + (int64_t)min(m0 + row, M - 1) * lda + 8 * ch
                            : bt + (int64_t)min(n0 + row - kBigBM, N - 1) * ldb + 8 * ch;
    }
  }
  auto issue = [&](int st) {
    T* buf = lds + (st % kBigBufs) * kBigStage + wave * kBigCopiesPerWave * 512;
#pragma unroll
    for (int c = 0; c < kBigCopiesPerWave; ++c) copy_to_lds16(src[c] + 64 * st, buf + c * 512);
  };

  // Fragment read offsets (elements): row r of a 16-row block, chunk 4 s + q.
  const int frag_off[2] = {r * 64 + ((q ^ (r & 7)) << 3), r * 64 + (((4 + q) ^ (r & 7)) << 3)};

  f32x4 total[4][4], acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) total[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nst = K / 64;  // K % 256 == 0: 4 stages per group
  issue(0);
  if (nst > 1) issue(1);
  for (int g = 0; g < nst / 4; ++g) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int st = 4 * g + p;
      // stage st visible to all waves; stage st - 1 no longer read by any wave
      if (st + 1 < nst) stage_barrier<kBigCopiesPerWave>();
      else stage_barrier<0>();
      if (st + 2 < nst) issue(st + 2);
      const T* buf = lds + (st % kBigBufs) * kBigStage;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        F af[4], bf[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          af[i] = *reinterpret_cast<const F*>(buf + (64 * wm + 16 * i) * 64 + frag_off[s]);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          bf[j] = *reinterpret_cast<const F*>(buf + (kBigBM + 64 * wn + 16 * j) * 64 + frag_off[s]);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = mfma_step(af[i], bf[j], (p == 0 && s == 0) ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[i][j]);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) total[i][j] = total[i][j] + acc[i][j];
  }

#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + 64 * wn + 16 * j + r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 64 * wm + 16 * i + 4 * q + e;
        if (m < M && n < N) out[(int64_t)m * N + n] = to_store<T>(total[i][j][e]);
      }
    }
}

}  // namespace bi
