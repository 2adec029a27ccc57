// bi_gemm_big.h — the large-M dense tile: 256 x 128 outputs per workgroup of
// 8 waves (4 x 2, 64 x 64 outputs each, two waves per SIMD), operands copied
// global -> LDS by the load unit (buffer_load ... lds, no VGPR staging). A
// 128 x 128 form (2 x 2 waves, one per SIMD) serves shapes whose 256-row
// tiles would leave CUs idle; everything below holds for both, with the
// A rows and copy counts scaled.
//
// Same arithmetic as every other matmul launch (bi_gemm_tile.h, dense k-slot
// map k = 256 g + 32 s + 8 q + e): per 256-k group eight MFMA steps from zero,
// then total = total + acc. Only the staging and the instruction order differ.
//
// Stage = 64 k (two MFMA steps) of 256 A rows and 128 B rows. Each row is 128
// bytes in LDS (8 chunks of 8 elements) with chunk c of row r stored in slot
// c ^ (r & 7). One copy instruction moves 8 whole rows: lane l fetches row
// l / 8, chunk (l % 8) ^ (l / 8), and lands at 16 l, which is exactly that
// chunk's swizzled slot. Rows are read as whole 128-byte lines, and the MFMA
// fragment reads (lane 16 q + r: row r, chunk 4 s + q) hit 8 distinct slots
// in every 8-lane group: no LDS bank conflicts.
//
// Copies go through buffer resources whose range ends at the last valid row
// of the tile: rows past M (N) read as zero without touching memory, so no
// address is clamped. Past the last stage the copies use an empty resource
// (no memory traffic), which keeps the stage loop free of branches.
//
// Rings: A in 3 stage buffers (3 x 32 KB), B in 4 (4 x 16 KB) = 160 KB. Each
// stage has one mid-stage barrier, between its two MFMA steps:
//   step (st, 0): MFMAs on fragments already in registers; the fragment
//                 reads of step (st, 1); the B copies of stage st + 3 (B buffer
//                 (st + 3) % 4 was last read before the previous barrier);
//   barrier:      this wave's copies of stage st + 1 have landed and its reads
//                 of stage st are done, then every wave's;
//   step (st, 1): MFMAs; the reads of step (st + 1, 0); the A copies of stage
//                 st + 3 (A buffer st % 3, free since the barrier).
// Copies and fragment reads are spread one per MFMA pair with hard scheduling
// fences, so the load unit, the LDS and the matrix core work side by side
// instead of in bursts. An A fragment is re-read for the next step right
// after its last MFMA of the current step (single-buffered); B fragments are
// double-buffered.
//
// The group fold (total += acc, one VALU add per accumulator) is spread over
// the last step of a group (tiles already final) and the first step of the
// next (each tile just before its first MFMA overwrites acc).
//
// Tile order: workgroup ids are dealt round-robin to the 8 XCDs; each XCD
// takes a contiguous run of tile indices, and the run walks groups of 4 tile
// rows column by column, so the tiles an XCD runs at once share 4 rows of A
// and 8 columns of B in its L2.
//
// K need not be whole groups: stages at or past K (K % 64 == 0) are copied
// through the empty resource, i.e. computed with exact-zero fragments, so the
// last group still runs its eight steps.
//
// Requirements (checked by the host policy): 2-byte T, K % 64 == 0, rows of
// A and B 16-byte aligned (lda, ldb % 8 == 0), lda, ldb < 2^22 (a tile's
// rows are addressed with 32-bit byte offsets).
#pragma once

#include "bi_gemm_tile.h"

namespace bi {

constexpr int kBigBM = 256, kBigBN = 128;
constexpr int kBigWavesM = 4, kBigWavesN = 2, kBigWaves = kBigWavesM * kBigWavesN;
constexpr int kBigTI = kBigBM / 16 / kBigWavesM;            // 4 row blocks of 16 per wave
constexpr int kBigTJ = kBigBN / 16 / kBigWavesN;            // 4 column blocks of 16 per wave
constexpr int kBigACopies = kBigBM / 8 / kBigWaves;         // 4 copy instructions per wave per stage
constexpr int kBigBCopies = kBigBN / 8 / kBigWaves;         // 2
constexpr int kBigAStage = kBigBM * 64, kBigBStage = kBigBN * 64;  // elements per stage buffer
constexpr int kBigABufs = 3, kBigBBufs = 4;
constexpr int kBigGroupM = 4;
constexpr int64_t kBigMaxLd = (int64_t)1 << 22;
// The large tile is taken from M = 256 with at least this many tiles (fewer
// tiles than CUs still beat the smaller LDS tiles at these shapes).
constexpr int kBigMinM = 256;
constexpr int kBigMinTiles = 96;

// WM = waves along M: 4 for the 256 x 128 tile (8 waves, two per SIMD), 2
// for a 128 x 128 tile (4 waves, one per SIMD, 112 KB of LDS), which puts
// twice as many workgroups on the chip when the 256-row tiles are fewer than
// the CUs. BN = tile columns: 128 (64 x 64 per wave) or 64 (128 x 64 tiles,
// 64 x 32 per wave, 80 KB of LDS: two workgroups per CU), which puts twice as
// many workgroups again on the chip for mid-size M. Same steps per output
// element, same bits.
template <int WM, int BN = kBigBN>
struct BigTile {
  static constexpr int kBM = 64 * WM, kBN = BN, kWaves = 2 * WM;
  static constexpr int kTJ = BN / 16 / kBigWavesN;     // column blocks of 16 per wave: 4 or 2
  static constexpr int kACopies = kBM / 8 / kWaves;   // 4
  static constexpr int kBCopies = BN / 8 / kWaves;     // 2 (WM = 4) or 4 (WM = 2, BN = 128) or 2 (BN = 64)
  static constexpr int kAStage = kBM * 64;
  static constexpr int kBStage = BN * 64;
  static constexpr int kLdsElems = kBigABufs * kAStage + kBigBBufs * kBStage;
  static_assert(WM == 2 || WM == 4, "gemm_big: 128- or 256-row tiles");
  static_assert(BN == 128 || (BN == 64 && WM == 2), "gemm_big: 128 columns, or 64 with 128 rows");
};
static_assert(BigTile<4>::kBM == kBigBM && BigTile<4>::kWaves == kBigWaves && BigTile<4>::kACopies == kBigACopies &&
                  BigTile<4>::kBCopies == kBigBCopies,
              "gemm_big: the default tile is the 256 x 128 one");

template <int WM, int BN>
constexpr int big_threads() { return 64 * BigTile<WM, BN>::kWaves; }

template <typename T, int WM = kBigWavesM, int BN = kBigBN>
__global__ __launch_bounds__((big_threads<WM, BN>())) void gemm_big(const T* __restrict__ a, int64_t lda,
                                                                     const T* __restrict__ bt, int64_t ldb,
                                                                     T* __restrict__ out, int M, int N, int K,
                                                                     int tiles_m, int tiles_n) {
  static_assert(sizeof(T) == 2, "gemm_big: 2-byte element types only");
  typedef typename Frag<T>::type F;
  typedef BigTile<WM, BN> BT;
  constexpr int kBM = BT::kBM, kWavesAll = BT::kWaves, kACop = BT::kACopies, kBCop = BT::kBCopies;
  constexpr int kAStg = BT::kAStage, kBStg = BT::kBStage;
  constexpr int TI = kBigTI, TJ = BT::kTJ, NT = TI * TJ, NCH = NT / 2;
  static_assert(kACop <= NCH && kBCop <= NCH, "gemm_big: one copy per MFMA chunk at most");
  __shared__ __attribute__((aligned(1024))) T lds[BT::kLdsElems];

  const int tiles_total = tiles_m * tiles_n;
  const int groups = (K + kGroupK - 1) / kGroupK;
  const int work = tiles_total;
  const int bid = blockIdx.x;
  const int per_xcd = (work + 7) / 8;
  const int w_id = (bid % 8) * per_xcd + bid / 8;
  if (w_id >= work) return;  // uniform per workgroup, before any barrier
  const int t = w_id;
  const int span = kBigGroupM * tiles_n;
  const int first_m = (t / span) * kBigGroupM;
  const int gm = min(tiles_m - first_m, kBigGroupM);
  const int tm = first_m + (t % span) % gm, tn = (t % span) / gm;
  const int m0 = tm * kBM, n0 = tn * BN;

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int r = lane % 16, q = lane / 16;
  const int wm = wave / kBigWavesN, wn = wave % kBigWavesN;

  // LDS element offset of row `row` of stage st (A rows 0..255, B rows 0..127).
  auto a_row = [&](int st, int row) { return (st % kBigABufs) * kAStg + row * 64; };
  auto b_row = [&](int st, int row) { return kBigABufs * kAStg + (st % kBigBBufs) * kBStg + row * 64; };

  // Copy c of this wave moves the 8-row block c * 8 + wave of A (or of B):
  // lane l takes row l / 8 of the block, chunk (l % 8) ^ (l / 8).
  const int rr = lane / 8, ch = (lane % 8) ^ rr;
  const int rows_a = min(M - m0, kBM), rows_b = min(N - n0, BN);
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc((void*)(a + (int64_t)m0 * lda), (short)0, (int)(rows_a * lda * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc((void*)(bt + (int64_t)n0 * ldb), (short)0, (int)(rows_b * ldb * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t r_none = __builtin_amdgcn_make_buffer_rsrc((void*)a, (short)0, 0, 0x00020000);
  const unsigned voa = (unsigned)(((8 * wave + rr) * lda + 8 * ch) * 2);
  const unsigned vob = (unsigned)(((8 * wave + rr) * ldb + 8 * ch) * 2);
  // Stage st is 64 k (128 bytes of each row); stages at or past K read as zero.
  const int kst_valid = K / 64;
  auto copy_a = [&](int st, bool real, int c) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(real && st < kst_valid ? ra : r_none,
                                             (lds_void_t*)(lds + a_row(st, 8 * (c * kWavesAll + wave))),
                                             16, voa + (unsigned)(c * 8 * kWavesAll * lda * 2), st * 128, 0, 0);
  };
  auto copy_b = [&](int st, bool real, int c) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(real && st < kst_valid ? rb : r_none,
                                             (lds_void_t*)(lds + b_row(st, 8 * (c * kWavesAll + wave))),
                                             16, vob + (unsigned)(c * 8 * kWavesAll * ldb * 2), st * 128, 0, 0);
  };

  // Fragment reads: row r of a 16-row block, chunk 4 s + q of step s.
  const int frag_off[2] = {r * 64 + ((q ^ (r & 7)) << 3), r * 64 + (((4 + q) ^ (r & 7)) << 3)};
  auto read_a = [&](F& f, int st, int s, int i) {
    f = *reinterpret_cast<const F*>(lds + a_row(st, 16 * TI * wm + 16 * i) + frag_off[s]);
  };
  auto read_b = [&](F& f, int st, int s, int j) {
    f = *reinterpret_cast<const F*>(lds + b_row(st, 16 * TJ * wn + 16 * j) + frag_off[s]);
  };

  f32x4 total[TI][TJ], acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      total[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};  // the first group's "previous" partial
    }
  auto fold = [&](int tt) { total[tt / TJ][tt % TJ] = total[tt / TJ][tt % TJ] + acc[tt / TJ][tt % TJ]; };
  constexpr int kFoldLast = NCH - 1;  // tiles 0 .. kFoldLast-1 fold during a group's last step

  const int nst = 4 * groups;  // 4 stages per group
#pragma unroll
  for (int st = 0; st < 3; ++st) {
#pragma unroll
    for (int c = 0; c < kACop; ++c) copy_a(st, true, c);
#pragma unroll
    for (int c = 0; c < kBCop; ++c) copy_b(st, true, c);
  }
  wait_vm_lgkm0<2 * (kACop + kBCop)>();
  __builtin_amdgcn_s_barrier();
  F fa[TI], fb0[TJ], fb1[TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i) read_a(fa[i], 0, 0, i);
#pragma unroll
  for (int j = 0; j < TJ; ++j) read_b(fb0[j], 0, 0, j);

  // One MFMA step: NCH chunks of two MFMAs (tiles 2x, 2x + 1; tile tt is A
  // block tt / TJ, B block tt % TJ), each chunk fenced.
  //   bc / bn: this step's B fragments / the next step's (read here);
  //   (rst, rs): the stage and step the reads are for;
  //   copies: 0 none, 1 the B rows of stage cst, 2 the A rows of stage cst;
  //   fold_mode: 0 none, 1 a group's last step, 2 a group's first step.
  auto step = [&](F (&bc)[TJ], F (&bn)[TJ], int rst, int rs, int copies, int cst, bool real, bool first,
                  int fold_mode) {
    int f = fold_mode == 1 ? 0 : kFoldLast;
#pragma unroll
    for (int x = 0; x < NCH; ++x) {
      if (copies == 1 && x < kBCop) copy_b(cst, real, x);
      if (copies == 2 && x < kACop) copy_a(cst, real, x);
      if (x < TJ) read_b(bn[x], rst, rs, x);
      if (fold_mode == 1) {
        if (x >= 1 && f < 2 * x && f < kFoldLast) fold(f++);  // tiles final in earlier chunks
      } else if (fold_mode == 2) {
        if (f < NT) fold(f++);
        while (f < 2 * x + 2) fold(f++);                       // before their first MFMA
      }
#pragma unroll
      for (int y = 0; y < 2; ++y) {
        const int tt = 2 * x + y, i = tt / TJ, j = tt % TJ;
        acc[i][j] = mfma_step(fa[i], bc[j], first ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[i][j]);
        if (j == TJ - 1) read_a(fa[i], rst, rs, i);  // last use this step: read the next step's
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  for (int g = 0; g < nst / 4; ++g) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int st = 4 * g + p;
      step(fb0, fb1, st, 1, 1, st + 3, st + 3 < nst, p == 0, p == 0 ? 2 : 0);
      // stage st + 1 landed (younger: stage st + 2 and the B rows of st + 3);
      // this wave's reads of stage st are done; then every wave's are.
      wait_vm_lgkm0<kACop + 2 * kBCop>();
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      step(fb1, fb0, st + 1, 0, 2, st + 3, st + 3 < nst, false, p == 3 ? 1 : 0);
    }
  }
  wait_vm_lgkm0<0>();  // no copy may still be writing this workgroup's LDS when it exits
#pragma unroll
  for (int tt = kFoldLast; tt < NT; ++tt) fold(tt);

#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int n = n0 + 16 * TJ * wn + 16 * j + r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 16 * TI * wm + 16 * i + 4 * q + e;
        if (m < M && n < N) out[(int64_t)m * N + n] = to_store<T>(total[i][j][e]);
      }
    }
}

}  // namespace bi
