// bi_gemm_tall.h — the dense mid-M launch (16 < M <= 128): a weight stream
// read once from HBM through a deep LDS ring, the M rows of A beside it.
//
// Same arithmetic as every other matmul launch (bi_gemm_tile.h, dense k-slot
// map k = 256 g + 32 s + 8 q + e): per 256-k group eight MFMA steps from zero,
// then total = total + acc in group order. k >= K contributes exact zeros: a
// stage past K is computed with zero fragments, so every group still runs its
// eight steps.
//
// Workgroup tile BM x BN = (16 TI WM) x (16 WN) with 4 waves in WM x WN; wave
// (wm, wn) owns TI row blocks of 16 and the 16 columns of block wn for the
// whole of its K range, so the group fold stays in registers. A stage is SK k
// (128, or 64 when K is not a multiple of 128) of the tile's BM A rows and BN
// B rows, each row SK * 2 bytes in LDS with chunk c of row r in slot
// c ^ (r % chunks) (one copy instruction moves whole rows; the 16 rows of a
// fragment read hit distinct slots). 256-byte row pieces matter: a stream of
// 128-byte pieces of the weight rows measured 2.6 TB/s, of 256-byte pieces
// 4.1 TB/s, of 512-byte pieces 5.1 TB/s (DRAM page locality). Stages stream through a
// ring of R buffers: stage st + R - 1 is requested right after the barrier
// that opens stage st, so R - 1 stages (up to 144 KB per workgroup) are in
// flight: the weight stream needs that much per CU to cover HBM latency.
//
// Copies go through buffer resources that end at the tile's last valid row:
// rows past M (N) read as zero without touching memory. Copy slots beyond the
// tile's rows, and every copy of a stage past K, use an empty resource, so
// each wave issues the same number of copies per stage and the wait counts
// are compile-time constants.
//
// SPLIT: grid.z chunks of CG groups; each group's raw fp32 partial goes to
// part[g][m][n] and fold_groups folds them in group order (the launch for
// shapes with too few column tiles to fill the chip).
//
// Requirements (host policy): 2-byte T, K % SK == 0, lda, ldb % 8 == 0 and
// < 2^22, 16-byte aligned operands.
#pragma once

#include "bi_gemm_big.h"

namespace bi {

template <int TI, int WM, int WN, int SK, int RMAX = 12>
struct TallCfg {
  static constexpr int kBM = 16 * TI * WM, kBN = 16 * WN;
  static constexpr int kRowElems = SK;                           // elements of a row per stage
  static constexpr int kChunks = SK / 8;                         // 16-byte chunks per row
  static constexpr int kRowsPerCopy = 64 / kChunks;              // rows per 1 KB copy instruction
  static constexpr int kSlotRows = 4 * kRowsPerCopy;             // rows per copy slot over 4 waves
  static constexpr int kCopiesA = kBM / kSlotRows;               // A copy slots per wave (all real)
  static constexpr int kCopiesB = (kBN + kSlotRows - 1) / kSlotRows;  // B copy slots per wave
  static constexpr int kCopies = kCopiesA + kCopiesB;            // per wave per stage
  static constexpr int kRowsAlloc = kSlotRows * kCopies;         // B slots past BN land in padding rows
  static constexpr int kStageBytes = kRowsAlloc * SK * 2;
  // As deep as LDS allows, capped at RMAX (a smaller ring leaves room for
  // more resident workgroups per CU).
  static constexpr int kRing = (160 * 1024 / kStageBytes) < RMAX ? (160 * 1024 / kStageBytes) : RMAX;
  static constexpr int kStagesPerGroup = kGroupK / SK;
  static_assert(SK == 64 || SK == 128, "gemm_tall: 64- or 128-k stages");
  static_assert(WM * WN == 4, "gemm_tall: 4 waves");
  static_assert(kBM % kSlotRows == 0, "gemm_tall: A rows in whole copy slots");
  static_assert(kRing >= 3, "gemm_tall: ring of at least 3 stages");
  static_assert((kRing - 2) * kCopies < 64, "gemm_tall: vmcnt range");
  // Chunk c of row r sits in slot c ^ (r % kChunks): the 16 rows of a
  // fragment read hit distinct slots (conflict-free ds_read_b128).
  static __device__ __forceinline__ int slot(int r, int c) { return c ^ (r & (kChunks - 1)); }
};

template <typename T, int TI, int WM, int WN, int SK, bool SPLIT, int RMAX = 12>
__global__ __launch_bounds__(256) void gemm_tall(const T* __restrict__ a, int64_t lda, const T* __restrict__ bt,
                                                 int64_t ldb, T* __restrict__ out, float* __restrict__ part,
                                                 int M, int N, int K, int G, int CG) {
  static_assert(sizeof(T) == 2, "gemm_tall: 2-byte element types only");
  typedef TallCfg<TI, WM, WN, SK, RMAX> C;
  constexpr int SPG = C::kStagesPerGroup;
  typedef typename Frag<T>::type F;
  constexpr int R = C::kRing;
  __shared__ __attribute__((aligned(1024))) T lds[R * C::kRowsAlloc * SK];

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int r = lane % 16, q = lane / 16;
  const int wm = wave / WN, wn = wave % WN;
  const int n0 = blockIdx.x * C::kBN, m0 = blockIdx.y * C::kBM;
  const int g_begin = SPLIT ? blockIdx.z * CG : 0;
  const int g_end = SPLIT ? min(G, g_begin + CG) : G;
  const int st0 = SPG * g_begin, nst = SPG * (g_end - g_begin);  // stages of this workgroup
  const int st_valid = K / SK;                                      // stages inside K (global index)

  // A copy slot c of this wave moves A rows kRowsPerCopy (4 c + wave) .. of
  // the stage, B slot c the same B rows (B rows start at BM in the stage
  // buffer; slots past BN land in its padding rows through the empty
  // resource). Lane l takes row l / kChunks of the slot and the chunk that
  // belongs in slot l % kChunks of it; the swizzle key is the row's index in
  // the stage mod kChunks, kRowsPerCopy * wave + l / kChunks (copy slots start
  // at multiples of 4 kRowsPerCopy rows, and the B rows at BM, a multiple of 16).
  constexpr int RPC = C::kRowsPerCopy;
  const int rr = lane / C::kChunks, ch = C::slot(RPC * wave + rr, lane % C::kChunks);
  const int rows_a = min(M - m0, C::kBM), rows_b = min(N - n0, C::kBN);
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc((void*)(a + (int64_t)m0 * lda), (short)0, (int)(rows_a * lda * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc((void*)(bt + (int64_t)n0 * ldb), (short)0, (int)(rows_b * ldb * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t r_none = __builtin_amdgcn_make_buffer_rsrc((void*)a, (short)0, 0, 0x00020000);
  const unsigned voa = (unsigned)(((RPC * wave + rr) * lda + 8 * ch) * 2);
  const unsigned vob = (unsigned)(((RPC * wave + rr) * ldb + 8 * ch) * 2);
  // Stage st (global index) into buffer st % R. A stage past the workgroup's
  // range or past K goes through the empty resource: no memory traffic, and
  // its buffer is one no stage in flight uses.
  auto copy_stage = [&](int st) {
    const bool real = st - st0 < nst && st < st_valid;
    T* buf = lds + (st % R) * (C::kRowsAlloc * SK);
#pragma unroll
    for (int c = 0; c < C::kCopiesA; ++c)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(real ? ra : r_none,
                                               (lds_void_t*)(buf + RPC * (4 * c + wave) * SK), 16,
                                               voa + (unsigned)(4 * RPC * c * lda * 2), st * SK * 2, 0, 0);
#pragma unroll
    for (int c = 0; c < C::kCopiesB; ++c) {
      const bool live = real && RPC * (4 * c + wave) < C::kBN;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rb : r_none,
                                               (lds_void_t*)(buf + (C::kBM + RPC * (4 * c + wave)) * SK), 16,
                                               vob + (unsigned)(4 * RPC * c * ldb * 2), st * SK * 2, 0, 0);
    }
  };

  // Fragment of step s of a stage: row r of a 16-row block, chunk 4 s + q.
  auto frag_off = [&](int s) { return r * SK + (C::slot(r, 4 * s + q) << 3); };

  f32x4 total[TI], acc[TI];
#pragma unroll
  for (int i = 0; i < TI; ++i) total[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Prologue: stages 0 .. R - 2 of this workgroup's range.
#pragma unroll
  for (int j = 0; j < R - 1; ++j) copy_stage(st0 + j);
  for (int j = 0; j < nst; ++j) {
    const int st = st0 + j;
    // Stage j landed (younger: stages j + 1 .. j + R - 2); every wave is past
    // stage j - 1, whose buffer takes stage j + R - 1.
    wait_vm_lgkm0<(R - 2) * C::kCopies>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    copy_stage(st + R - 1);
    asm volatile("" ::: "memory");
    const T* buf = lds + (st % R) * (C::kRowsAlloc * SK);
    const bool live = st < st_valid;
    const int p = j % SPG;
#pragma unroll
    for (int s = 0; s < SK / 32; ++s) {
      F bf = *reinterpret_cast<const F*>(buf + (C::kBM + 16 * wn) * SK + frag_off(s));
      F af[TI];
#pragma unroll
      for (int i = 0; i < TI; ++i) af[i] = *reinterpret_cast<const F*>(buf + (16 * TI * wm + 16 * i) * SK + frag_off(s));
      if (!live) {
        bf = frag_zero<F>();
#pragma unroll
        for (int i = 0; i < TI; ++i) af[i] = frag_zero<F>();
      }
#pragma unroll
      for (int i = 0; i < TI; ++i)
        acc[i] = mfma_step(af[i], bf, (p == 0 && s == 0) ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[i]);
    }
    if (p == SPG - 1) {
      if constexpr (SPLIT) {
        const int g = st / SPG;
        const int n = n0 + 16 * wn + r;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int m = m0 + 16 * TI * wm + 16 * i + 4 * q + e;
            if (m < M && n < N) part[((int64_t)g * M + m) * N + n] = acc[i][e];
          }
      } else {
#pragma unroll
        for (int i = 0; i < TI; ++i) total[i] = total[i] + acc[i];
      }
    }
  }
  wait_vm_lgkm0<0>();  // no copy may still be writing this workgroup's LDS when it exits
  if constexpr (!SPLIT) {
    const int n = n0 + 16 * wn + r;
    if (n < N) {
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = m0 + 16 * TI * wm + 16 * i + 4 * q + e;
          if (m < M) out[(int64_t)m * N + n] = to_store<T>(total[i][e]);
        }
    }
  }
}

}  // namespace bi
