// bi_gemm_big.h — the large-M dense tile: 256 x 128 outputs per workgroup,
// operands copied global -> LDS by the load unit (global_load_lds_dwordx4),
// three stage buffers in flight.
//
// Same arithmetic as every other matmul launch (bi_gemm_tile.h, dense k-slot
// map k = 256 g + 32 s + 8 q + e): per 256-k group eight MFMA steps from zero,
// then total = total + acc. Only the staging differs.
//
// LDS layout: a stage is 64 k (steps 2p and 2p+1 of a group). Each operand is
// stored as 1 KB "fragment blocks", one per (16-row block, step): lane
// l = 16 q + r of the block holds the 8 elements row r, k = 32 s + 8 q .. +7,
// i.e. exactly that lane's MFMA operand. The DMA writes lane l's 16 bytes at
// block + 16 l, and the MFMA reads them back with one ds_read_b128 at the same
// address: no VGPR staging, no bank conflicts, no index math in the loop.
//
// Wave roles: 4 waves in 2 x 2, each 128 x 64 outputs (8 x 4 MFMA tiles, fp32
// acc + total = 256 registers, the acc half lives in AGPRs). For the copies,
// wave w fetches A row blocks 4w .. 4w+3 and B row blocks 2w, 2w+1 of every
// stage (12 blocks). Stage st + 2 is requested right after the barrier that
// opens stage st, so each copy has two stages of MFMA work to land.
//
// Requirements (checked by the host policy): 2-byte T, K % 256 == 0, rows of
// A and B 16-byte aligned (lda, ldb % 8 == 0). Rows past M / columns past N
// are clamped to the last valid one (never stored).
#pragma once

#include "bi_gemm_tile.h"

namespace bi {

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void gbl_void_t;

constexpr int kBigBM = 256, kBigBN = 128;
constexpr int kBigBlk = 512;                                  // elements per 1 KB fragment block
constexpr int kBigABlocks = kBigBM / 16 * 2;                  // 32 per stage
constexpr int kBigBBlocks = kBigBN / 16 * 2;                  // 16 per stage
constexpr int kBigStage = (kBigABlocks + kBigBBlocks) * kBigBlk;  // 48 KB of 2-byte elements
constexpr int kBigBufs = 3;
constexpr int kBigCopiesPerWave = (kBigABlocks + kBigBBlocks) / 4;  // 12

// One 16-byte-per-lane copy global -> LDS; lane l lands at lds_block + 16 l.
__device__ __forceinline__ void copy_to_lds16(const void* src, void* lds_block) {
  __builtin_amdgcn_global_load_lds((gbl_void_t*)src, (lds_void_t*)lds_block, 16, 0, 0);
}

// Stage barrier: wait until at most N vector-memory operations of this wave
// are outstanding (vmcnt counts global_load_lds copies until their data is in
// LDS; they complete in issue order) and all of its LDS reads have returned,
// then s_barrier. Unlike __syncthreads() this does not drain the copies of
// later stages that are still in flight. The empty asm statements keep the
// compiler from moving memory accesses across the barrier.
template <int N>
__device__ __forceinline__ void stage_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("" ::: "memory");
  // gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <typename T>
__global__ __launch_bounds__(256) void gemm_big(const T* __restrict__ a, int64_t lda,
                                                const T* __restrict__ bt, int64_t ldb,
                                                T* __restrict__ out, int M, int N, int K,
                                                int tiles_n, int tiles_total) {
  static_assert(sizeof(T) == 2, "gemm_big: 2-byte element types only");
  typedef typename Frag<T>::type F;
  __shared__ __attribute__((aligned(1024))) T lds[kBigBufs * kBigStage];

  // XCD-aware order: workgroup ids are dealt round-robin to the 8 XCDs; give
  // each XCD a contiguous run of tiles (same row of tiles -> shared A in L2).
  const int bid = blockIdx.x;
  const int per_xcd = (tiles_total + 7) / 8;
  const int tile = (bid % 8) * per_xcd + bid / 8;
  if (tile >= tiles_total) return;  // uniform per workgroup, before any barrier
  const int m0 = (tile / tiles_n) * kBigBM, n0 = (tile % tiles_n) * kBigBN;

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int r = lane % 16, q = lane / 16;
  const int wm = wave / 2, wn = wave % 2;

  // Copy sources of this wave (row r of each block, quarter q's 8 k).
  const T* asrc[4];
  const T* bsrc[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) asrc[i] = a + (int64_t)min(m0 + 16 * (4 * wave + i) + r, M - 1) * lda + 8 * q;
#pragma unroll
  for (int j = 0; j < 2; ++j) bsrc[j] = bt + (int64_t)min(n0 + 16 * (2 * wave + j) + r, N - 1) * ldb + 8 * q;

  auto issue = [&](int st) {
    T* buf = lds + (st % kBigBufs) * kBigStage;
    const int k0 = st * 64;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int s = 0; s < 2; ++s) copy_to_lds16(asrc[i] + k0 + 32 * s, buf + ((4 * wave + i) * 2 + s) * kBigBlk);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int s = 0; s < 2; ++s)
        copy_to_lds16(bsrc[j] + k0 + 32 * s, buf + (kBigABlocks + (2 * wave + j) * 2 + s) * kBigBlk);
  };

  f32x4 total[8][4], acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
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
        F af[8], bf[4];
#pragma unroll
        for (int i = 0; i < 8; ++i) af[i] = *reinterpret_cast<const F*>(buf + ((8 * wm + i) * 2 + s) * kBigBlk + 8 * lane);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          bf[j] = *reinterpret_cast<const F*>(buf + (kBigABlocks + (4 * wn + j) * 2 + s) * kBigBlk + 8 * lane);
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = mfma_step(af[i], bf[j], (p == 0 && s == 0) ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[i][j]);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) total[i][j] = total[i][j] + acc[i][j];
  }

#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + 64 * wn + 16 * j + r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 128 * wm + 16 * i + 4 * q + e;
        if (m < M && n < N) out[(int64_t)m * N + n] = to_store<T>(total[i][j][e]);
      }
    }
}

}  // namespace bi
