// bi_attn_mfma.h — the split-KV attention kernels (decode, prefill) with every
// product on the matrix cores. The per-split arithmetic (bi_attn_common.h) is
// one text shared by both kernels, so a row gets the same bits from either.
//
// Layouts (v_mfma_f32_16x16x32_{bf16,f16}; fp32 runs eight 16x16x4 steps per
// 32-wide step with the same element order):
//   scores  S^T = MFMA(A = K rows, B = Q^T): A lane (key r, quarter qq) holds
//           K[key r][32 st + 8 qq + e], B lane (row n, qq) holds
//           Q[row n][32 st + 8 qq + e]; the result lane (n, qq) holds the
//           scores of row n with keys 16 t + 4 qq + i (i = 0..3) of tile t.
//   P.V     acc = MFMA(A = P, B = V^T) per 32-key step ks: A lane (row r, qq)
//           holds P of keys 32 ks + {4 qq + i, 16 + 4 qq + i} — exactly what
//           the score layout leaves in that lane for tiles 2 ks, 2 ks + 1 —
//           and B lane (dim n, qq) holds V of the same keys for dim n; the
//           result lane (n, qq) holds rows 4 qq + i of dim n.
//   V^T     V rows sit in LDS as loaded ([key][D], 16-byte chunk c of row r in
//           slot c ^ (r & 7)); ds_read_b64_tr_b16 returns, in each 16-lane
//           group, element (t % 4) of the 8 bytes read by lane 4 j + t / 4 as
//           slot j of lane t, so lane 4 j + c reading V[key j][4 c .. 4 c + 3]
//           hands every lane 4 keys of one dim. fp32 V is read one element
//           per lane (ds_read_b32).
#pragma once

#include <type_traits>

#include "bi_attn_common.h"

namespace bi {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// LDS tile of K or V rows: row r, 16-byte chunk c at byte offset off(r, c).
// Rows are stored back to back (D * sizeof(T) bytes); when a row holds a
// multiple of 8 chunks, chunk c sits in slot c ^ (r & 7) (a fragment read's 16
// rows then hit distinct bank groups), otherwise in slot c.
template <typename T, int D>
struct KVTile {
  static constexpr int kRowBytes = D * (int)sizeof(T);
  static constexpr int kCPR = kRowBytes / 16;          // 16-byte chunks per row
  static constexpr bool kSwz = kCPR % 8 == 0;
  static_assert(kCPR % 4 == 0, "KVTile: D * sizeof(T) must be a multiple of 64 bytes");
  static __device__ __forceinline__ int off(int r, int c) {
    return r * kRowBytes + ((kSwz ? (c ^ (r & 7)) : c) << 4);
  }
  // Copy instruction ci of a tile moves its flat chunks 64 ci .. 64 ci + 63
  // (1 KB): lane l fetches the chunk that belongs in flat slot 64 ci + l,
  // landing at tile + 1024 ci + 16 l. `row(i)` gives the first element of
  // tile row i (0 <= i < nrows_valid; rows past it repeat the last valid row).
  template <class RowPtr>
  static __device__ __forceinline__ void copy(char* tile, int ci, RowPtr row, int nrows_valid, int lane) {
    const int f = 64 * ci + lane;
    const int r = f / kCPR;
    const int slot = f - r * kCPR;
    const int c = kSwz ? (slot ^ (r & 7)) : slot;
    const T* src = row(min(r, nrows_valid - 1)) + c * (16 / (int)sizeof(T));
    copy_to_lds16(src, tile + 1024 * ci);
  }
  // Copy instructions that move `rows` whole rows.
  static constexpr int copies(int rows) { return rows * kCPR / 64; }
  // A-operand fragment of the score MFMA: row r, dims 32 st + 8 qq .. + 7.
  static __device__ __forceinline__ typename Frag<T>::type kfrag(const char* tile, int r, int st, int qq) {
    typedef typename Frag<T>::type F;
    if constexpr (sizeof(T) == 2) {
      return __builtin_bit_cast(F, *reinterpret_cast<const u32x4*>(tile + off(r, 4 * st + qq)));
    } else {
      F f;
      f.lo = *reinterpret_cast<const f32x4*>(tile + off(r, 8 * st + 2 * qq));
      f.hi = *reinterpret_cast<const f32x4*>(tile + off(r, 8 * st + 2 * qq + 1));
      return f;
    }
  }
  // B-operand fragment of the P.V MFMA for the 32 keys key0 .. key0 + 31 of
  // the tile and dims 16 dt .. 16 dt + 15: slot e of lane (n, qq) holds
  // V[key0 + (e < 4 ? 4 qq + e : 16 + 4 qq + e - 4)][16 dt + n].
  static __device__ __forceinline__ typename Frag<T>::type vfrag(const char* tile, int key0, int dt, int lane) {
    typedef typename Frag<T>::type F;
    const int qq = lane / 16, u = lane % 16;
    if constexpr (sizeof(T) == 2) {
      const int j = u / 4, c = u % 4;
      const int chunk = 2 * dt + (c >> 1);
      const int r0 = key0 + 4 * qq + j, r1 = r0 + 16;
      const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_s16x4*)(tile + off(r0, chunk) + ((c & 1) << 3)));
      const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_s16x4*)(tile + off(r1, chunk) + ((c & 1) << 3)));
      const s16x8 v = __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
      return __builtin_bit_cast(F, v);
    } else {
      const int dim = 16 * dt + u;
      const int chunk = dim >> 2, within = (dim & 3) << 2;
      F f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f.lo[e] = *reinterpret_cast<const float*>(tile + off(key0 + 4 * qq + e, chunk) + within);
        f.hi[e] = *reinterpret_cast<const float*>(tile + off(key0 + 16 + 4 * qq + e, chunk) + within);
      }
      return f;
    }
  }
};

// ---------------------------------------------------------------------------
// Decode: a resident grid of 256-thread workgroups walks the active work items
// (sequence b, split, kv head, head chunk of GU) in that nesting order; only
// splits below a sequence's own length are items, so a ragged batch launches
// no workgroup that has nothing to do (with a grid over every possible split,
// the empty workgroups of short sequences cost as much dispatch time as the
// real work). DYN = false: workgroup w takes items w, w + P, w + 2P, ...
// (P = grid size). DYN = true: each workgroup takes the next item from a
// counter (a.ctr, zero at launch), so workgroups that finish early take more
// items. Either way items come in increasing order per workgroup, which finds
// each item's sequence by walking the lengths forward.
// Per item: GU query heads are the 16 columns of the score tile (GU <= 16).
// Every wave first requests all of its memory: Q^T, the K rows of its 64 keys
// (registers, 16-byte loads, rows past the sequence end clamped to its last
// key) and a quarter of the split's V rows, which the load unit copies
// straight into LDS. Wave w scores keys 64 w .. 64 w + 63; the split maximum
// is exchanged through LDS; each wave writes its keys' weights to LDS; then
// wave w computes the P.V tiles of dims 16 dt, dt = w, w + 4, ..., and wave 0
// also the weight sum. Writes (m, l, acc) of its split. The arithmetic of an
// item does not depend on which workgroup runs it.
// ---------------------------------------------------------------------------
// V of a split is staged in LDS NVP dim slices of DV = D / NVP dims each: one
// slice (the whole row) when the split's V fits in 128 KB, two otherwise
// (fp32 with D > 128), the second copied after the first slice's P.V. The
// order of every output element's P.V chain is the same either way.
template <typename T, int D>
constexpr int decode_v_slices() {
  return kSplit * D * (int)sizeof(T) <= (128 << 10) ? 1 : 2;
}

template <typename T, int D, int GU, bool DYN, int MODE>
__global__ __launch_bounds__(256) void attn_decode_mfma(DecodeArgs a) {
  constexpr bool ROWPAGED = MODE == kKvRowPaged;
  typedef typename Frag<T>::type F;
  constexpr int NVP = decode_v_slices<T, D>();
  constexpr int DV = D / NVP;                           // dims per V slice
  typedef KVTile<T, DV> KV;
  constexpr int KT = 4;                                 // score tiles per wave
  constexpr int NDTV = DV / 16;                         // P.V dim tiles per slice
  constexpr int NCOPY = KV::copies(kSplit);             // copy instructions per slice
  constexpr int CPW = NCOPY / 4;                        // ... per wave
  static_assert(GU >= 1 && GU <= 16, "attn_decode_mfma: 1..16 heads per workgroup");
  static_assert(DV % 16 == 0 && CPW >= 1 && CPW < 64, "attn_decode_mfma: V slice tiling");
  __shared__ __attribute__((aligned(1024))) char Vs[kSplit * KV::kRowBytes];
  __shared__ __attribute__((aligned(16))) float Ps[GU][kSplit];
  __shared__ float mxs[4][16];
  __shared__ unsigned item_s;

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int per_split = a.Hkv * a.nchunk;  // items per (sequence, split)
  // Fixed V copy offsets (see copy_v): a copy moves 64 / kCPR whole rows, so
  // the swizzle key (row & 7) repeats every kVPeriod copies. The host keeps
  // 256 rows of the V stride below 2^31 bytes.
  constexpr bool kVFixed = MODE == kKvContig && (64 % KV::kCPR) == 0;
  constexpr int kRowsPerCopy = kVFixed ? 64 / KV::kCPR : 1;
  constexpr int kVPeriod = !KV::kSwz ? 1 : kRowsPerCopy >= 8 ? 1 : 8 / kRowsPerCopy;
  int v_off0[kVPeriod];
  const int v_step = kVPeriod * kRowsPerCopy * (int)(a.v_sl * (int64_t)sizeof(T));
#pragma unroll
  for (int c = 0; c < kVPeriod; ++c) {
    const int f = 64 * (wave * CPW + c) + lane;
    const int rr = f / KV::kCPR, slot = f - rr * KV::kCPR;
    const int cc = KV::kSwz ? (slot ^ (rr & 7)) : slot;
    v_off0[c] = (int)(rr * a.v_sl * (int64_t)sizeof(T)) + cc * 16;
  }
  int b = 0;
  int64_t base = 0;                         // items of sequences before b
  int len = 0;
  for (int64_t next = blockIdx.x;; next += gridDim.x) {
  int64_t item = next;
  if constexpr (DYN) {
    // The end-of-item barrier below keeps thread 0 from overwriting item_s
    // before every thread has read it.
    if (tid == 0) item_s = atomicAdd(a.ctr, 1u);
    __syncthreads();
    item = item_s;
  }
  // Advance to the sequence holding `item` (uniform per workgroup). A length
  // outside [0, L] is clamped, so no key past the cache is ever read.
  for (; b < a.B; ++b) {
    len = a.kv_lens ? min(max(a.kv_lens[b], 0), a.L) : a.L;
    const int64_t nb = (int64_t)((len + kSplit - 1) / kSplit) * per_split;
    if (item < base + nb) break;
    base += nb;
  }
  if (b >= a.B) break;
  const int64_t local = item - base;
  const int split = (int)(local / per_split);
  const int hk = (int)(local % per_split) / a.nchunk;
  const int chunk = (int)(local % per_split) % a.nchunk;
  const int j0 = split * kSplit;
  const int n_act = min(kSplit, len - j0);
  const int G = a.Hq / a.Hkv;
  const int h0 = hk * G + chunk * GU;
  const int r = lane % 16, qq = lane / 16;

  const T* qb = static_cast<const T*>(a.q) + (int64_t)b * a.q_sb;
  const T* kbase = static_cast<const T*>(a.k);
  const T* vbase = static_cast<const T*>(a.v);
  // This wave's K rows and V copies are keys 64 w .. 64 w + 63 of the split,
  // clamped to the last active key: one 64-key segment (the last active one
  // for a wave past the end).
  const int seg = __builtin_amdgcn_readfirstlane(min(wave, (n_act - 1) >> 6));
  const T* kseg = ROWPAGED ? kbase : kv_segment<MODE>(a, kbase, a.k_sb, a.k_sh, a.k_sl, b, hk, j0 + 64 * seg);
  const T* vseg = ROWPAGED ? vbase : kv_segment<MODE>(a, vbase, a.v_sb, a.v_sh, a.v_sl, b, hk, j0 + 64 * seg);
  auto krow = [&](int key) {
    if constexpr (ROWPAGED) return kbase + kv_row_off(a, a.k_sb, a.k_sh, a.k_sl, b, hk, j0 + key);
    else return kseg + (int64_t)(key - 64 * seg) * a.k_sl;
  };
  int vdim0 = 0;                                        // first dim of the V slice being staged
  auto vrow = [&](int key) {
    if constexpr (ROWPAGED) return vbase + kv_row_off(a, a.v_sb, a.v_sh, a.v_sl, b, hk, j0 + key) + vdim0;
    else return vseg + (int64_t)(key - 64 * seg) * a.v_sl + vdim0;
  };

  // V copies of this wave (rows 64 w .. 64 w + 63 of the split's V slice).
  // Contiguous cache with rows of a power-of-two number of 16-byte chunks: a
  // buffer resource from the split's first row to its last active one (rows
  // past it read as zero; their weights are exactly 0) and per-lane offsets
  // from the kernel's start (v_off0), advanced by a wave-uniform row step per
  // copy, instead of a 64-bit row address per copy.
  auto copy_v = [&]() {
    if constexpr (kVFixed) {
      const auto rs = buffer_rsrc(vbase + (int64_t)b * a.v_sb + (int64_t)hk * a.v_sh + (int64_t)j0 * a.v_sl,
                                  (int)(n_act * a.v_sl * (int64_t)sizeof(T)));
      const int vbytes = vdim0 * (int)sizeof(T);
#pragma unroll
      for (int c = 0; c < CPW; ++c)
        copy_to_lds16(rs, v_off0[c % kVPeriod] + (c / kVPeriod) * v_step + vbytes, Vs + 1024 * (wave * CPW + c));
    } else {
#pragma unroll
      for (int c = 0; c < CPW; ++c) KV::copy(Vs, wave * CPW + c, vrow, n_act, lane);
    }
  };

  // Memory requests, in this order: Q^T, this wave's K rows, its V copies.
  F qf[D / 32];
  {
    const T* qrow = qb + (int64_t)(h0 + (r < GU ? r : 0)) * a.q_sh;
#pragma unroll
    for (int st = 0; st < D / 32; ++st) qf[st] = r < GU ? frag_load(qrow + 32 * st + 8 * qq) : frag_zero<F>();
  }
  F kf[KT][D / 32];
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    const T* kr = krow(min(64 * wave + 16 * t + r, n_act - 1)) + 8 * qq;
#pragma unroll
    for (int st = 0; st < D / 32; ++st) kf[t][st] = frag_load(kr + 32 * st);
  }
  asm volatile("" ::: "memory");
  copy_v();

  // Scores of this wave's 64 keys; lane (r, qq) holds row r, keys 64 w + 16 t + 4 qq + i.
  float s[KT][4];
  float mloc = -INFINITY;
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < D / 32; ++st) acc = mfma_step(kf[t][st], qf[st], acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = 64 * wave + 16 * t + 4 * qq + i;
      s[t][i] = key < n_act ? acc[i] * a.scale_log2 : -INFINITY;
      mloc = fmaxf(mloc, s[t][i]);
    }
  }
  mloc = fmaxf(mloc, __shfl_xor(mloc, 16, kWave));
  mloc = fmaxf(mloc, __shfl_xor(mloc, 32, kWave));
  if (qq == 0) mxs[wave][r] = mloc;
  stage_barrier<CPW>();  // the wave maxima visible; V copies may still be in flight
  const float m = fmaxf(fmaxf(mxs[0][r], mxs[1][r]), fmaxf(mxs[2][r], mxs[3][r]));
  if (r < GU) {
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      const int key0 = 64 * wave + 16 * t + 4 * qq;
      f32x4 p;
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = split_weight(s[t][i], m, key0 + i < n_act);
      *reinterpret_cast<f32x4*>(&Ps[r][key0]) = p;
    }
  }
  const int64_t pbase = ((int64_t)b * a.Hq + h0) * a.nsplit + split;
  if (wave == 0 && qq == 0 && r < GU) a.pm[pbase + (int64_t)r * a.nsplit] = m;
  stage_barrier<0>();  // V landed (own copies: vmcnt; everyone's: the barrier); weights visible

  // P.V over the split's 8 key steps, this wave's dim tiles of each V slice
  // (dims 16 dt, dt = wave, wave + 4, ...); wave 0 also the weight sum.
  f32x4 lsum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int vp = 0; vp < NVP; ++vp) {
    if (vp > 0) {
      __syncthreads();                                  // every wave is done with the previous slice
      vdim0 = vp * DV;
      copy_v();
      stage_barrier<0>();
    }
    f32x4 acc[(NDTV + 3) / 4];
#pragma unroll
    for (int j = 0; j < (NDTV + 3) / 4; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
    for (int ks = 0; ks < kSplit / 32; ++ks) {
      float p8[8];
      if (r < GU) {
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(&Ps[r][32 * ks + 4 * qq]);
        const f32x4 x1 = *reinterpret_cast<const f32x4*>(&Ps[r][32 * ks + 16 + 4 * qq]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          p8[e] = x0[e];
          p8[4 + e] = x1[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) p8[e] = 0.f;
      }
      const PFrag<T> pf = make_pfrag<T>(p8);
#pragma unroll
      for (int j = 0; j < (NDTV + 3) / 4; ++j) {
        const int dt = wave + 4 * j;
        if (dt < NDTV) acc[j] = pv_step<T>(pf, KV::vfrag(Vs, 32 * ks, dt, lane), acc[j]);
      }
      if (vp == 0 && wave == 0) lsum = pv_step<T>(pf, ones_frag<T>(), lsum);
    }

#pragma unroll
    for (int j = 0; j < (NDTV + 3) / 4; ++j) {
      const int dt = wave + 4 * j;
      if (dt >= NDTV) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 4 * qq + i;
        if (row < GU) a.pacc[(pbase + (int64_t)row * a.nsplit) * D + vp * DV + 16 * dt + r] = acc[j][i];
      }
    }
  }
  if (wave == 0 && r == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * qq + i;
      if (row < GU) a.pl[pbase + (int64_t)row * a.nsplit] = lsum[i];
    }
  }
  __syncthreads();  // every wave is done with Vs, Ps and mxs before the next item's copies
  }
}

// ---------------------------------------------------------------------------
// Prefill: one 256-thread workgroup per (sequence, kv head, 64 (token, head)
// rows, token-major); wave w owns the 16 rows 16 w .. 16 w + 15 of them (the
// columns of its score tiles). K and V stream through a ring of NBUF LDS
// buffers of CH keys (prefill_ring, prefill_chunk), shared by the four waves:
// per split, the K chunks (each wave scores its rows against the chunk's keys,
// scores kept
// in registers), the split maximum and weights (in registers), then the V
// chunks (P.V and the weight sum), then the in-register merge. Chunk
// c + NBUF - 1 is requested right after the barrier that opens chunk c. Only the chunks the
// workgroup's rows need are loaded (the last split may be short); rows past
// a row's causal or kv_lens limit are masked.
// ---------------------------------------------------------------------------
// Ring depth of the prefill kernel: 2 chunk buffers (one chunk requested
// ahead of the one being computed). Measured at the config-4 shape (bf16,
// D = 128, causal T = 2048), B = 1 / 4 / 16: 0.133 / 0.412 / 1.497 ms with 2
// buffers against 0.141 / 0.440 / 1.520 with 3 and 0.138 / 0.424 / 1.521 with
// 5: the smaller ring leaves LDS for more workgroups per CU, and the other
// resident workgroups hide a chunk's copy better than a deeper ring does.
template <typename T, int D>
constexpr int prefill_ring() {
  return 2;
}

// Keys per ring chunk: 128 for contiguous caches whose rows are at most 256
// bytes (16-bit D <= 128), else 64 (paged caches address 64-key segments).
// A chunk costs a barrier and its copy issue; 128-key chunks halve both per
// split.
template <typename T, int D, int MODE>
constexpr int prefill_chunk() {
  return MODE == kKvContig && D * (int)sizeof(T) <= 256 ? 128 : 64;
}

// Workgroups per CU the prefill kernel's registers are held to: two (two
// waves per SIMD, 256 registers each) for a contiguous cache of a 16-bit type
// with D <= 128, which fits that budget without spilling; otherwise no bound
// (D >= 192 needs more registers per wave; the paged forms' addressing takes
// a few more registers and would spill under the bound).
template <typename T, int D, int MODE>
constexpr int prefill_min_blocks() {
  return sizeof(T) == 2 && D <= 128 && MODE == kKvContig ? 2 : 1;
}

template <typename T, int D, int MODE, int NBUF = prefill_ring<T, D>(), int CH = prefill_chunk<T, D, MODE>()>
__global__ __launch_bounds__(256, (prefill_min_blocks<T, D, MODE>())) void attn_prefill_mfma(PrefillArgs a) {
  constexpr bool ROWPAGED = MODE == kKvRowPaged;
  typedef typename Frag<T>::type F;
  typedef KVTile<T, D> KV;
  static_assert(CH == 64 || (CH == 128 && MODE == kKvContig), "attn_prefill_mfma: chunk size");
  constexpr int KC = kSplit / CH;                       // chunks per split (of K, then of V)
  constexpr int TPC = CH / 16;                          // 16-key score tiles per chunk
  constexpr int CHB = CH * KV::kRowBytes;               // bytes per chunk
  static_assert(NBUF >= 2 && NBUF <= 5 && NBUF * CHB <= (160 << 10), "attn_prefill_mfma: ring depth");
  constexpr int PF = NBUF - 1;                          // chunks requested ahead of the current one
  constexpr int CPW = KV::copies(CH) / 4;               // copy instructions per wave per chunk
  constexpr int NDT = D / 16;
  static_assert(CPW >= 1, "attn_prefill_mfma: chunk copy tiling");
  __shared__ __attribute__((aligned(1024))) char ring[NBUF * CHB];

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int r = lane % 16, qq = lane / 16;
  const int G = a.Hq / a.Hkv;
  const int npairs = a.Tq * G;
  // Work items (sequence b, kv head hk, workgroup wg of 64 (token, head)
  // pairs) in that nesting order, each (b, hk)'s workgroups heaviest (latest
  // tokens) first. The 1-D grid is padded to a multiple of 8 and block i runs
  // item (i % 8) per_xcd + i / 8: workgroups are dispatched to the 8 XCDs
  // round-robin, so each XCD walks its own contiguous range of items and its
  // L2 holds the K/V of about one (b, hk) at a time rather than of every
  // (b, hk) the whole grid has in flight.
  const int wgs = (npairs + 63) / 64;
  const int64_t items = (int64_t)wgs * a.Hkv * a.B;
  const int64_t per_xcd = (items + 7) / 8;
  const int64_t item = (int64_t)(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (item >= items) return;  // uniform per workgroup, before any barrier
  const int wg = wgs - 1 - (int)(item % wgs);
  const int hk = (int)(item / wgs % a.Hkv);
  const int b = (int)(item / wgs / a.Hkv);
  const int len = a.kv_lens ? min(max(a.kv_lens[b], 0), a.L) : a.L;
  auto nkeys_of = [&](int pair) -> int {
    if (pair >= npairs) return 0;
    return a.causal ? len - a.Tq + pair / G + 1 : len;
  };
  const int last_pair = min(64 * wg + 63, npairs - 1);
  const int maxkeys = nkeys_of(last_pair);              // keys the workgroup needs (nkeys grows with the token)
  const int my_pair = 64 * wg + 16 * wave + r;          // score-layout row of this lane
  const int my_nkeys = nkeys_of(my_pair);
  int acc_nkeys[4];                                     // accumulator-layout rows 4 qq + i
#pragma unroll
  for (int i = 0; i < 4; ++i) acc_nkeys[i] = nkeys_of(64 * wg + 16 * wave + 4 * qq + i);

  const T* qb = static_cast<const T*>(a.q) + (int64_t)b * a.q_sb;
  const T* kbase = static_cast<const T*>(a.k);
  const T* vbase = static_cast<const T*>(a.v);
  // Contiguous cache: this (sequence, kv head)'s rows, once per workgroup.
  const T* kb = kbase + (int64_t)b * a.k_sb + (int64_t)hk * a.k_sh;
  const T* vb = vbase + (int64_t)b * a.v_sb + (int64_t)hk * a.v_sh;

  F qf[D / 32];
  {
    const bool ok = my_pair < npairs;
    const T* qrow = qb + (ok ? (int64_t)(hk * G + my_pair % G) * a.q_sh + (int64_t)(my_pair / G) * a.q_st : 0);
#pragma unroll
    for (int st = 0; st < D / 32; ++st) qf[st] = ok ? frag_load(qrow + 32 * st + 8 * qq) : frag_zero<F>();
  }

  // Chunk schedule: split sp has nkc(sp) = KC chunks of CH keys (the last
  // split: enough for maxkeys), K chunks then V chunks.
  const int nsplit = maxkeys > 0 ? (maxkeys + kSplit - 1) / kSplit : 0;
  const int last_keys = nsplit > 0 ? maxkeys - (nsplit - 1) * kSplit : 0;
  const int nkc_last = (last_keys + CH - 1) / CH;
  const int nchunks = nsplit > 0 ? 2 * KC * (nsplit - 1) + 2 * nkc_last : 0;
  // Contiguous cache: a chunk's copies go through a buffer resource whose
  // base is the chunk's first row and whose range ends at the sequence's last
  // key, with a per-lane byte offset that is the same for every chunk (the
  // lane's row of the chunk times the row stride, plus its 16-byte piece of
  // the row), computed once here: no per-copy address arithmetic. Rows past
  // the sequence read as zero (their keys are masked and their weights are
  // exactly 0). The host keeps 64 rows of either stride below 2^30 bytes.
  int koff[CPW], voff[CPW];
  if constexpr (MODE == kKvContig) {
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
      const int f = 64 * (wave * CPW + i) + lane;
      const int rr = f / KV::kCPR, slot = f - rr * KV::kCPR;
      const int cc = KV::kSwz ? (slot ^ (rr & 7)) : slot;
      koff[i] = (int)((rr * a.k_sl + cc * (16 / (int)sizeof(T))) * (int64_t)sizeof(T));
      voff[i] = (int)((rr * a.v_sl + cc * (16 / (int)sizeof(T))) * (int64_t)sizeof(T));
    }
  }
  auto issue = [&](int c) {
    if (c >= nchunks) return;
    int sp, kind, kc;
    if (c < 2 * KC * (nsplit - 1)) {
      sp = c / (2 * KC); kind = (c % (2 * KC)) / KC; kc = c % KC;
    } else {
      const int cl = c - 2 * KC * (nsplit - 1);
      sp = nsplit - 1; kind = cl / nkc_last; kc = cl % nkc_last;
    }
    const int key0 = sp * kSplit + kc * CH;
    const int64_t sl = kind ? a.v_sl : a.k_sl;
    char* buf = ring + (c % NBUF) * CHB;
    if constexpr (MODE == kKvContig) {
      const int rows = min(CH, len - key0);             // >= 1: chunks start below maxkeys <= len
      const auto rs = buffer_rsrc((kind ? vb : kb) + (int64_t)key0 * sl, (int)(rows * sl * (int64_t)sizeof(T)));
      char* dst = buf + 1024 * wave * CPW;
      if (kind) {
#pragma unroll
        for (int i = 0; i < CPW; ++i) copy_to_lds16(rs, voff[i], dst + 1024 * i);
      } else {
#pragma unroll
        for (int i = 0; i < CPW; ++i) copy_to_lds16(rs, koff[i], dst + 1024 * i);
      }
    } else {
      const T* segp = nullptr;                          // chunks are aligned 64-key segments
      if constexpr (MODE == kKvPaged) {
        segp = kind ? kv_segment<MODE>(a, vbase, a.v_sb, a.v_sh, sl, b, hk, key0)
                    : kv_segment<MODE>(a, kbase, a.k_sb, a.k_sh, sl, b, hk, key0);
      }
      auto row = [&](int i) {
        if constexpr (ROWPAGED)
          return kind ? vbase + kv_row_off(a, a.v_sb, a.v_sh, sl, b, hk, key0 + i)
                      : kbase + kv_row_off(a, a.k_sb, a.k_sh, sl, b, hk, key0 + i);
        else return segp + (int64_t)i * sl;
      };
#pragma unroll
      for (int i = 0; i < CPW; ++i) KV::copy(buf, wave * CPW + i, row, len - key0, lane);
    }
  };
  auto open_chunk = [&](int c) {
    // Chunk c landed; the min(PF - 1, nchunks - 1 - c) chunks requested after
    // it may still be in flight (copies complete in issue order).
    const int ahead = min(PF - 1, nchunks - 1 - c);
    if (PF >= 4 && ahead >= 3) stage_barrier<3 * CPW>();
    else if (PF >= 3 && ahead >= 2) stage_barrier<2 * CPW>();
    else if (PF >= 2 && ahead >= 1) stage_barrier<CPW>();
    else stage_barrier<0>();
    issue(c + PF);                              // every wave is past chunk c - 1: its buffer is free
  };

  float M[4], Lsum[4];
  f32x4 A[NDT];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    M[i] = -INFINITY;
    Lsum[i] = 0.0f;
  }
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) A[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int c = 0; c < PF; ++c) issue(c);
  int ci = 0;
  // A split entirely below every valid row's key limit needs no per-key mask
  // (the wave's first row has the smallest limit; padding rows past npairs
  // are never stored and MFMA rows do not interact): the same arithmetic on
  // every active key, without the compares and selects.
  const int wave_min_nkeys = __builtin_amdgcn_readfirstlane(nkeys_of(64 * wg + 16 * wave));
  auto split_body = [&](const int sp, auto masked) {
    constexpr bool MASKED = decltype(masked)::value;
    const int j0 = sp * kSplit;
    // An unmasked split lies below every valid row's key limit, so it is a
    // whole split of the workgroup too (its last split then holds 256 keys).
    const int nkc = !MASKED || sp + 1 < nsplit ? KC : nkc_last;
    // Scores of the wave's 16 rows against the split's keys (tile t: keys j0 + 16 t + ...).
    float s[16][4];
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      if (kc < nkc) {
        open_chunk(ci);
        const char* buf = ring + (ci % NBUF) * CHB;
        // Key j0 + CH kc + 16 t + 4 qq + i is below this row's limit iff
        // 16 t + i < lim: one lane value per chunk against constants.
        const int lim = my_nkeys - (j0 + CH * kc + 4 * qq);
#pragma unroll
        for (int t = 0; t < TPC; ++t) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int st = 0; st < D / 32; ++st) acc = mfma_step(KV::kfrag(buf, 16 * t + r, st, qq), qf[st], acc);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            s[TPC * kc + t][i] = (!MASKED || 16 * t + i < lim) ? acc[i] * a.scale_log2 : -INFINITY;
        }
        ++ci;
      } else {
#pragma unroll
        for (int t = 0; t < TPC; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) s[TPC * kc + t][i] = -INFINITY;
      }
    }
    float m = -INFINITY;
#pragma unroll
    for (int t = 0; t < 16; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) m = fmaxf(m, s[t][i]);
    m = fmaxf(m, __shfl_xor(m, 16, kWave));
    m = fmaxf(m, __shfl_xor(m, 32, kWave));
    // Weights exp2(s - m): a masked key's score is -inf, so its weight is
    // exactly +0 (v_exp_f32(-inf) = 0), the value an active-key select gives.
    // A row with no active key in the split (m = -inf; such a row is not
    // merged) subtracts 0 instead, so its weights are 0 rather than NaN.
    const float msub = MASKED && m == -INFINITY ? 0.0f : m;
#pragma unroll
    for (int t = 0; t < 16; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) s[t][i] = __builtin_amdgcn_exp2f(s[t][i] - msub);

    // P.V and the weight sum over the split's V chunks.
    f32x4 acc[NDT];
    f32x4 lsum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      if (kc < nkc) {
        open_chunk(ci);
        const char* buf = ring + (ci % NBUF) * CHB;
#pragma unroll
        for (int h = 0; h < CH / 32; ++h) {
          const int t0 = TPC * kc + 2 * h;
          float p8[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            p8[e] = s[t0][e];
            p8[4 + e] = s[t0 + 1][e];
          }
          const PFrag<T> pf = make_pfrag<T, !ROWPAGED>(p8);
          // The P.V steps at raised wave priority: while they issue, the
          // SIMD's other wave (the other resident workgroup, usually in its
          // score or weight phase) gets the vector ALU only between them.
          // Measured at config 4, B = 16: 1.236 -> 1.177 ms; the same around
          // the whole V chunk 1.236, around the score steps 1.278.
          __builtin_amdgcn_s_setprio(1);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) acc[dt] = pv_step<T>(pf, KV::vfrag(buf, 32 * h, dt, lane), acc[dt]);
          __builtin_amdgcn_s_setprio(0);
          lsum = pv_step<T>(pf, ones_frag<T>(), lsum);
        }
        ++ci;
      }
    }
    // Merge into the running state (accumulator layout: rows 4 qq + i). A
    // row whose keys end before the split skips it; in an unmasked split every
    // valid row has keys in it (padding rows are merged too, never stored).
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float mi = __shfl(m, 4 * qq + i, kWave);
      if (!MASKED || acc_nkeys[i] > j0) {
        float ai[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) ai[dt] = A[dt][i];
        float acci[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) acci[dt] = acc[dt][i];
        merge_split<NDT>(M[i], Lsum[i], ai, mi, lsum[i], acci);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) A[dt][i] = ai[dt];
      }
    }
  };
  for (int sp = 0; sp < nsplit; ++sp) {
    if (sp * kSplit + kSplit <= wave_min_nkeys) split_body(sp, std::false_type());
    else split_body(sp, std::true_type());
  }

#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int pair = 64 * wg + 16 * wave + 4 * qq + i;
    if (pair >= npairs) continue;
    T* o = static_cast<T*>(a.out) +
           ((((int64_t)b * a.Hq + hk * G + pair % G) * a.Tq) + pair / G) * D + r;
    // A row with no key (causal chunk longer than its sequence's kv_lens, or
    // a length of 0) has Lsum == 0: its output is defined as 0.
    const bool any = Lsum[i] > 0.0f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[16 * dt] = to_store<T>(any ? A[dt][i] / Lsum[i] : 0.0f);
  }
}

}  // namespace bi
