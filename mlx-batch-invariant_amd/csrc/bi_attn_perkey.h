// bi_attn_perkey.h — attention in the reference's own per-key order, on the
// vector ALUs (mlx-batch-invariant kernels/attention.py: canonical order
// :1-32, _KEY_UPDATE :47-75, _MERGE :77-85, decode :87-147, combine :149-171,
// prefill :173-254). The matrix-core kernels of bi_attn_mfma.h compute the
// same quantity in another order; these are for callers who need the
// reference order's values, which the CPU oracle restates bit for bit.
//
// Canonical order, per (sequence, head, query):
//   q is pre-scaled once: qs[d] = fp32(float(q[d]) * scale);
//   score of key j: 32 lane partials, lane l owning dims [l DL, l DL + DL)
//     (DL = D / 32) accumulated in dim order with fma from 0, then folded by
//     the xor butterfly 16, 8, 4, 2, 1 over the 32 lanes (every lane ends up
//     with the same sum: the reference's lane-0 value);
//   inside a split, key by key for the active keys:
//     m' = max(m, s); corr = exp(m - m'); p = exp(s - m');
//     l = fma(l, corr, p); acc[d] = fma(acc[d], corr, p * v[d]); m = m';
//   splits of a.split keys (256 unless the caller picks another size, as the
//   reference's split_size) merged left to right from M = -inf, L = 0, A = 0:
//     M' = max(M, m); c_old = exp(M - M'); c_new = exp(m - M');
//     L = fma(L, c_old, l * c_new); A[d] = fma(A[d], c_old, acc[d] * c_new);
//   out[d] = T(A[d] / L) (IEEE division; 0 for a row that sees no key).
// exp is the fp32 exponential rounded from double precision, exp_cr below
// (the reference asks for metal::precise::exp; this build fixes the rounding).
//
// One 32-lane half of a wave runs one unit: decode (b, kv head, chunk of NQ
// query heads, split), prefill (b, query head, pk_prefill_qb(D) queries). The
// halves of a wave never exchange data (shuffles of width 32) and each half's
// control flow is uniform. The reference evaluates a key's score on 32 lanes
// (one per partial) and its butterfly on every lane; here the lanes compute
// the partials of a block of keys, then each lane folds one (query, key)'s 32
// partials by the butterfly's own tree (pk_span): the same sums, once.
#pragma once

#include <type_traits>

#include "bi_attn_api.h"

namespace bi {

// exp(x) of an fp32 argument: the double-precision exponential rounded once to
// fp32. That is the correctly rounded fp32 exp unless the double result lies
// within the double routine's error of an fp32 rounding midpoint.
__device__ __forceinline__ float exp_cr(float x) { return (float)exp((double)x); }

// Keys whose K/V rows a unit holds at once (about 64 registers of rows).
template <int DL>
constexpr int pk_ahead() { return DL >= 4 ? 32 / DL : 8; }

template <int DL>
__device__ __forceinline__ void pk_merge(float& M, float& L, float* A, float m, float l, const float* acc) {
  const float M_new = fmaxf(M, m);
  const float c_old = exp_cr(M - M_new);
  const float c_new = exp_cr(m - M_new);
  L = __builtin_fmaf(L, c_old, l * c_new);
#pragma unroll
  for (int d = 0; d < DL; ++d) A[d] = __builtin_fmaf(A[d], c_old, acc[d] * c_new);
  M = M_new;
}

template <typename T, int DL>
__device__ __forceinline__ void pk_load(const T* p, float (&out)[DL]) {
#pragma unroll
  for (int d = 0; d < DL; ++d) out[d] = (float)p[d];
}

template <typename T, int DL>
__device__ __forceinline__ void pk_load_q(const T* row, float scale, float (&qs)[DL]) {
  pk_load<T, DL>(row, qs);
#pragma unroll
  for (int d = 0; d < DL; ++d) qs[d] = qs[d] * scale;
}

// A unit's LDS: the lane partials of a key block (32 keys x 32 lanes for one
// query, KB = 32 / NQ keys x 32 lanes x NQ queries in general) and the
// block's (corr, p) pairs, per query and key.
constexpr int kPkTable = 32 * 32;
constexpr int kPkPairs = 2 * 32;
constexpr int kPkUnitFloats = kPkTable + kPkPairs;

// Keys per block of a unit scoring NQ queries: one (query, key) score per lane.
template <int NQ>
constexpr int pk_block() { return 32 / NQ; }

constexpr int pk_pow2_floor(int n) { return n >= 16 ? 16 : n >= 8 ? 8 : n >= 4 ? 4 : n >= 2 ? 2 : 1; }

// NQ floats stored as one LDS write.
template <int NQ> struct PkVec { typedef float type __attribute__((ext_vector_type(NQ))); };
template <> struct PkVec<1> {
  struct type {
    float x;
    __device__ float& operator[](int) { return x; }
  };
};

// The xor butterfly 16, 8, 4, 2, 1 of 32 lane partials, evaluated by one lane:
// level k adds the value of lane i + h to that of lane i (h = 16, 8, 4, 2, 1),
// which is what lane 0 of the butterfly computes (every lane of it computes
// the same sums in the other operand order, and the adds commute).
__device__ __forceinline__ float pk_tree(float (&v)[32]) {
#pragma unroll
  for (int h = 16; h >= 1; h >>= 1)
#pragma unroll
    for (int i = 0; i < h; ++i) v[i] = v[i] + v[i + h];
  return v[0];
}

// Inclusive prefix maximum over the G consecutive lanes of a group (G = 8, 16
// or 32 within a 32-lane half; lanes of a group are the keys of one query in
// key order). The maximum is exact and order-free (v_max_f32 treats -0 < +0;
// NaN operands are dropped as by fmaxf), so the scan equals the key-by-key
// running maximum.
template <int G>
__device__ __forceinline__ float pk_scan_max(float x, int jl) {
#pragma unroll
  for (int off = 1; off < G; off <<= 1) {
    const float y = __shfl_up(x, off, G);
    x = jl >= off ? fmaxf(x, y) : x;
  }
  return x;
}

// Keys [j0, j1) of (sequence b, kv head hk) for NQ queries; query iq takes
// key j only if j < nkeys[iq]. tb / cp: the unit's LDS (kPkTable / kPkPairs
// floats, written and read back by this half-wave only: DS operations of one
// wave complete in order).
//
// Blocks of KB = 32 / NQ keys, in three phases with the recurrence's own
// values and order:
//   1. lanes own dims: lane l's score partials of every (key, query) of the
//      block (fma chains over its DL dims from 0), written to LDS;
//   2. lanes own (query q, key j): the 32 partials of (q, j) read back and
//      folded by the butterfly's tree (pk_tree), the running maximum of the
//      query's active keys by an exact prefix-maximum scan, and the key's
//      corr = exp(m_prev - m') (1 when the maximum did not move: exp(0) = 1)
//      and p = exp(s - m'), each evaluated once;
//   3. lanes own dims again: l = fma(l, corr, p), acc = fma(acc, corr, p v)
//      for every query in key order, (corr, p) read from LDS.
// The same numbers as evaluating the recurrence key by key with the
// butterfly on every lane; the K / V rows of a block are converted once for
// all NQ queries. Blocks whose keys every query takes (FULL) run without
// per-key checks and address row jb + u as the block's row pointer plus u
// row strides. The cache is contiguous (the per-key entry points take no
// page table).
template <typename T, int DL, int NQ, class Args>
__device__ __forceinline__ void pk_span(const Args& a, int b, int hk, int lane, int j0, int j1,
                                             const float (&qs)[NQ][DL], const int (&nkeys)[NQ], float (&m)[NQ],
                                             float (&l)[NQ], float (&acc)[NQ][DL], float* __restrict__ tb,
                                             float* __restrict__ cp) {
  constexpr int KB = pk_block<NQ>();
  constexpr int AH = pk_pow2_floor(pk_ahead<DL>() < KB ? pk_ahead<DL>() : KB);   // rows held at once
  static_assert(KB % AH == 0, "pk_span: whole row batches per block");
  typedef typename PkVec<NQ>::type qvec;
  const int jl = lane % KB, ql = lane / KB;    // phase 2: key jl of the block, query ql
  int kend[NQ];
  int kend_q = 0, kmin = j1;
  float mq = m[0];
#pragma unroll
  for (int iq = 0; iq < NQ; ++iq) {
    kend[iq] = min(j1, nkeys[iq]);
    kmin = min(kmin, kend[iq]);
    if (ql == iq) {
      kend_q = kend[iq];
      mq = m[iq];
    }
  }
  // The lane's elements of row 0 of (b, hk).
  const T* kbase = static_cast<const T*>(a.k) + lane * DL + (int64_t)b * a.k_sb + (int64_t)hk * a.k_sh;
  const T* vbase = static_cast<const T*>(a.v) + lane * DL + (int64_t)b * a.v_sb + (int64_t)hk * a.v_sh;
  auto krow = [&](int j) -> const T* { return kbase + (int64_t)j * a.k_sl; };
  auto vrow = [&](int j) -> const T* { return vbase + (int64_t)j * a.v_sl; };

  auto block = [&](int jb, auto full_t) {
    constexpr bool FULL = decltype(full_t)::value;
    // Row u0 + u of the block: row jb + u0 + u, or (partial blocks) the last
    // row of the span in place of rows past it.
    auto rowp = [&](auto rowf, int64_t sl, int u) -> const T* {
      if constexpr (FULL) return rowf(jb) + (int64_t)u * sl;
      else return rowf(min(jb + u, j1 - 1));
    };
    // Phase 1: partial of lane l for (key u, query iq) at tb[(u 32 + (l ^ u)) NQ + iq]
    // (the xor spreads the 32 readers of phase 2 over distinct banks).
#pragma unroll 1
    for (int u0 = 0; u0 < KB; u0 += AH) {
      float kr[AH][DL];
#pragma unroll
      for (int u = 0; u < AH; ++u) pk_load<T, DL>(rowp(krow, a.k_sl, u0 + u), kr[u]);
#pragma unroll
      for (int u = 0; u < AH; ++u) {
        qvec pq;
#pragma unroll
        for (int iq = 0; iq < NQ; ++iq) {
          float part = 0.0f;
#pragma unroll
          for (int d = 0; d < DL; ++d) part = __builtin_fmaf(qs[iq][d], kr[u][d], part);
          pq[iq] = part;
        }
        *reinterpret_cast<qvec*>(tb + ((u0 + u) * 32 + (lane ^ (u0 + u))) * NQ) = pq;
      }
    }
    asm volatile("" ::: "memory");
    // Phase 2.
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = tb[(jl * 32 + (i ^ jl)) * NQ + ql];
    const float s = pk_tree(v);
    const bool act = FULL || jb + jl < kend_q;
    const float mj = fmaxf(mq, pk_scan_max<KB>(act ? s : -INFINITY, jl));
    float mp = __shfl_up(mj, 1, KB);
    mp = jl == 0 ? mq : mp;
    mq = __shfl(mj, ql * KB + KB - 1, 32);
    const float carg = mp - mj;
    float corr = 1.0f;
    if (carg != 0.0f) corr = exp_cr(carg);
    const float p = exp_cr(s - mj);
    *reinterpret_cast<float2*>(cp + 2 * (ql * KB + jl)) = float2{corr, p};
    asm volatile("" ::: "memory");
    // Phase 3.
#pragma unroll 1
    for (int u0 = 0; u0 < KB; u0 += AH) {
      float vr[AH][DL];
#pragma unroll
      for (int u = 0; u < AH; ++u) pk_load<T, DL>(rowp(vrow, a.v_sl, u0 + u), vr[u]);
#pragma unroll
      for (int u = 0; u < AH; ++u) {
        const int key = jb + u0 + u;
#pragma unroll
        for (int iq = 0; iq < NQ; ++iq) {
          if (FULL || key < kend[iq]) {
            const float2 e = *reinterpret_cast<const float2*>(cp + 2 * (iq * KB + u0 + u));
            l[iq] = __builtin_fmaf(l[iq], e.x, e.y);
#pragma unroll
            for (int d = 0; d < DL; ++d) acc[iq][d] = __builtin_fmaf(acc[iq][d], e.x, e.y * vr[u][d]);
          }
        }
      }
    }
    asm volatile("" ::: "memory");
  };
  int jb = j0;
  for (; jb + KB <= kmin; jb += KB) block(jb, std::true_type());
  for (; jb < j1; jb += KB) block(jb, std::false_type());
#pragma unroll
  for (int iq = 0; iq < NQ; ++iq) m[iq] = __shfl(mq, iq * KB, 32);
}

// Decode: unit = (b, kv head hk, chunk of NQ query heads, split), split
// fastest; writes (m, l, acc) of each head's split for attn_combine_perkey.
// Splits at or past the sequence's length are no unit's work.
template <typename T, int D, int NQ>
__global__ __launch_bounds__(256) void attn_decode_perkey(DecodeArgs a) {
  constexpr int DL = D / 32;
  __shared__ __attribute__((aligned(16))) float lds[8][kPkUnitFloats];
  const int lane = threadIdx.x % 32;
  float* tb = lds[threadIdx.x / 32];
  int64_t u = (int64_t)blockIdx.x * 8 + threadIdx.x / 32;
  if (u >= (int64_t)a.B * a.Hkv * a.nchunk * a.nsplit) return;
  const int split = (int)(u % a.nsplit);
  u /= a.nsplit;
  const int chunk = (int)(u % a.nchunk);
  u /= a.nchunk;
  const int hk = (int)(u % a.Hkv);
  const int b = (int)(u / a.Hkv);
  const int h0 = hk * (a.Hq / a.Hkv) + chunk * NQ;
  const int len = a.kv_lens ? min(max(a.kv_lens[b], 0), a.L) : a.L;
  const int j0 = split * a.split, j1 = min(len, j0 + a.split);
  if (j0 >= j1) return;
  float qs[NQ][DL], m[NQ], l[NQ], acc[NQ][DL];
  int nkeys[NQ];
#pragma unroll
  for (int iq = 0; iq < NQ; ++iq) {
    pk_load_q<T, DL>(static_cast<const T*>(a.q) + (int64_t)b * a.q_sb + (int64_t)(h0 + iq) * a.q_sh + lane * DL,
                         a.scale, qs[iq]);
    nkeys[iq] = len;
    m[iq] = -INFINITY;
    l[iq] = 0.0f;
#pragma unroll
    for (int d = 0; d < DL; ++d) acc[iq][d] = 0.0f;
  }
  pk_span<T, DL, NQ>(a, b, hk, lane, j0, j1, qs, nkeys, m, l, acc, tb, tb + kPkTable);
#pragma unroll
  for (int iq = 0; iq < NQ; ++iq) {
    const int64_t po = ((int64_t)b * a.Hq + h0 + iq) * a.nsplit + split;
    if (lane == 0) {
      a.pm[po] = m[iq];
      a.pl[po] = l[iq];
    }
#pragma unroll
    for (int d = 0; d < DL; ++d) a.pacc[po * D + lane * DL + d] = acc[iq][d];
  }
}

// One thread per (sequence, head, d): the sequence's own splits merged left to
// right, then the division.
template <typename T, int D>
__global__ __launch_bounds__(256) void attn_combine_perkey(DecodeArgs a) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (int64_t)a.B * a.Hq * D) return;
  const int64_t bh = gid / D;
  const int d = (int)(gid % D);
  const int b = (int)(bh / a.Hq);
  const int len = a.kv_lens ? min(max(a.kv_lens[b], 0), a.L) : a.L;
  const int ns = (len + a.split - 1) / a.split;
  float M = -INFINITY, Ls = 0.0f, A = 0.0f;
  for (int i = 0; i < ns; ++i) {
    const int64_t po = bh * a.nsplit + i;
    const float acc = a.pacc[po * D + d];
    pk_merge<1>(M, Ls, &A, a.pm[po], a.pl[po], &acc);
  }
  static_cast<T*>(a.out)[bh * D + d] = to_store<T>(Ls > 0.0f ? A / Ls : 0.0f);
}

// Prefill: unit = (b, query head h, queries QB blk .. QB blk + QB - 1), blk
// fastest and latest (most keys) first (QB = pk_prefill_qb(D)); a workgroup
// runs 8 consecutive units, one per half-wave. The 1-D grid is padded to a
// multiple of 8 and block i runs workgroup (i mod 8) ceil(nwg / 8) + i / 8:
// workgroups reach the 8 XCDs round-robin, so each XCD walks its own range of
// heads and its L2 holds about one head's K/V rather than those of every head
// in flight.
// Query t sees keys [0, nkeys(t)), nkeys = len - Tq + t + 1 when causal
// (bottom-right aligned), else len; a split merges into a query's running
// result only if the query saw one of its keys.
template <typename T, int D>
__global__ __launch_bounds__(256) void attn_prefill_perkey(PrefillArgs a) {
  constexpr int DL = D / 32, QB = pk_prefill_qb(D);
  __shared__ __attribute__((aligned(16))) float lds[8][kPkUnitFloats];
  const int lane = threadIdx.x % 32;
  float* tb = lds[threadIdx.x / 32];
  const int nblk = (a.Tq + QB - 1) / QB;
  const int64_t units = (int64_t)a.B * a.Hq * nblk;
  const int64_t nwg = (units + 7) / 8;
  const int64_t wg = (int64_t)(blockIdx.x % 8) * ((nwg + 7) / 8) + blockIdx.x / 8;
  int64_t u = wg * 8 + threadIdx.x / 32;
  if (wg >= nwg || u >= units) return;   // half-waves are independent: no barrier below
  const int blk = nblk - 1 - (int)(u % nblk);
  u /= nblk;
  const int h = (int)(u % a.Hq);
  const int b = (int)(u / a.Hq);
  const int hk = h / (a.Hq / a.Hkv);
  const int len = a.kv_lens ? min(max(a.kv_lens[b], 0), a.L) : a.L;
  const int t0 = blk * QB;
  int nkeys[QB];
  float qs[QB][DL], M[QB], Ls[QB], A[QB][DL];
  int nmax = 0;
#pragma unroll
  for (int iq = 0; iq < QB; ++iq) {
    const int t = min(t0 + iq, a.Tq - 1);
    nkeys[iq] = t0 + iq < a.Tq ? max(0, a.causal ? len - a.Tq + t + 1 : len) : 0;
    nmax = max(nmax, nkeys[iq]);
    pk_load_q<T, DL>(static_cast<const T*>(a.q) + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh +
                             (int64_t)t * a.q_st + lane * DL,
                         a.scale, qs[iq]);
    M[iq] = -INFINITY;
    Ls[iq] = 0.0f;
#pragma unroll
    for (int d = 0; d < DL; ++d) A[iq][d] = 0.0f;
  }
  for (int j0 = 0; j0 < nmax; j0 += a.split) {
    float m[QB], l[QB], acc[QB][DL];
#pragma unroll
    for (int iq = 0; iq < QB; ++iq) {
      m[iq] = -INFINITY;
      l[iq] = 0.0f;
#pragma unroll
      for (int d = 0; d < DL; ++d) acc[iq][d] = 0.0f;
    }
    pk_span<T, DL, QB>(a, b, hk, lane, j0, min(nmax, j0 + a.split), qs, nkeys, m, l, acc, tb, tb + kPkTable);
#pragma unroll
    for (int iq = 0; iq < QB; ++iq)
      if (j0 < nkeys[iq]) pk_merge<DL>(M[iq], Ls[iq], A[iq], m[iq], l[iq], acc[iq]);
  }
#pragma unroll
  for (int iq = 0; iq < QB; ++iq) {
    if (t0 + iq >= a.Tq) continue;
    T* o = static_cast<T*>(a.out) + (((int64_t)b * a.Hq + h) * a.Tq + t0 + iq) * D + lane * DL;
#pragma unroll
    for (int d = 0; d < DL; ++d) o[d] = to_store<T>(Ls[iq] > 0.0f ? A[iq][d] / Ls[iq] : 0.0f);
  }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------

template <typename T, int D>
int launch_decode_perkey(DecodeArgs& a, hipStream_t st) {
  const unsigned blocks = (unsigned)(((int64_t)a.B * a.Hkv * a.nchunk * a.nsplit + 7) / 8);
  switch (a.GU) {
    case 4: attn_decode_perkey<T, D, 4><<<blocks, 256, 0, st>>>(a); break;
    case 2: attn_decode_perkey<T, D, 2><<<blocks, 256, 0, st>>>(a); break;
    default: attn_decode_perkey<T, D, 1><<<blocks, 256, 0, st>>>(a); break;
  }
  int rc = bi_host::launch_status("bi_attn_decode_per_key");
  if (rc) return rc;
  const int64_t n = (int64_t)a.B * a.Hq * D;
  attn_combine_perkey<T, D><<<(unsigned)((n + 255) / 256), 256, 0, st>>>(a);
  return bi_host::launch_status("bi_attn_decode_per_key(combine)");
}

template <typename T, int D>
int launch_prefill_perkey(PrefillArgs& a, hipStream_t st) {
  constexpr int QB = pk_prefill_qb(D);
  const int64_t units = (int64_t)a.B * a.Hq * ((a.Tq + QB - 1) / QB);
  const int64_t nwg = (units + 7) / 8;
  attn_prefill_perkey<T, D><<<(unsigned)(8 * ((nwg + 7) / 8)), 256, 0, st>>>(a);
  return bi_host::launch_status("bi_attn_prefill_per_key");
}

}  // namespace bi
