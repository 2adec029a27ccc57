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
// One 32-lane half of a wave runs one unit, as one simdgroup does in the
// reference: decode (b, kv head, chunk of NQ query heads, split), prefill (b,
// query head, kPkQB queries). The halves of a wave never exchange data (shuffles
// of width 32) and each half's control flow is uniform. A unit loads the K
// and V rows of several keys before running their updates in key order.
#pragma once

#include "bi_attn_api.h"

namespace bi {

// exp(x) of an fp32 argument: the double-precision exponential rounded once to
// fp32. That is the correctly rounded fp32 exp unless the double result lies
// within the double routine's error of an fp32 rounding midpoint.
__device__ __forceinline__ float exp_cr(float x) { return (float)exp((double)x); }

// Keys whose K/V rows a unit holds at once (about 64 registers of rows).
template <int DL>
constexpr int pk_ahead() { return DL >= 4 ? 32 / DL : 8; }

// The xor butterfly 16, 8, 4, 2, 1 within each 32-lane half, each step
// part + part[lane ^ off], without LDS-routed shuffles: xor 16 and 4 by
// ds_swizzle (bitmask mode: and 0x1f, xor off, within 32 lanes), xor 8 by a
// DPP row rotation of 8 (in a 16-lane row, i + 8 mod 16 == i ^ 8), xor 2 and
// 1 by DPP quad permutations. The same pairs as __shfl_xor(part, off, 32), so
// the same sums (measured 7% faster per-key decode than the shuffles).
__device__ __forceinline__ float pk_swizzle_xor16(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x1F | (16 << 10)));
}
__device__ __forceinline__ float pk_swizzle_xor4(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x1F | (4 << 10)));
}
template <int CTRL>
__device__ __forceinline__ float pk_dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppRowRor8 = 0x128, kDppQuadXor2 = 0x4E, kDppQuadXor1 = 0xB1;  // quad_perm [2,3,0,1] / [1,0,3,2]

template <int DL>
__device__ __forceinline__ float pk_score(const float (&qs)[DL], const float (&k)[DL]) {
  float part = 0.0f;
#pragma unroll
  for (int d = 0; d < DL; ++d) part = __builtin_fmaf(qs[d], k[d], part);
  part = part + pk_swizzle_xor16(part);
  part = part + pk_dpp<kDppRowRor8>(part);
  part = part + pk_swizzle_xor4(part);
  part = part + pk_dpp<kDppQuadXor2>(part);
  part = part + pk_dpp<kDppQuadXor1>(part);
  return part;
}

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

// Keys [j0, j1) of (sequence b, kv head hk) for NQ queries; query iq takes
// key j only if j < nkeys[iq] (its score is still computed: every lane of
// the half-wave takes part in the butterfly).
//
// A block of AH keys is evaluated in three passes with the recurrence's own
// values and order:
//   1. the scores of every (key, query) (each lane ends up with all of them);
//   2. per query, key by key: m' = max(m, s) for its active keys, and the two
//      exp arguments m - m' and s - m' (the maxima depend on the scores only);
//   3. every exp of the block once, one argument per lane of the half-wave
//      (all 32 lanes hold the same arguments), then back to every lane by a
//      shuffle, and the updates l = fma(l, corr, p), acc = fma(acc, corr, p v)
//      in key order.
// The same numbers as evaluating the recurrence key by key on every lane
// (which computed each exp 32 times).
template <typename T, int DL, int NQ, class Args>
__device__ __forceinline__ void pk_span(const Args& a, int b, int hk, int lane, int j0, int j1,
                                        const float (&qs)[NQ][DL], const int (&nkeys)[NQ], float (&m)[NQ],
                                        float (&l)[NQ], float (&acc)[NQ][DL]) {
  constexpr int AH = pk_ahead<DL>();
  constexpr int NE = 2 * AH * NQ;              // exp arguments per block: (corr, p) per (key, query)
  constexpr int ROUNDS = (NE + 31) / 32;       // exps per lane per block
  const T* kbase = static_cast<const T*>(a.k) + lane * DL;
  const T* vbase = static_cast<const T*>(a.v) + lane * DL;
  for (int j = j0; j < j1; j += AH) {
    float kr[AH][DL], vr[AH][DL];
#pragma unroll
    for (int u = 0; u < AH; ++u) {
      const int jj = min(j + u, j1 - 1);
      pk_load<T, DL>(kbase + kv_row_off(a, a.k_sb, a.k_sh, a.k_sl, b, hk, jj), kr[u]);
      pk_load<T, DL>(vbase + kv_row_off(a, a.v_sb, a.v_sh, a.v_sl, b, hk, jj), vr[u]);
    }
    // Passes 1 and 2: scores, running maxima, and this lane's exp arguments
    // (argument 2 (u NQ + iq) is corr, + 1 is p; lane i of round r takes
    // argument 32 r + i).
    float ein[ROUNDS];
#pragma unroll
    for (int r = 0; r < ROUNDS; ++r) ein[r] = 0.0f;
#pragma unroll
    for (int u = 0; u < AH; ++u) {
#pragma unroll
      for (int iq = 0; iq < NQ; ++iq) {
        const float s = pk_score<DL>(qs[iq], kr[u]);
        const bool act = j + u < j1 && j + u < nkeys[iq];
        const float m_new = act ? fmaxf(m[iq], s) : m[iq];
        const int i = 2 * (u * NQ + iq);
        if (lane == i % 32) ein[i / 32] = m[iq] - m_new;
        if (lane == (i + 1) % 32) ein[(i + 1) / 32] = s - m_new;
        m[iq] = m_new;
      }
    }
    float e[ROUNDS];
#pragma unroll
    for (int r = 0; r < ROUNDS; ++r) e[r] = exp_cr(ein[r]);
    // Pass 3: the updates in key order.
#pragma unroll
    for (int u = 0; u < AH; ++u) {
      if (j + u >= j1) break;
#pragma unroll
      for (int iq = 0; iq < NQ; ++iq) {
        const int i = 2 * (u * NQ + iq);
        const float corr = __shfl(e[i / 32], i % 32, 32);
        const float p = __shfl(e[(i + 1) / 32], (i + 1) % 32, 32);
        if (j + u < nkeys[iq]) {
          l[iq] = __builtin_fmaf(l[iq], corr, p);
#pragma unroll
          for (int d = 0; d < DL; ++d) acc[iq][d] = __builtin_fmaf(acc[iq][d], corr, p * vr[u][d]);
        }
      }
    }
  }
}

// Decode: unit = (b, kv head hk, chunk of NQ query heads, split), split
// fastest; writes (m, l, acc) of each head's split for attn_combine_perkey.
// Splits at or past the sequence's length are no unit's work.
template <typename T, int D, int NQ>
__global__ __launch_bounds__(256) void attn_decode_perkey(DecodeArgs a) {
  constexpr int DL = D / 32;
  const int lane = threadIdx.x % 32;
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
  pk_span<T, DL, NQ>(a, b, hk, lane, j0, j1, qs, nkeys, m, l, acc);
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
// fastest (QB = kPkQB).
// Query t sees keys [0, nkeys(t)), nkeys = len - Tq + t + 1 when causal
// (bottom-right aligned), else len; a split merges into a query's running
// result only if the query saw one of its keys.
template <typename T, int D>
__global__ __launch_bounds__(256) void attn_prefill_perkey(PrefillArgs a) {
  constexpr int DL = D / 32, QB = kPkQB;
  const int lane = threadIdx.x % 32;
  const int nblk = (a.Tq + QB - 1) / QB;
  int64_t u = (int64_t)blockIdx.x * 8 + threadIdx.x / 32;
  if (u >= (int64_t)a.B * a.Hq * nblk) return;
  const int blk = (int)(u % nblk);
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
    pk_span<T, DL, QB>(a, b, hk, lane, j0, min(nmax, j0 + a.split), qs, nkeys, m, l, acc);
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
  const int64_t units = (int64_t)a.B * a.Hq * ((a.Tq + kPkQB - 1) / kPkQB);
  attn_prefill_perkey<T, D><<<(unsigned)((units + 7) / 8), 256, 0, st>>>(a);
  return bi_host::launch_status("bi_attn_prefill_per_key");
}

}  // namespace bi
