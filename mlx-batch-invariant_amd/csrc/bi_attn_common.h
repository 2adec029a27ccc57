// bi_attn_common.h — the per-key online-softmax update and the split merge,
// shared verbatim by the decode kernel, the decode combine kernel and the
// prefill kernel (reference: kernels/attention.py:44-85, `_KEY_UPDATE` and
// `_MERGE`, which are likewise one source text used by both kernels).
//
// Canonical order for one (sequence, head, query) with key count n:
//   keys are cut into fixed splits [256 i, 256 i + 256) in index order;
//   score s_j = fp32( MFMA-dot(q, k_j) * scale ), the dot taken by a chain of
//     v_mfma_f32_16x16x32 steps over D with d-slot map d = 32 s + 8 quarter + e;
//   inside a split, from m = -inf, l = 0, acc = 0, for each key j in order:
//       m' = max(m, s_j); corr = expf(m - m'); p = expf(s_j - m')
//       l = fmaf(l, corr, p);  acc[d] = fmaf(acc[d], corr, p * v_j[d]);  m = m'
//   splits that hold at least one of the n keys are merged left to right from
//   M = -inf, L = 0, A = 0:
//       M' = max(M, m); c_old = expf(M - M'); c_new = expf(m - M')
//       L = fmaf(L, c_old, l * c_new); A[d] = fmaf(A[d], c_old, acc[d] * c_new)
//   out[d] = T(A[d] / L).
//
// The recurrence is evaluated in an equivalent parallel form: the running
// maxima m_j are a prefix maximum over the split (max is exact, so any
// evaluation order gives the same values), corr_j and p_j depend only on
// (m_{j-1}, m_j, s_j) and are computed for all keys at once, and only the
// l / acc chains run key by key. Every value equals the sequential one.
#pragma once

#include "bi_common.h"

namespace bi {

// ---- scores ----------------------------------------------------------------
// One 16-key column tile of scores: A operand = 16 query rows (qf, one
// fragment per 32-wide d step), B operand = keys key0 + r. Keys at or beyond
// `nvalid` are not loaded (zero operand). Result register i of lane l is the
// raw dot of row 4 (l/16) + i with key key0 + l % 16.
template <typename T, int D>
__device__ __forceinline__ f32x4 score_tile(const typename Frag<T>::type* qf, const T* kbase,
                                            int64_t kstride, int key0, int nvalid, int lane) {
  typedef typename Frag<T>::type F;
  const int r = lane % 16, q = lane / 16;
  const bool ok = r < nvalid;
  const T* kr = kbase + (int64_t)(key0 + (ok ? r : 0)) * kstride + 8 * q;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < D / 32; ++s) {
    const F kf = ok ? frag_load(kr + 32 * s) : frag_zero<F>();
    acc = mfma_step(qf[s], kf, acc);
  }
  return acc;
}

// Query fragment of one row for the score MFMA (A operand): d = 32 s + 8 q + e.
template <typename T, int D>
__device__ __forceinline__ void load_q_frags(typename Frag<T>::type* qf, const T* qrow, bool valid,
                                             int lane) {
  typedef typename Frag<T>::type F;
  const int q = lane / 16;
#pragma unroll
  for (int s = 0; s < D / 32; ++s) qf[s] = valid ? frag_load(qrow + 32 * s + 8 * q) : frag_zero<F>();
}

// ---- per-key softmax weights of one split, one row, one wave ----------------
// s: this lane's 4 scores (keys 4l .. 4l+3 of the split); keys at or beyond
// n_act (>= 1) are ignored by the caller. Returns p_j and corr_j of the
// lane's keys and, in m_last, m at the last active key.
struct SplitWeights {
  f32x4 p, corr;
  float m_last;
};
__device__ __forceinline__ SplitWeights split_weights_core(f32x4 s, int n_act, int lane) {
  float loc = fmaxf(fmaxf(fmaxf(s[0], s[1]), s[2]), s[3]);
  float incl = loc;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const float o = __shfl_up(incl, off, kWave);
    if (lane >= off) incl = fmaxf(incl, o);
  }
  float prev = __shfl_up(incl, 1, kWave);
  if (lane == 0) prev = -INFINITY;
  SplitWeights w;
  float mk[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float m_new = fmaxf(prev, s[k]);
    w.corr[k] = expf(prev - m_new);
    w.p[k] = expf(s[k] - m_new);
    mk[k] = m_new;
    prev = m_new;
  }
  const int last = n_act - 1;
  const float mine = mk[last & 3];
  w.m_last = __shfl(mine, last >> 2, kWave);
  return w;
}

// S_row: 256 scores in LDS. Writes PC_row[j] = (p_j, corr_j) for every key
// and returns m at the last active key. Lane l owns keys 4l .. 4l+3.
__device__ __forceinline__ float split_weights(const float* S_row, float2* PC_row, int n_act,
                                               int lane) {
  const SplitWeights w = split_weights_core(reinterpret_cast<const f32x4*>(S_row)[lane], n_act, lane);
  const f32x4 out01 = {w.p[0], w.corr[0], w.p[1], w.corr[1]};
  const f32x4 out23 = {w.p[2], w.corr[2], w.p[3], w.corr[3]};
  reinterpret_cast<f32x4*>(PC_row)[2 * lane] = out01;
  reinterpret_cast<f32x4*>(PC_row)[2 * lane + 1] = out23;
  return w.m_last;
}

// Same weights, p written over the scores in SP_row and corr into C_row.
__device__ __forceinline__ float split_weights_inplace(float* SP_row, float* C_row, int n_act,
                                                       int lane) {
  const SplitWeights w = split_weights_core(reinterpret_cast<const f32x4*>(SP_row)[lane], n_act, lane);
  reinterpret_cast<f32x4*>(SP_row)[lane] = w.p;
  reinterpret_cast<f32x4*>(C_row)[lane] = w.corr;
  return w.m_last;
}

// ---- per-key accumulation over one split, one (row, DL dims) per lane -------
template <typename T, int DL>
__device__ __forceinline__ void load_dims(const T* p, float* out) {
  if constexpr (sizeof(T) == 2 && DL % 8 == 0) {
#pragma unroll
    for (int c = 0; c < DL / 8; ++c) {
      const u32x4 raw = reinterpret_cast<const u32x4*>(p)[c];
      const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
      for (int i = 0; i < 8; ++i) out[8 * c + i] = (float)e[i];
    }
  } else if constexpr (sizeof(T) == 4 && DL % 4 == 0) {
#pragma unroll
    for (int c = 0; c < DL / 4; ++c) {
      const f32x4 raw = reinterpret_cast<const f32x4*>(p)[c];
#pragma unroll
      for (int i = 0; i < 4; ++i) out[4 * c + i] = raw[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < DL; ++i) out[i] = (float)p[i];
  }
}

template <typename T, int DL>
__device__ __forceinline__ void split_accumulate(const float2* PC_row, const T* vbase,
                                                 int64_t vstride, int n_act, float& l,
                                                 float* acc) {
  l = 0.0f;
#pragma unroll
  for (int d = 0; d < DL; ++d) acc[d] = 0.0f;
  constexpr int U = 4;
  int j = 0;
  for (; j + U <= n_act; j += U) {
    float v[U][DL];
#pragma unroll
    for (int u = 0; u < U; ++u) load_dims<T, DL>(vbase + (int64_t)(j + u) * vstride, v[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float2 pc = PC_row[j + u];
      l = __builtin_fmaf(l, pc.y, pc.x);
#pragma unroll
      for (int d = 0; d < DL; ++d) acc[d] = __builtin_fmaf(acc[d], pc.y, pc.x * v[u][d]);
    }
  }
  for (; j < n_act; ++j) {
    float v[DL];
    load_dims<T, DL>(vbase + (int64_t)j * vstride, v);
    const float2 pc = PC_row[j];
    l = __builtin_fmaf(l, pc.y, pc.x);
#pragma unroll
    for (int d = 0; d < DL; ++d) acc[d] = __builtin_fmaf(acc[d], pc.y, pc.x * v[d]);
  }
}

// ---- split merge -------------------------------------------------------------
template <int DL>
__device__ __forceinline__ void merge_split(float& M, float& L, float* A, float m, float l,
                                            const float* acc) {
  const float M_new = fmaxf(M, m);
  const float c_old = expf(M - M_new);
  const float c_new = expf(m - M_new);
  L = __builtin_fmaf(L, c_old, l * c_new);
#pragma unroll
  for (int d = 0; d < DL; ++d) A[d] = __builtin_fmaf(A[d], c_old, acc[d] * c_new);
  M = M_new;
}

}  // namespace bi
