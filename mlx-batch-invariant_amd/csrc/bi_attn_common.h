// bi_attn_common.h — the per-split arithmetic of batch-invariant attention,
// shared verbatim by the decode kernel, the decode combine kernel and the
// prefill kernel (the reference keeps its in-split update and split merge as
// one source text used by both of its kernels for the same reason:
// kernels/attention.py:44-85, `_KEY_UPDATE` and `_MERGE`).
//
// Canonical order for one (sequence, head, query) with key count n:
//   keys are cut into fixed splits [256 i, 256 i + 256) in index order
//   (reference kernels/attention.py:6-8);
//   score s_j = fp32( MFMA-dot(k_j, q) * (scale * log2 e) ): a chain of
//     v_mfma_f32_16x16x32 steps over D (K rows as the A operand, Q^T as B,
//     d-slot map d = 32 st + 8 quarter + e);
//   per split with n_act >= 1 active keys:
//     m   = max of the active s_j (exact, so independent of evaluation order);
//     p_j = exp2(s_j - m) for active keys (v_exp_f32), exactly 0 otherwise;
//     acc[d] and l are MFMA chains over the split's 8 steps of 32 keys, step
//       ks holding keys 32 ks + {4 q + i, 16 + 4 q + i} in k-slots
//       (q, i) / (q, 4 + i): for 16-bit types each step adds hi(P).V then
//       lo(P).V, hi = T(p), lo = T(p - hi) (together 16 (bf16) / 22 (f16)
//       significant bits of p); for fp32 one fp32 step with P as is; l uses
//       the same steps with V = 1;
//   splits are merged left to right from M = -inf, L = 0, A = 0:
//       M' = max(M, m); c_old = exp2(M - M'); c_new = exp2(m - M')
//       L = fmaf(L, c_old, l * c_new); A[d] = fmaf(A[d], c_old, acc[d] * c_new)
//   out[d] = T(A[d] / L).
//
// The reference runs the softmax recurrence key by key inside a split
// (m' = max(m, s); corr = exp(m - m'); l = fma(l, corr, p); acc = fma(acc,
// corr, p v)). That is the same quantity evaluated in another order: on this
// GPU its per-(row, key, dim) fp32 chains keep the prefill kernel on the
// vector ALUs at a fraction of the matrix cores' rate, so here the split
// maximum comes first and every product runs on the MFMA units. Results agree
// with the reference order to fp32 rounding (the attention tests check one
// storage ulp against the oracle, which follows the reference order); the
// invariance properties (batch size, chunking, decode == prefill) hold because
// every row runs this one sequence whichever kernel computes it.
#pragma once

#include <type_traits>

#include "bi_common.h"

namespace bi {

constexpr float kLog2e = 1.44269504088896340736f;
constexpr int kMaxDev = 64;  // devices the host-side per-device caches cover

struct DecodeArgs {
  const void* q;
  const void* k;
  const void* v;
  const int32_t* kv_lens;
  float* pm;
  float* pl;
  float* pacc;
  unsigned* ctr;  // decode item counter (dynamic item order only), zero at launch
  void* out;
  int B, Hq, Hkv, L, nsplit, nchunk, GU;
  int64_t q_sb, q_sh, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl;
  float scale_log2;  // scale * log2(e), rounded once on the host
  float scale;       // the caller's scale (per-key order)
  int split;         // keys per split (per-key order; the matrix-core kernels use kSplit)
  // Paged K/V (null table = contiguous): see kv_row_off.
  const int32_t* table;
  int64_t table_stride;
  int page_shift;
  int num_pages;  // pages in the pool; table entries are clamped to [0, num_pages)
};

struct PrefillArgs {
  const void* q;
  const void* k;
  const void* v;
  const int32_t* kv_lens;
  void* out;
  int B, Hq, Hkv, Tq, L, causal;
  int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl;
  float scale_log2;
  float scale;
  int split;
  const int32_t* table;
  int64_t table_stride;
  int page_shift;
  int num_pages;
};

// Element offset of key `pos` of (sequence b, kv head hk) in a K or V cache
// with strides (sb, sh, sl). Contiguous (a.table null): b sb + hk sh + pos sl.
// Paged: the cache is a pool of pages of 2^page_shift keys, sb the page
// stride; key pos of sequence b lives in page table[b table_stride +
// (pos >> page_shift)] at row pos mod 2^page_shift. Addressing only: the
// arithmetic of every split is the same either way. A table entry outside
// [0, num_pages) is clamped into the pool, as lengths are clamped to L: a
// stale or corrupt table gives wrong values, never a read outside the pool.
__device__ __forceinline__ int clamp_page(int page, int num_pages) { return min(max(page, 0), num_pages - 1); }

template <class Args>
__device__ __forceinline__ int64_t kv_row_off(const Args& a, int64_t sb, int64_t sh, int64_t sl, int b, int hk,
                                              int pos) {
  if (a.table) {
    const int page = clamp_page(a.table[(int64_t)b * a.table_stride + (pos >> a.page_shift)], a.num_pages);
    return (int64_t)page * sb + (int64_t)hk * sh + (int64_t)(pos & ((1 << a.page_shift) - 1)) * sl;
  }
  return (int64_t)b * sb + (int64_t)hk * sh + (int64_t)pos * sl;
}

// A 32-bit read through the scalar data cache, for a wave-uniform address: it
// does not queue behind the wave's (or the CU's) vector memory traffic. The
// wait is inside the statement, so the compiler's own counters stay exact.
__device__ __forceinline__ int load_uniform_i32(const int32_t* p) {
  int v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
  return v;
}

// K/V addressing mode of a kernel instantiation: a contiguous cache, a paged
// one with pages of 64 keys or more, or one with smaller pages.
enum KvMode { kKvContig = 0, kKvPaged = 1, kKvRowPaged = 2 };

// The K/V rows a kernel reads come in aligned 64-key segments (a decode wave's
// keys of a split, a prefill chunk). Pointer to the first element of segment
// key `key0` (a multiple of 64) of (sequence b, kv head hk) for kKvContig and
// kKvPaged (one wave-uniform table read per segment; a page of 64 keys or
// more holds the whole segment); rows of the segment are then `sl` elements
// apart. kKvRowPaged kernels resolve every row through kv_row_off instead.
template <int MODE, typename T, class Args>
__device__ __forceinline__ const T* kv_segment(const Args& a, const T* base, int64_t sb, int64_t sh, int64_t sl,
                                               int b, int hk, int key0) {
  if constexpr (MODE == kKvContig) {
    return base + (int64_t)b * sb + (int64_t)hk * sh + (int64_t)key0 * sl;
  } else {
    const int page =
        clamp_page(load_uniform_i32(a.table + (int64_t)b * a.table_stride + (key0 >> a.page_shift)), a.num_pages);
    return base + (int64_t)page * sb + (int64_t)hk * sh + (int64_t)(key0 & ((1 << a.page_shift) - 1)) * sl;
  }
}

// Weight of one key of a split: exp2(s - m) if active, exactly 0 otherwise.
__device__ __forceinline__ float split_weight(float s, float m, bool active) {
  return active ? __builtin_amdgcn_exp2f(s - m) : 0.0f;
}

// The A operand of one P.V step: 8 weights of one row (k-slots 0..7).
template <typename T> struct PFrag;
template <> struct PFrag<bf16> { bf16x8 hi, lo; };
template <> struct PFrag<f16> { f16x8 hi, lo; };
template <> struct PFrag<float> { f32x8 f; };

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// PAIRED (bf16): the hi halves of a pair of weights come from one packed
// conversion; both forms round the same values the same way, so they give the
// same bits (a kernel picks the one that fits its register budget).
template <typename T, bool PAIRED = true>
__device__ __forceinline__ PFrag<T> make_pfrag(const float (&p)[8]) {
  PFrag<T> r;
  if constexpr (PAIRED && std::is_same_v<T, bf16>) {
    // Per pair of weights: one packed round-to-nearest-even conversion gives
    // both hi halves; their fp32 values are the converted bits moved to the
    // top half (an exact widening), so the residuals p - hi are the same
    // exact differences, rounded once by the second packed conversion.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bf16x2_t h = __builtin_convertvector(f32x2_t{p[2 * j], p[2 * j + 1]}, bf16x2_t);
      const uint32_t hb = __builtin_bit_cast(uint32_t, h);
      const float h0 = __builtin_bit_cast(float, hb << 16);
      const float h1 = __builtin_bit_cast(float, hb & 0xffff0000u);
      const bf16x2_t l = __builtin_convertvector(f32x2_t{p[2 * j] - h0, p[2 * j + 1] - h1}, bf16x2_t);
      r.hi[2 * j] = h[0];
      r.hi[2 * j + 1] = h[1];
      r.lo[2 * j] = l[0];
      r.lo[2 * j + 1] = l[1];
    }
  } else if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const T h = to_store<T>(p[e]);
      r.hi[e] = h;
      r.lo[e] = to_store<T>(p[e] - (float)h);  // exact difference, rounded once
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      r.f.lo[e] = p[e];
      r.f.hi[e] = p[4 + e];
    }
  }
  return r;
}

template <typename T>
__device__ __forceinline__ f32x4 pv_step(const PFrag<T>& pf, typename Frag<T>::type b, f32x4 acc) {
  if constexpr (sizeof(T) == 2) {
    acc = mfma_step(pf.hi, b, acc);
    return mfma_step(pf.lo, b, acc);
  } else {
    return mfma_step(pf.f, b, acc);
  }
}

template <typename T>
__device__ __forceinline__ typename Frag<T>::type ones_frag() {
  typename Frag<T>::type f;
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (T)1.0f;
  } else {
    f.lo = f32x4{1.f, 1.f, 1.f, 1.f};
    f.hi = f.lo;
  }
  return f;
}

// ---- split merge -------------------------------------------------------------
template <int DL>
__device__ __forceinline__ void merge_split(float& M, float& L, float* A, float m, float l,
                                            const float* acc) {
  const float M_new = fmaxf(M, m);
  const float c_old = __builtin_amdgcn_exp2f(M - M_new);
  const float c_new = __builtin_amdgcn_exp2f(m - M_new);
  L = __builtin_fmaf(L, c_old, l * c_new);
#pragma unroll
  for (int d = 0; d < DL; ++d) A[d] = __builtin_fmaf(A[d], c_old, acc[d] * c_new);
  M = M_new;
}

}  // namespace bi
