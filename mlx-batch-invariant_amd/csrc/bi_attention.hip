// bi_attention.hip — batch-invariant split-KV decode and prefill attention.
//
// Reference: kernels/attention.py of mlx-batch-invariant — decode kernel
// :87-147 (one simdgroup per (batch, kv head, head chunk, split), partials per
// split), combine :149-171 (left fold of splits, precise divide), prefill
// :173-254 (queries share K/V rows, splits folded in registers, bottom-right
// causal mask nkeys = L - Tq + t + 1). Arithmetic order: bi_attn_common.h.
//
// gfx950 layout:
//   decode  one wave64 per (sequence, kv head, head chunk of GU, split). The
//           GU query heads are rows of the score MFMA tile; the wave computes
//           256 scores per head with 64 MFMAs, the per-key weights with a wave
//           prefix-max, then runs the l/acc chains with lane = (head, D*GU/64
//           dims). Writes (m, l, acc) of its split.
//   combine one thread per (sequence, head, d); merges the sequence's own
//           ceil(len/256) splits left to right and divides.
//   prefill one 256-thread workgroup per (sequence, kv head, 16 (token, head)
//           rows, token-major). Each split: the 4 waves compute 64 keys of
//           scores each for all 16 rows, each wave derives the weights of 4
//           rows and then runs their l/acc chains (lane = (row, D/16 dims)),
//           merging into registers.
#include <type_traits>

#include "bi_attn_common.h"

namespace bi {

struct DecodeArgs {
  const void* q;
  const void* k;
  const void* v;
  const int32_t* kv_lens;
  float* pm;
  float* pl;
  float* pacc;
  void* out;
  int B, Hq, Hkv, L, nsplit, nchunk, GU;
  int64_t q_sb, q_sh, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl;
  float scale;
};

template <typename T, int D, int GU>
__global__ __launch_bounds__(kWave) void attn_decode_kernel(DecodeArgs a) {
  typedef typename Frag<T>::type F;
  constexpr int LPR = kWave / GU;  // lanes per head row in the accumulation phase
  constexpr int DL = D / LPR;      // dims per lane
  static_assert(DL >= 1 && D % LPR == 0, "bad decode tiling");
  __shared__ __attribute__((aligned(16))) float S[GU][kSplit];
  __shared__ __attribute__((aligned(16))) float2 PC[GU][kSplit];
  __shared__ float mfin[GU];

  const int lane = threadIdx.x;
  const int split = blockIdx.x;
  const int hk = blockIdx.y / a.nchunk;
  const int chunk = blockIdx.y % a.nchunk;
  const int b = blockIdx.z;
  // A length outside [0, L] is clamped, so no key past the cache is ever read.
  const int len = a.kv_lens ? min(max(a.kv_lens[b], 0), a.L) : a.L;
  const int j0 = split * kSplit;
  if (j0 >= len) return;  // this sequence has no keys in this split
  const int n_act = min(kSplit, len - j0);
  const int G = a.Hq / a.Hkv;
  const int h0 = hk * G + chunk * GU;

  const T* qb = static_cast<const T*>(a.q) + (int64_t)b * a.q_sb;
  const T* kb = static_cast<const T*>(a.k) + (int64_t)b * a.k_sb + (int64_t)hk * a.k_sh +
                (int64_t)j0 * a.k_sl;
  const T* vb = static_cast<const T*>(a.v) + (int64_t)b * a.v_sb + (int64_t)hk * a.v_sh +
                (int64_t)j0 * a.v_sl;

  // Phase 1: scores. A operand row r = head h0 + r (rows >= GU are zero).
  F qf[D / 32];
  {
    const int r = lane % 16;
    load_q_frags<T, D>(qf, qb + (int64_t)(h0 + (r < GU ? r : 0)) * a.q_sh, r < GU, lane);
  }
  for (int c = 0; c < kSplit / 16; ++c) {
    const int key0 = 16 * c;
    if (key0 >= n_act) {  // wave-uniform: the rest of the split is past the sequence end
      if (lane < 16)
#pragma unroll
        for (int rr = 0; rr < GU; ++rr) S[rr][key0 + lane] = -INFINITY;
      continue;
    }
    const f32x4 acc = score_tile<T, D>(qf, kb, a.k_sl, key0, n_act - key0, lane);
    const int key = key0 + lane % 16;
    const int row0 = 4 * (lane / 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = row0 + i;
      if (row < GU) S[row][key] = key < n_act ? acc[i] * a.scale : -INFINITY;
    }
  }
  __syncthreads();

  // Phase 2: per-key weights, one head row at a time.
  for (int h = 0; h < GU; ++h) {
    const float mf = split_weights(S[h], PC[h], n_act, lane);
    if (lane == 0) mfin[h] = mf;
  }
  __syncthreads();

  // Phase 3: l / acc chains.
  const int row = lane / LPR;
  const int dim0 = (lane % LPR) * DL;
  float l, acc[DL];
  split_accumulate<T, DL>(PC[row], vb + dim0, a.v_sl, n_act, l, acc);

  const int64_t po = ((int64_t)b * a.Hq + h0 + row) * a.nsplit + split;
#pragma unroll
  for (int d = 0; d < DL; ++d) a.pacc[po * D + dim0 + d] = acc[d];
  if (lane % LPR == 0) {
    a.pm[po] = mfin[row];
    a.pl[po] = l;
  }
}

// ---------------------------------------------------------------------------
// attn_decode_wg: the bandwidth-shaped decode launch, one 256-thread workgroup
// per (sequence, kv head, head chunk of GU, split), GU * D a multiple of 256.
// Every wave first requests all of its memory at once: the K rows of its 64
// keys (straight into registers, 16-byte loads, rows past the sequence end
// clamped to its last key) and a quarter of the split's V rows, which the
// load unit copies straight into LDS (global_load_lds_dwordx4, [key][D]).
// Scores (wave w: keys 64 w .. 64 w + 63, GU query heads as MFMA rows) and the
// per-key weights (one head per wave) run while V lands; the l / acc chains
// then read V from LDS (thread = (head, DL dims)). Same per-split arithmetic
// as attn_decode_kernel, same partial layout, same combine.
// ---------------------------------------------------------------------------
template <typename T, int D, int GU>
__global__ __launch_bounds__(256) void attn_decode_wg(DecodeArgs a) {
  typedef typename Frag<T>::type F;
  constexpr int kThreads = 256;
  static_assert((GU * D) % kThreads == 0, "attn_decode_wg: GU * D must be a multiple of 256");
  constexpr int DL = GU * D / kThreads;        // dims per thread in the l / acc phase
  constexpr int LPR = D / DL;                  // threads per head row
  constexpr int CE = 16 / (int)sizeof(T);      // elements per 16-byte chunk
  constexpr int CPR = D / CE;                  // chunks per V row
  constexpr int KPI = kWave / CPR;             // V rows per copy instruction
  constexpr int CPW = kSplit / KPI / 4;        // copy instructions per wave
  constexpr int KT = kSplit / 4 / 16;          // score tiles per wave
  static_assert(KPI >= 1 && (kSplit / KPI) % 4 == 0, "attn_decode_wg: V copy tiling");
  __shared__ __attribute__((aligned(1024))) T Vs[kSplit * D];
  __shared__ __attribute__((aligned(16))) float S[GU][kSplit];
  __shared__ __attribute__((aligned(16))) float2 PC[GU][kSplit];
  __shared__ float mfin[GU];

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int split = blockIdx.x;
  const int hk = blockIdx.y / a.nchunk;
  const int chunk = blockIdx.y % a.nchunk;
  const int b = blockIdx.z;
  // A length outside [0, L] is clamped, so no key past the cache is ever read.
  const int len = a.kv_lens ? min(max(a.kv_lens[b], 0), a.L) : a.L;
  const int j0 = split * kSplit;
  if (j0 >= len) return;  // uniform per workgroup, before any barrier
  const int n_act = min(kSplit, len - j0);
  const int G = a.Hq / a.Hkv;
  const int h0 = hk * G + chunk * GU;

  const T* qb = static_cast<const T*>(a.q) + (int64_t)b * a.q_sb;
  const T* kb = static_cast<const T*>(a.k) + (int64_t)b * a.k_sb + (int64_t)hk * a.k_sh +
                (int64_t)j0 * a.k_sl;
  const T* vb = static_cast<const T*>(a.v) + (int64_t)b * a.v_sb + (int64_t)hk * a.v_sh +
                (int64_t)j0 * a.v_sl;
  const int r = lane % 16, q = lane / 16;

  // Memory requests, in this order: q, this wave's K rows, this wave's V copies.
  F qf[D / 32];
  load_q_frags<T, D>(qf, qb + (int64_t)(h0 + (r < GU ? r : 0)) * a.q_sh, r < GU, lane);
  F kf[KT][D / 32];
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    const int key = min(64 * wave + 16 * t + r, n_act - 1);
    const T* kr = kb + (int64_t)key * a.k_sl + 8 * q;
#pragma unroll
    for (int st = 0; st < D / 32; ++st) kf[t][st] = frag_load(kr + 32 * st);
  }
  asm volatile("" ::: "memory");
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    const int ci = wave * CPW + c;                         // copy instruction of the split
    const int key = min(ci * KPI + lane / CPR, n_act - 1);
    copy_to_lds16(vb + (int64_t)key * a.v_sl + CE * (lane % CPR), Vs + ci * KPI * D);
  }

  // Scores of this wave's 64 keys (rows: the GU heads).
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < D / 32; ++st) acc = mfma_step(qf[st], kf[t][st], acc);
    const int key = 64 * wave + 16 * t + r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * q + i;
      if (row < GU) S[row][key] = key < n_act ? acc[i] * a.scale : -INFINITY;
    }
  }
  stage_barrier<CPW>();  // scores visible; this wave's V copies may still be in flight
  // Per-key weights, one head per wave.
  for (int h = wave; h < GU; h += 4) {
    const float mf = split_weights(S[h], PC[h], n_act, lane);
    if (lane == 0) mfin[h] = mf;
  }
  // V landed (this wave's copies: vmcnt; everyone's: the barrier).
  stage_barrier<0>();

  // l / acc chains over the split's keys, V from LDS.
  const int row = tid / LPR;
  const int dim0 = (tid % LPR) * DL;
  float l = 0.0f, acc[DL];
#pragma unroll
  for (int d = 0; d < DL; ++d) acc[d] = 0.0f;
  const float2* pcr = PC[row];
  const T* vs = Vs + dim0;
  int j = 0;
  for (; j + 8 <= n_act; j += 8) {
    float v[8][DL];
#pragma unroll
    for (int u = 0; u < 8; ++u) load_dims<T, DL>(vs + (j + u) * D, v[u]);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float2 pc = pcr[j + u];
      l = __builtin_fmaf(l, pc.y, pc.x);
#pragma unroll
      for (int d = 0; d < DL; ++d) acc[d] = __builtin_fmaf(acc[d], pc.y, pc.x * v[u][d]);
    }
  }
  for (; j < n_act; ++j) {
    float v[DL];
    load_dims<T, DL>(vs + j * D, v);
    const float2 pc = pcr[j];
    l = __builtin_fmaf(l, pc.y, pc.x);
#pragma unroll
    for (int d = 0; d < DL; ++d) acc[d] = __builtin_fmaf(acc[d], pc.y, pc.x * v[d]);
  }

  const int64_t po = ((int64_t)b * a.Hq + h0 + row) * a.nsplit + split;
#pragma unroll
  for (int d = 0; d < DL; ++d) a.pacc[po * D + dim0 + d] = acc[d];
  if (tid % LPR == 0) {
    a.pm[po] = mfin[row];
    a.pl[po] = l;
  }
}

template <typename T, int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(DecodeArgs a) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)a.B * a.Hq * D;
  if (gid >= total) return;
  const int64_t bh = gid / D;
  const int d = (int)(gid % D);
  const int b = (int)(bh / a.Hq);
  const int len = a.kv_lens ? min(max(a.kv_lens[b], 0), a.L) : a.L;
  const int ns = (len + kSplit - 1) / kSplit;
  float M = -INFINITY, Ls = 0.0f, A = 0.0f;
  for (int i = 0; i < ns; ++i) {
    const int64_t po = bh * a.nsplit + i;
    const float acc = a.pacc[po * D + d];
    merge_split<1>(M, Ls, &A, a.pm[po], a.pl[po], &acc);
  }
  static_cast<T*>(a.out)[bh * D + d] = to_store<T>(A / Ls);
}

struct PrefillArgs {
  const void* q;
  const void* k;
  const void* v;
  const int32_t* kv_lens;
  void* out;
  int B, Hq, Hkv, Tq, L, causal;
  int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl;
  float scale;
};

template <typename T, int D>
__global__ __launch_bounds__(256) void attn_prefill_kernel(PrefillArgs a) {
  typedef typename Frag<T>::type F;
  constexpr int DL = D / 16;  // 16 lanes per row, 4 rows per wave
  __shared__ __attribute__((aligned(16))) float S[16][kSplit];
  __shared__ __attribute__((aligned(16))) float2 PC[16][kSplit];
  __shared__ float mfin[16];

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int tile = blockIdx.x;
  const int hk = blockIdx.y;
  const int b = blockIdx.z;
  const int G = a.Hq / a.Hkv;
  const int npairs = a.Tq * G;
  const int len = a.kv_lens ? min(max(a.kv_lens[b], 0), a.L) : a.L;

  auto row_token = [&](int r) { return (tile * 16 + r) / G; };
  auto row_head = [&](int r) { return hk * G + (tile * 16 + r) % G; };
  auto row_valid = [&](int r) { return tile * 16 + r < npairs; };
  auto row_nkeys = [&](int r) {
    if (!row_valid(r)) return 0;
    return a.causal ? len - a.Tq + row_token(r) + 1 : len;
  };

  int maxkeys = 0;
#pragma unroll
  for (int r = 0; r < 16; ++r) maxkeys = max(maxkeys, row_nkeys(r));

  const T* qb = static_cast<const T*>(a.q) + (int64_t)b * a.q_sb;
  const T* kb = static_cast<const T*>(a.k) + (int64_t)b * a.k_sb + (int64_t)hk * a.k_sh;
  const T* vb = static_cast<const T*>(a.v) + (int64_t)b * a.v_sb + (int64_t)hk * a.v_sh;

  F qf[D / 32];
  {
    const int r = lane % 16;
    const bool ok = row_valid(r);
    const T* qrow = qb + (ok ? (int64_t)row_head(r) * a.q_sh + (int64_t)row_token(r) * a.q_st : 0);
    load_q_frags<T, D>(qf, qrow, ok, lane);
  }

  const int my_row = 4 * wave + lane / 16;
  const int dim0 = (lane % 16) * DL;
  const int my_nkeys = row_nkeys(my_row);
  float M = -INFINITY, Lsum = 0.0f, A[DL];
#pragma unroll
  for (int d = 0; d < DL; ++d) A[d] = 0.0f;

  const int nsplit = (maxkeys + kSplit - 1) / kSplit;
  for (int sp = 0; sp < nsplit; ++sp) {
    const int j0 = sp * kSplit;
    const int span = min(kSplit, maxkeys - j0);  // keys any row of the tile needs
    // Phase 1: wave w scores keys [64 w, 64 w + 64) of the split for all 16
    // rows. All of the wave's K loads are issued before the first MFMA
    // (unconditional: rows past the tile's last needed key are clamped to it).
    {
      const int r = lane % 16, q = lane / 16;
      const T* ks = kb + (int64_t)j0 * a.k_sl;
      F kf[4][D / 32];
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        const int key = min(64 * wave + 16 * cc + r, span - 1);
        const T* kr = ks + (int64_t)key * a.k_sl + 8 * q;
#pragma unroll
        for (int st = 0; st < D / 32; ++st) kf[cc][st] = frag_load(kr + 32 * st);
      }
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < D / 32; ++st) acc = mfma_step(qf[st], kf[cc][st], acc);
        const int key = 64 * wave + 16 * cc + r;
#pragma unroll
        for (int i = 0; i < 4; ++i) S[4 * q + i][key] = key < span ? acc[i] * a.scale : -INFINITY;
      }
    }
    __syncthreads();
    // Phase 2: wave w derives the weights of rows 4w .. 4w+3.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * wave + i;
      const int n_act = min(kSplit, row_nkeys(row) - j0);
      if (n_act > 0) {
        const float mf = split_weights(S[row], PC[row], n_act, lane);
        if (lane == 0) mfin[row] = mf;
      }
    }
    __syncthreads();
    // Phase 3: l / acc chains of this lane's row, then the in-register merge.
    const int n_act = min(kSplit, my_nkeys - j0);
    if (n_act > 0) {
      float l, acc[DL];
      split_accumulate<T, DL>(PC[my_row], vb + (int64_t)j0 * a.v_sl + dim0, a.v_sl, n_act, l, acc);
      merge_split<DL>(M, Lsum, A, mfin[my_row], l, acc);
    }
    __syncthreads();
  }

  if (row_valid(my_row)) {
    T* o = static_cast<T*>(a.out) +
           ((((int64_t)b * a.Hq + row_head(my_row)) * a.Tq) + row_token(my_row)) * D + dim0;
#pragma unroll
    for (int d = 0; d < DL; ++d) o[d] = to_store<T>(A[d] / Lsum);
  }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
static int decode_gu(int G) {
  for (int gu : {8, 4, 2, 1})
    if (G % gu == 0) return gu;
  return 1;
}

template <typename T, int D>
static int launch_decode(DecodeArgs& a, hipStream_t st) {
  dim3 grid(a.nsplit, a.Hkv * a.nchunk, a.B);
  if (a.GU * D >= 256) {
    switch (a.GU) {
      case 8: attn_decode_wg<T, D, 8><<<grid, 256, 0, st>>>(a); break;
      case 4: attn_decode_wg<T, D, 4><<<grid, 256, 0, st>>>(a); break;
      default:
        if constexpr (D == 128) attn_decode_wg<T, D, 2><<<grid, 256, 0, st>>>(a);
        break;
    }
  } else {
    switch (a.GU) {
      case 2: attn_decode_kernel<T, D, 2><<<grid, kWave, 0, st>>>(a); break;
      default: attn_decode_kernel<T, D, 1><<<grid, kWave, 0, st>>>(a); break;
    }
  }
  int rc = bi_host::launch_status("bi_attn_decode");
  if (rc) return rc;
  const int64_t n = (int64_t)a.B * a.Hq * D;
  attn_combine_kernel<T, D><<<(unsigned)((n + 255) / 256), 256, 0, st>>>(a);
  return bi_host::launch_status("bi_attn_decode(combine)");
}

template <typename T, int D>
static int launch_prefill(PrefillArgs& a, hipStream_t st) {
  const int G = a.Hq / a.Hkv;
  const int64_t tiles = ((int64_t)a.Tq * G + 15) / 16;
  dim3 grid((unsigned)tiles, a.Hkv, a.B);
  attn_prefill_kernel<T, D><<<grid, 256, 0, st>>>(a);
  return bi_host::launch_status("bi_attn_prefill");
}

}  // namespace bi

namespace {

int check_attn_shape(const char* what, int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t D) {
  using namespace bi_host;
  if (B < 0 || Hq <= 0 || Hkv <= 0 || L <= 0 || D <= 0)
    return fail(BI_E_INVALID_ARG, "%s: bad shape B=%lld Hq=%lld Hkv=%lld L=%lld D=%lld", what,
                (long long)B, (long long)Hq, (long long)Hkv, (long long)L, (long long)D);
  if (Hq % Hkv) return fail(BI_E_INVALID_ARG, "%s: Hq=%lld not a multiple of Hkv=%lld", what,
                            (long long)Hq, (long long)Hkv);
  if (D != 64 && D != 128)
    return fail(BI_E_UNSUPPORTED, "%s: head dim %lld (supported: 64, 128)", what, (long long)D);
  if (B > 65535 || Hkv > 65535 || L > 0x7fffffffLL - bi::kSplit || Hq > 0x7fffffffLL / 16)
    return fail(BI_E_UNSUPPORTED, "%s: shape exceeds the grid limits", what);
  return BI_OK;
}

}  // namespace

extern "C" size_t bi_attn_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t L, int64_t D) {
  if (B <= 0 || Hq <= 0 || L <= 0 || D <= 0) return 0;
  const int64_t ns = (L + bi::kSplit - 1) / bi::kSplit;
  const int64_t bh = B * Hq * ns;
  // pm | pl | pacc, each 16-byte aligned
  auto up = [](int64_t x) { return (x + 3) / 4 * 4; };
  return (size_t)(up(bh) * 2 + bh * D) * sizeof(float);
}

extern "C" int bi_attn_decode(const void* q, const void* k, const void* v, const int32_t* kv_lens,
                              void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t D,
                              const int64_t* strides, float scale, int dtype, void* ws,
                              size_t ws_bytes, void* stream) {
  using namespace bi_host;
  int rc = check_attn_shape("bi_attn_decode", B, Hq, Hkv, L, D);
  if (rc) return rc;
  if (B == 0) return BI_OK;
  if (!q || !k || !v || !out || !strides)
    return fail(BI_E_INVALID_ARG, "bi_attn_decode: null pointer argument");
  const size_t need = bi_attn_decode_workspace_bytes(B, Hq, L, D);
  if (!ws || ws_bytes < need)
    return fail(BI_E_WORKSPACE, "bi_attn_decode: workspace of %zu bytes required, got %zu", need,
                ws ? ws_bytes : (size_t)0);
  const size_t es = dtype_size(dtype);
  for (int i = 0; i < 8; ++i)
    if (strides[i] < 0 || ((strides[i] * (int64_t)es) % 16))
      return fail(BI_E_INVALID_ARG, "bi_attn_decode: stride %d (%lld) must be >= 0 and 16-byte aligned",
                  i, (long long)strides[i]);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(ws))
    return fail(BI_E_INVALID_ARG, "bi_attn_decode: q, k, v and workspace must be 16-byte aligned");
  bi::DecodeArgs a;
  a.q = q; a.k = k; a.v = v; a.kv_lens = kv_lens; a.out = out;
  a.B = (int)B; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.L = (int)L;
  a.nsplit = (int)((L + bi::kSplit - 1) / bi::kSplit);
  const int G = (int)(Hq / Hkv);
  a.GU = bi::decode_gu(G);
  a.nchunk = G / a.GU;
  a.q_sb = strides[0]; a.q_sh = strides[1];
  a.k_sb = strides[2]; a.k_sh = strides[3]; a.k_sl = strides[4];
  a.v_sb = strides[5]; a.v_sh = strides[6]; a.v_sl = strides[7];
  a.scale = scale;
  const int64_t bh = B * Hq * a.nsplit;
  const int64_t up = (bh + 3) / 4 * 4;
  a.pm = static_cast<float*>(ws);
  a.pl = a.pm + up;
  a.pacc = a.pl + up;
  if ((int64_t)a.Hkv * a.nchunk > 65535 || a.nsplit > 0x7fffffff)
    return fail(BI_E_UNSUPPORTED, "bi_attn_decode: grid too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
#define BI_DEC(TY)                                                         \
  return D == 64 ? bi::launch_decode<TY, 64>(a, st) : bi::launch_decode<TY, 128>(a, st);
  switch (dtype) {
    case BI_BF16: BI_DEC(bi::bf16)
    case BI_F16: BI_DEC(bi::f16)
    case BI_F32: BI_DEC(float)
    default: return fail(BI_E_UNSUPPORTED, "bi_attn_decode: unknown dtype %d", dtype);
  }
#undef BI_DEC
}

extern "C" int bi_attn_prefill(const void* q, const void* k, const void* v, const int32_t* kv_lens,
                               void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t L,
                               int64_t D, const int64_t* strides, int causal, float scale, int dtype,
                               void* stream) {
  using namespace bi_host;
  int rc = check_attn_shape("bi_attn_prefill", B, Hq, Hkv, L, D);
  if (rc) return rc;
  if (Tq <= 0) return fail(BI_E_INVALID_ARG, "bi_attn_prefill: Tq=%lld", (long long)Tq);
  if (causal && Tq > L)
    return fail(BI_E_INVALID_ARG, "bi_attn_prefill: causal needs Tq (%lld) <= L (%lld)",
                (long long)Tq, (long long)L);
  if (B == 0) return BI_OK;
  if (!q || !k || !v || !out || !strides)
    return fail(BI_E_INVALID_ARG, "bi_attn_prefill: null pointer argument");
  const size_t es = dtype_size(dtype);
  for (int i = 0; i < 9; ++i)
    if (strides[i] < 0 || ((strides[i] * (int64_t)es) % 16))
      return fail(BI_E_INVALID_ARG, "bi_attn_prefill: stride %d (%lld) must be >= 0 and 16-byte aligned",
                  i, (long long)strides[i]);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return fail(BI_E_INVALID_ARG, "bi_attn_prefill: q, k, v, out must be 16-byte aligned");
  const int64_t tiles = (Tq * (Hq / Hkv) + 15) / 16;
  if (tiles > 0x7fffffffLL) return fail(BI_E_UNSUPPORTED, "bi_attn_prefill: grid too large");
  bi::PrefillArgs a;
  a.q = q; a.k = k; a.v = v; a.kv_lens = kv_lens; a.out = out;
  a.B = (int)B; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.Tq = (int)Tq; a.L = (int)L;
  a.causal = causal ? 1 : 0;
  a.q_sb = strides[0]; a.q_sh = strides[1]; a.q_st = strides[2];
  a.k_sb = strides[3]; a.k_sh = strides[4]; a.k_sl = strides[5];
  a.v_sb = strides[6]; a.v_sh = strides[7]; a.v_sl = strides[8];
  a.scale = scale;
  hipStream_t st = static_cast<hipStream_t>(stream);
#define BI_PRE(TY)                                                           \
  return D == 64 ? bi::launch_prefill<TY, 64>(a, st) : bi::launch_prefill<TY, 128>(a, st);
  switch (dtype) {
    case BI_BF16: BI_PRE(bi::bf16)
    case BI_F16: BI_PRE(bi::f16)
    case BI_F32: BI_PRE(float)
    default: return fail(BI_E_UNSUPPORTED, "bi_attn_prefill: unknown dtype %d", dtype);
  }
#undef BI_PRE
}
