// bi_matmul.hip — batch-invariant dense and affine-quantized matmul for gfx950.
//
// Kernels (all run the tile body of bi_gemm_tile.h):
//   gemm_direct<..., SPLIT=true>   one workgroup per (column tile, K group);
//                                  writes the raw fp32 group partial
//                                  part[g, m, n]  (small M, several groups)
//   bi_fold_groups                 out = T(((0 + part[0]) + part[1]) + ...)
//   gemm_direct<..., SPLIT=false>  folds all groups in registers and writes T
// Reference launchers: kernels/matmul.py:279-314 (launch_tiled; split for
// M <= SPLIT_M_MAX and more than one group, fused otherwise), the combine
// kernel kernels/matmul.py:226-234, and kernels/quantized.py:106-125.
#include "bi_gemm_tile.h"

namespace bi {

constexpr int kSplitMMax = 32;

// MT m-tiles x NT n-tiles of 16x16 per wave, WAVES waves per workgroup along n.
template <typename T, class BSrc, int MT, int NT, int WAVES, bool SPLIT>
__global__ __launch_bounds__(kWave* WAVES) void gemm_direct(const T* __restrict__ a,
                                                            int64_t lda, BSrc bsrc,
                                                            T* __restrict__ out,
                                                            float* __restrict__ part, int M,
                                                            int N, int K, int G) {
  typedef typename Frag<T>::type F;
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int r = lane % 16, q = lane / 16;
  const int n_base = (blockIdx.x * WAVES + wave) * 16 * NT;
  const int m_base = blockIdx.y * 16 * MT;
  if (n_base >= N) return;  // wave-uniform; the kernel has no block barrier
  const int g0 = SPLIT ? (int)blockIdx.z : 0;
  const int g1 = SPLIT ? g0 + 1 : G;

  f32x4 total[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) total[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int g = g0; g < g1; ++g) {
    typename BSrc::Raw braw[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) bsrc.load(braw[j], n_base + 16 * j + r, g, q);
    f32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      F af[MT];
#pragma unroll
      for (int i = 0; i < MT; ++i) af[i] = load_a_frag(a, lda, m_base + 16 * i + r, M, K, g, q, s);
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const F bf = bsrc.frag(braw[j], s);
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[i][j] = mfma_step(af[i], bf, acc[i][j]);
      }
    }
    if constexpr (SPLIT) {
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          const int n = n_base + 16 * j + r;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int m = m_base + 16 * i + 4 * q + e;
            if (m < M && n < N) part[((int64_t)g * M + m) * N + n] = acc[i][j][e];
          }
        }
    } else {
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) total[i][j] = total[i][j] + acc[i][j];
    }
  }
  if constexpr (!SPLIT) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int n = n_base + 16 * j + r;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = m_base + 16 * i + 4 * q + e;
          if (m < M && n < N) out[(int64_t)m * N + n] = to_store<T>(total[i][j][e]);
        }
      }
  }
}

// Left fold of the group partials, exactly the fused kernel's fold:
// total = 0; total = total + part[g] for g = 0 .. G-1; out = T(total).
template <typename T>
__global__ __launch_bounds__(256) void fold_groups(const float* __restrict__ part,
                                                   T* __restrict__ out, int64_t MN, int G) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= MN) return;
  float total = 0.0f;
  for (int g = 0; g < G; ++g) total = total + part[(int64_t)g * MN + idx];
  out[idx] = to_store<T>(total);
}

static inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// Launch-shape policy (kernels/matmul.py:279-314): M <= 32 with more than one
// group -> split partials + fold; otherwise fused. Bits never depend on it.
static inline bool use_split(int64_t M, int G) { return M <= kSplitMMax && G > 1; }

template <typename T, class BSrc>
static int run_gemm(const T* a, int64_t lda, const BSrc& bsrc, T* out, int M, int N, int K,
                    float* ws, hipStream_t st, const char* what) {
  const int G = ceil_div(K, kGroupK);
  constexpr int WAVES = 4;
  if (use_split(M, G)) {
    if (M <= 16) {
      dim3 grid(ceil_div(N, 16 * WAVES), 1, G);
      gemm_direct<T, BSrc, 1, 1, WAVES, true><<<grid, kWave * WAVES, 0, st>>>(a, lda, bsrc, out, ws,
                                                                          M, N, K, G);
    } else {
      dim3 grid(ceil_div(N, 16 * WAVES), 1, G);
      gemm_direct<T, BSrc, 2, 1, WAVES, true><<<grid, kWave * WAVES, 0, st>>>(a, lda, bsrc, out, ws,
                                                                          M, N, K, G);
    }
    int rc = bi_host::launch_status(what);
    if (rc) return rc;
    const int64_t MN = (int64_t)M * N;
    fold_groups<T><<<(unsigned)((MN + 255) / 256), 256, 0, st>>>(ws, out, MN, G);
    return bi_host::launch_status(what);
  }
  if (M <= 16) {
    dim3 grid(ceil_div(N, 16 * WAVES), 1, 1);
    gemm_direct<T, BSrc, 1, 1, WAVES, false><<<grid, kWave * WAVES, 0, st>>>(a, lda, bsrc, out,
                                                                         nullptr, M, N, K, G);
  } else if (M <= 32) {
    dim3 grid(ceil_div(N, 16 * WAVES), 1, 1);
    gemm_direct<T, BSrc, 2, 1, WAVES, false><<<grid, kWave * WAVES, 0, st>>>(a, lda, bsrc, out,
                                                                         nullptr, M, N, K, G);
  } else {
    constexpr int MT = sizeof(T) == 4 ? 2 : 4;
    dim3 grid(ceil_div(N, 16 * WAVES), ceil_div(M, 16 * MT), 1);
    gemm_direct<T, BSrc, MT, 1, WAVES, false><<<grid, kWave * WAVES, 0, st>>>(a, lda, bsrc, out,
                                                                          nullptr, M, N, K, G);
  }
  return bi_host::launch_status(what);
}

}  // namespace bi

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
namespace {

size_t split_ws_bytes(int64_t M, int64_t N, int64_t K) {
  const int64_t G = (K + bi::kGroupK - 1) / bi::kGroupK;
  if (M <= 0 || N <= 0 || K <= 0 || !bi::use_split(M, (int)G)) return 0;
  return (size_t)(G * M * N) * sizeof(float);
}

int check_common(const char* what, int64_t M, int64_t N, int64_t K, void* out, void* ws,
                 size_t ws_bytes) {
  using namespace bi_host;
  if (M < 0 || N <= 0 || K <= 0)
    return fail(BI_E_INVALID_ARG, "%s: bad shape M=%lld N=%lld K=%lld", what, (long long)M,
                (long long)N, (long long)K);
  if (M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL || M * N > ((int64_t)1 << 46))
    return fail(BI_E_UNSUPPORTED, "%s: shape too large", what);
  if (M > 0 && !out) return fail(BI_E_INVALID_ARG, "%s: null out", what);
  const size_t need = split_ws_bytes(M, N, K);
  if (need && (!ws || ws_bytes < need))
    return fail(BI_E_WORKSPACE, "%s: workspace of %zu bytes required, got %zu", what, need,
                ws ? ws_bytes : (size_t)0);
  if (need && !aligned16(ws)) return fail(BI_E_INVALID_ARG, "%s: workspace not 16-byte aligned", what);
  return BI_OK;
}

}  // namespace

extern "C" int bi_split_m_max(void) { return bi::kSplitMMax; }

extern "C" size_t bi_matmul_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  return split_ws_bytes(M, N, K);
}

extern "C" size_t bi_quantized_matmul_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  return split_ws_bytes(M, N, K);
}

extern "C" int bi_matmul(const void* a, int64_t lda, const void* bt, int64_t ldb, void* out,
                         int64_t M, int64_t N, int64_t K, int dtype, void* ws, size_t ws_bytes,
                         void* stream) {
  using namespace bi_host;
  int rc = check_common("bi_matmul", M, N, K, out, ws, ws_bytes);
  if (rc) return rc;
  if (M == 0) return BI_OK;
  if (!a || !bt) return fail(BI_E_INVALID_ARG, "bi_matmul: null operand");
  if (K % 8 || lda % 8 || ldb % 8 || lda < K || ldb < K || !aligned16(a) || !aligned16(bt))
    return fail(BI_E_INVALID_ARG,
                "bi_matmul: needs K, lda, ldb multiples of 8 (lda, ldb >= K) and 16-byte "
                "aligned operands (K=%lld lda=%lld ldb=%lld)",
                (long long)K, (long long)lda, (long long)ldb);
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* wsf = static_cast<float*>(ws);
  const int Mi = (int)M, Ni = (int)N, Ki = (int)K;
  switch (dtype) {
    case BI_BF16: {
      bi::DenseB<bi::bf16> b{static_cast<const bi::bf16*>(bt), ldb, Ni, Ki};
      return bi::run_gemm(static_cast<const bi::bf16*>(a), lda, b, static_cast<bi::bf16*>(out), Mi,
                          Ni, Ki, wsf, st, "bi_matmul");
    }
    case BI_F16: {
      bi::DenseB<bi::f16> b{static_cast<const bi::f16*>(bt), ldb, Ni, Ki};
      return bi::run_gemm(static_cast<const bi::f16*>(a), lda, b, static_cast<bi::f16*>(out), Mi, Ni,
                          Ki, wsf, st, "bi_matmul");
    }
    case BI_F32: {
      bi::DenseB<float> b{static_cast<const float*>(bt), ldb, Ni, Ki};
      return bi::run_gemm(static_cast<const float*>(a), lda, b, static_cast<float*>(out), Mi, Ni,
                          Ki, wsf, st, "bi_matmul");
    }
    default: return fail(BI_E_UNSUPPORTED, "bi_matmul: unknown dtype %d", dtype);
  }
}

namespace {

template <typename T, int BITS, int GS>
int run_quant(const void* x, int64_t ldx, const uint32_t* w, const void* scales,
              const void* biases, void* out, int M, int N, int K, void* ws, hipStream_t st) {
  bi::QuantB<T, BITS, GS> b;
  b.w = w;
  b.scales = static_cast<const T*>(scales);
  b.biases = static_cast<const T*>(biases);
  b.N = N;
  b.K = K;
  b.words_per_row = (int64_t)K * BITS / 32;
  b.groups_per_row = K / GS;
  return bi::run_gemm(static_cast<const T*>(x), ldx, b, static_cast<T*>(out), M, N, K,
                      static_cast<float*>(ws), st, "bi_quantized_matmul");
}

template <typename T>
int dispatch_quant(int bits, int gs, const void* x, int64_t ldx, const uint32_t* w,
                   const void* scales, const void* biases, void* out, int M, int N, int K,
                   void* ws, hipStream_t st) {
#define BI_Q(B, G)                                                                       \
  if (bits == B && gs == G)                                                              \
    return run_quant<T, B, G>(x, ldx, w, scales, biases, out, M, N, K, ws, st);
  BI_Q(4, 32) BI_Q(4, 64) BI_Q(4, 128) BI_Q(8, 32) BI_Q(8, 64) BI_Q(8, 128)
#undef BI_Q
  return bi_host::fail(BI_E_UNSUPPORTED, "bi_quantized_matmul: bits=%d group_size=%d", bits, gs);
}

}  // namespace

extern "C" int bi_quantized_matmul(const void* x, int64_t ldx, const uint32_t* w,
                                   const void* scales, const void* biases, void* out, int64_t M,
                                   int64_t N, int64_t K, int bits, int group_size, int dtype,
                                   void* ws, size_t ws_bytes, void* stream) {
  using namespace bi_host;
  if ((bits != 4 && bits != 8) || (group_size != 32 && group_size != 64 && group_size != 128))
    return fail(BI_E_UNSUPPORTED, "bi_quantized_matmul: bits=%d group_size=%d not in {4,8}x{32,64,128}",
                bits, group_size);
  int rc = check_common("bi_quantized_matmul", M, N, K, out, ws, ws_bytes);
  if (rc) return rc;
  if (K % group_size)
    return fail(BI_E_INVALID_ARG, "bi_quantized_matmul: K=%lld not a multiple of group_size=%d",
                (long long)K, group_size);
  if (M == 0) return BI_OK;
  if (!x || !w || !scales || !biases)
    return fail(BI_E_INVALID_ARG, "bi_quantized_matmul: null operand");
  if (ldx % 8 || ldx < K || !aligned16(x) || !aligned16(w))
    return fail(BI_E_INVALID_ARG,
                "bi_quantized_matmul: needs ldx %% 8 == 0, ldx >= K, 16-byte aligned x and w");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int Mi = (int)M, Ni = (int)N, Ki = (int)K;
  switch (dtype) {
    case BI_BF16:
      return dispatch_quant<bi::bf16>(bits, group_size, x, ldx, w, scales, biases, out, Mi, Ni, Ki, ws, st);
    case BI_F16:
      return dispatch_quant<bi::f16>(bits, group_size, x, ldx, w, scales, biases, out, Mi, Ni, Ki, ws, st);
    case BI_F32:
      return dispatch_quant<float>(bits, group_size, x, ldx, w, scales, biases, out, Mi, Ni, Ki, ws, st);
    default: return fail(BI_E_UNSUPPORTED, "bi_quantized_matmul: unknown dtype %d", dtype);
  }
}
