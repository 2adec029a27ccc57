// bi_matmul.hip — C ABI of the batch-invariant dense and affine-quantized
// matmul for gfx950 (kernels and launch policy: bi_matmul_impl.h).
#include "bi_matmul_impl.h"

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
namespace {

// Group partials [G, M, N] fp32 of the small-M split launch, and of the
// mid-M launches when they split K (the dense tall tile, the quantized mid
// tile, the mid tile on a dense B with few columns and a long K; 2-byte types:
// the query has no dtype and reports the need of either).
size_t split_ws_bytes(int64_t M, int64_t N, int64_t K, bool dense) {
  const int64_t G = (K + bi::kGroupK - 1) / bi::kGroupK;
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const bool small_split = bi::use_split(M, (int)G) && !bi::use_wg(M, (int)G);
  const bool tall_split = dense && bi::tall_plan(M, N, K).chunks > 1;
  const bool mid_split = dense ? bi::few_columns_plan(M, N, K).use : bi::mid_plan(M, N, K).chunks > 1;
  if (!small_split && !tall_split && !mid_split) return 0;
  return (size_t)(G * M * N) * sizeof(float);
}

int check_common(const char* what, int64_t M, int64_t N, int64_t K, void* out, void* ws,
                 size_t ws_bytes, bool dense) {
  using namespace bi_host;
  if (M < 0 || N <= 0 || K <= 0)
    return fail(BI_E_INVALID_ARG, "%s: bad shape M=%lld N=%lld K=%lld", what, (long long)M,
                (long long)N, (long long)K);
  if (M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL || M * N > ((int64_t)1 << 46) ||
      ((M + 63) / 64) * ((N + 63) / 64) > 0x7fffffffLL - 8)
    return fail(BI_E_UNSUPPORTED, "%s: shape too large", what);
  if (M > 0 && !out) return fail(BI_E_INVALID_ARG, "%s: null out", what);
  const size_t need = split_ws_bytes(M, N, K, dense);
  if (need && (!ws || ws_bytes < need))
    return fail(BI_E_WORKSPACE, "%s: workspace of %zu bytes required, got %zu", what, need,
                ws ? ws_bytes : (size_t)0);
  if (need && !aligned16(ws)) return fail(BI_E_INVALID_ARG, "%s: workspace not 16-byte aligned", what);
  return BI_OK;
}

}  // namespace

extern "C" int bi_split_m_max(void) { return bi::kSplitMMax; }

extern "C" size_t bi_matmul_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  return split_ws_bytes(M, N, K, true);
}

// Quantized: the small-M split partials, or for large M (2-byte types) the
// dequantized weight and the reordered activations of the large-tile launch.
// The query has no dtype: it reports the larger need, which an fp32 call may
// also pass.
static size_t quant_ws_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  if (bi::qmm_use_big(M, N, K, 2)) return bi::qmm_big_ws_bytes(M, N, K);
  return split_ws_bytes(M, N, K, false);
}

extern "C" size_t bi_quantized_matmul_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  return quant_ws_bytes(M, N, K);
}

extern "C" const char* bi_matmul_launch(int64_t M, int64_t N, int64_t K) {
  thread_local char name[64];
  if (M <= 0 || N <= 0 || K <= 0 || M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL) return "other";
  const bi::BigPlan bp = bi::big_plan(M, N, K);
  if (bp.use) return bp.form == bi::kBig128x64 ? "big 128x64" : bp.form == bi::kBig128x128 ? "big 128x128" : "big";
  const bi::TallPlan p = bi::tall_plan(M, N, K);
  if (!p.use) return "other";
  const bi::TallShape& t = bi::kTallShapes[p.tile];
  snprintf(name, sizeof name, "tall %dx%d k%d r%d c%d", t.bm, t.bn, t.sk, t.ring, p.chunks);
  return name;
}

extern "C" int bi_matmul(const void* a, int64_t lda, const void* bt, int64_t ldb, void* out,
                         int64_t M, int64_t N, int64_t K, int dtype, void* ws, size_t ws_bytes,
                         void* stream) {
  using namespace bi_host;
  int rc = check_common("bi_matmul", M, N, K, out, ws, ws_bytes, true);
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

// ---------------------------------------------------------------------------
// A repacked copy of a dense 2-byte B for the decode GEMV (DensePacked in
// bi_gemm_tile.h): the same elements in the layout the streaming GEMV reads,
// so bi_matmul_packed equals bi_matmul bit for bit at every M.
// ---------------------------------------------------------------------------
extern "C" size_t bi_matmul_pack_bytes(int64_t N, int64_t K, int dtype) {
  if ((dtype != BI_BF16 && dtype != BI_F16) || N <= 0 || K <= 0 || K % 8 || N > 0x7fffffffLL || K > 0x7fffffffLL)
    return 0;
  return (size_t)bi::DensePacked<bi::bf16>::bytes(N, K);
}

extern "C" int bi_matmul_pack(const void* bt, int64_t ldb, void* packed, size_t packed_bytes, int64_t N, int64_t K,
                              int dtype, void* stream) {
  using namespace bi_host;
  if (dtype != BI_BF16 && dtype != BI_F16)
    return fail(BI_E_UNSUPPORTED, "bi_matmul_pack: dtype %d (bf16 and fp16 only)", dtype);
  if (N < 0 || K < 0 || N > 0x7fffffffLL || K > 0x7fffffffLL || K % 8)
    return fail(BI_E_INVALID_ARG, "bi_matmul_pack: N=%lld K=%lld (K a multiple of 8)", (long long)N, (long long)K);
  if (N == 0 || K == 0) return BI_OK;
  if (!bt || !packed || !aligned16(bt) || !aligned16(packed) || ldb % 8 || ldb < K)
    return fail(BI_E_INVALID_ARG,
                "bi_matmul_pack: null pointer, bt / packed not 16-byte aligned, or ldb (%lld) not a multiple of 8 "
                ">= K", (long long)ldb);
  const size_t need = bi_matmul_pack_bytes(N, K, dtype);
  if (packed_bytes < need)
    return fail(BI_E_INVALID_ARG, "bi_matmul_pack: packed holds %zu bytes, %zu required", packed_bytes, need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t n = (N + 15) / 16 * ((K + bi::kGroupK - 1) / bi::kGroupK) * bi::kWave;
  const unsigned grid = (unsigned)((n + 255) / 256);
  if (dtype == BI_BF16)
    bi::dense_pack_rows<bi::bf16><<<grid, 256, 0, st>>>(static_cast<const bi::bf16*>(bt), ldb,
                                                         static_cast<char*>(packed), (int)N, (int)K);
  else
    bi::dense_pack_rows<bi::f16><<<grid, 256, 0, st>>>(static_cast<const bi::f16*>(bt), ldb,
                                                        static_cast<char*>(packed), (int)N, (int)K);
  return launch_status("bi_matmul_pack");
}

extern "C" int bi_matmul_packed(const void* a, int64_t lda, const void* bt, int64_t ldb, const void* packed,
                                void* out, int64_t M, int64_t N, int64_t K, int dtype, void* ws, size_t ws_bytes,
                                void* stream) {
  using namespace bi_host;
  if (!packed) return bi_matmul(a, lda, bt, ldb, out, M, N, K, dtype, ws, ws_bytes, stream);
  if ((dtype != BI_BF16 && dtype != BI_F16) || K % 8)
    return fail(BI_E_UNSUPPORTED, "bi_matmul_packed: a packed copy needs bf16 / fp16 and K %% 8 == 0 (dtype=%d K=%lld)",
                dtype, (long long)K);
  if (!aligned16(packed)) return fail(BI_E_INVALID_ARG, "bi_matmul_packed: packed not 16-byte aligned");
  // The streaming GEMV's shapes on the copy; everything else (and any shape it
  // does not take) is bi_matmul on the row-major operands, checks included.
  if (M >= 1 && M <= 16 && N >= 1 && N <= 0x7fffffffLL && K <= 0x7fffffffLL && a && bt && out && lda % 8 == 0 &&
      lda >= K && ldb % 8 == 0 && ldb >= K && aligned16(a) && aligned16(bt)) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int Mi = (int)M, Ni = (int)N, Ki = (int)K;
    auto go = [&](auto tag) {
      typedef decltype(tag) T;
      bi::DensePacked<T> b;
      b.bt = static_cast<const T*>(bt);
      b.ldb = ldb;
      b.N = Ni;
      b.K = Ki;
      b.p = static_cast<const char*>(packed);
      b.G = (Ki + bi::kGroupK - 1) / bi::kGroupK;
      return bi::launch_stream_dense_packed<T>(static_cast<const T*>(a), lda, b, static_cast<T*>(out), Mi, Ni, Ki,
                                               b.G, st);
    };
    if (dtype == BI_BF16 ? go(bi::bf16{}) : go(bi::f16{})) return launch_status("bi_matmul_packed");
  }
  return bi_matmul(a, lda, bt, ldb, out, M, N, K, dtype, ws, ws_bytes, stream);
}

// Strided batch of independent matmuls: slice i is exactly bi_matmul on
// a + i * a_batch_stride, bt + i * b_batch_stride, out + i * out_batch_stride
// (element strides; 0 broadcasts an operand). The slices run one after the
// other on the stream and share the workspace.
extern "C" int bi_matmul_batched(const void* a, int64_t a_batch_stride, int64_t lda, const void* bt,
                                 int64_t b_batch_stride, int64_t ldb, void* out, int64_t out_batch_stride,
                                 int64_t batch, int64_t M, int64_t N, int64_t K, int dtype, void* ws,
                                 size_t ws_bytes, void* stream) {
  using namespace bi_host;
  if (batch < 0) return fail(BI_E_INVALID_ARG, "bi_matmul_batched: batch=%lld", (long long)batch);
  if (a_batch_stride < 0 || b_batch_stride < 0 || out_batch_stride < M * N)
    return fail(BI_E_INVALID_ARG, "bi_matmul_batched: negative batch stride or out_batch_stride < M*N");
  if (dtype != BI_BF16 && dtype != BI_F16 && dtype != BI_F32)
    return fail(BI_E_UNSUPPORTED, "bi_matmul_batched: unknown dtype %d", dtype);
  const size_t es = dtype == BI_F32 ? 4 : 2;
  for (int64_t i = 0; i < batch; ++i) {
    const char* ai = static_cast<const char*>(a) + (size_t)(i * a_batch_stride) * es;
    const char* bi_ = static_cast<const char*>(bt) + (size_t)(i * b_batch_stride) * es;
    char* oi = static_cast<char*>(out) + (size_t)(i * out_batch_stride) * es;
    const int rc = bi_matmul(ai, lda, bi_, ldb, oi, M, N, K, dtype, ws, ws_bytes, stream);
    if (rc) return rc;
  }
  return BI_OK;
}

namespace {

// Checks shared by bi_quantized_matmul and bi_quantized_matmul_packed: BI_OK
// to run, an error code (negative) to return, or kQmmEmpty for a call with
// nothing to compute (M = 0), which then returns BI_OK.
constexpr int kQmmEmpty = 1;
int qmm_check(const char* name, const void* x, int64_t ldx, const uint32_t* w, const void* scales,
              const void* biases, void* out, int64_t M, int64_t N, int64_t K, int bits, int group_size, int dtype,
              void* ws, size_t ws_bytes) {
  using namespace bi_host;
  if ((bits != 4 && bits != 8) || (group_size != 32 && group_size != 64 && group_size != 128))
    return fail(BI_E_UNSUPPORTED, "%s: bits=%d group_size=%d not in {4,8}x{32,64,128}", name, bits, group_size);
  int rc = check_common(name, M, N, K, out, ws, ws_bytes, false);
  if (rc) return rc;
  if (K % group_size)
    return fail(BI_E_INVALID_ARG, "%s: K=%lld not a multiple of group_size=%d", name, (long long)K, group_size);
  if (M == 0) return kQmmEmpty;
  if (!x || !w || !scales || !biases) return fail(BI_E_INVALID_ARG, "%s: null operand", name);
  if (ldx % 8 || ldx < K || !aligned16(x) || !aligned16(w))
    return fail(BI_E_INVALID_ARG, "%s: needs ldx %% 8 == 0, ldx >= K, 16-byte aligned x and w", name);
  if (dtype != BI_F32 && bi::qmm_use_big(M, N, K, 2)) {
    const size_t need = bi::qmm_big_ws_bytes(M, N, K);
    if (!ws || ws_bytes < need || !aligned16(ws))
      return fail(BI_E_WORKSPACE, "%s: 16-byte aligned workspace of %zu bytes required, got %zu", name, need,
                  ws ? ws_bytes : (size_t)0);
  }
  return BI_OK;
}

}  // namespace

extern "C" int bi_quantized_matmul(const void* x, int64_t ldx, const uint32_t* w,
                                   const void* scales, const void* biases, void* out, int64_t M,
                                   int64_t N, int64_t K, int bits, int group_size, int dtype,
                                   void* ws, size_t ws_bytes, void* stream) {
  using namespace bi_host;
  const int rc = qmm_check("bi_quantized_matmul", x, ldx, w, scales, biases, out, M, N, K, bits, group_size, dtype,
                           ws, ws_bytes);
  if (rc) return rc == kQmmEmpty ? BI_OK : rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int Mi = (int)M, Ni = (int)N, Ki = (int)K;
  switch (dtype) {
    case BI_BF16:
      return bi::qmm_bf16(bits, group_size, x, ldx, w, scales, biases, out, Mi, Ni, Ki, ws, st);
    case BI_F16:
      return bi::qmm_f16(bits, group_size, x, ldx, w, scales, biases, out, Mi, Ni, Ki, ws, st);
    case BI_F32:
      return bi::qmm_f32(bits, group_size, x, ldx, w, scales, biases, out, Mi, Ni, Ki, ws, st);
    default: return fail(BI_E_UNSUPPORTED, "bi_quantized_matmul: unknown dtype %d", dtype);
  }
}

// ---------------------------------------------------------------------------
// A repacked copy of a weight for the decode GEMV (QuantPacked in
// bi_gemm_tile.h): the same codes, scales and biases in the layout the
// streaming GEMV reads, so bi_quantized_matmul_packed equals
// bi_quantized_matmul bit for bit at every M.
// ---------------------------------------------------------------------------
namespace {

bool packable(int bits, int group_size) {
  return (bits == 4 || bits == 8) && (group_size == 32 || group_size == 64 || group_size == 128);
}

template <int BITS>
size_t pack_bytes_bits(int64_t N, int64_t K, int gs) {
  if (gs == 32) return (size_t)bi::QuantPacked<bi::bf16, BITS, 32>::bytes(N, K);
  if (gs == 64) return (size_t)bi::QuantPacked<bi::bf16, BITS, 64>::bytes(N, K);
  return (size_t)bi::QuantPacked<bi::bf16, BITS, 128>::bytes(N, K);
}

template <typename T, int BITS>
int pack_bits(int gs, const uint32_t* w, const void* scales, const void* biases, void* packed, int N, int K,
              hipStream_t st) {
  if (gs == 32) return bi::pack_quant<T, BITS, 32>(w, scales, biases, packed, N, K, st);
  if (gs == 64) return bi::pack_quant<T, BITS, 64>(w, scales, biases, packed, N, K, st);
  return bi::pack_quant<T, BITS, 128>(w, scales, biases, packed, N, K, st);
}

}  // namespace

extern "C" size_t bi_quantized_pack_bytes(int64_t N, int64_t K, int bits, int group_size) {
  if (!packable(bits, group_size) || N <= 0 || K <= 0 || K % bi::kGroupK || N > 0x7fffffffLL || K > 0x7fffffffLL)
    return 0;
  return bits == 4 ? pack_bytes_bits<4>(N, K, group_size) : pack_bytes_bits<8>(N, K, group_size);
}

extern "C" int bi_quantized_pack(const uint32_t* w, const void* scales, const void* biases, void* packed,
                                 size_t packed_bytes, int64_t N, int64_t K, int bits, int group_size, int dtype,
                                 void* stream) {
  using namespace bi_host;
  if (!packable(bits, group_size))
    return fail(BI_E_UNSUPPORTED, "bi_quantized_pack: bits=%d group_size=%d not in {4,8}x{32,64,128}", bits,
                group_size);
  if (dtype != BI_BF16 && dtype != BI_F16)
    return fail(BI_E_UNSUPPORTED, "bi_quantized_pack: dtype %d (bf16 and fp16 only)", dtype);
  if (N < 0 || K < 0 || N > 0x7fffffffLL || K > 0x7fffffffLL || K % bi::kGroupK)
    return fail(BI_E_INVALID_ARG, "bi_quantized_pack: N=%lld K=%lld (K a multiple of 256)", (long long)N,
                (long long)K);
  if (N == 0 || K == 0) return BI_OK;
  const size_t need = bi_quantized_pack_bytes(N, K, bits, group_size);
  if (!w || !scales || !biases || !packed || !aligned16(packed) || !aligned16(w))
    return fail(BI_E_INVALID_ARG, "bi_quantized_pack: null pointer, or w / packed not 16-byte aligned");
  if (packed_bytes < need)
    return fail(BI_E_INVALID_ARG, "bi_quantized_pack: packed holds %zu bytes, %zu required", packed_bytes, need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int Ni = (int)N, Ki = (int)K;
  if (dtype == BI_BF16)
    return bits == 4 ? pack_bits<bi::bf16, 4>(group_size, w, scales, biases, packed, Ni, Ki, st)
                     : pack_bits<bi::bf16, 8>(group_size, w, scales, biases, packed, Ni, Ki, st);
  return bits == 4 ? pack_bits<bi::f16, 4>(group_size, w, scales, biases, packed, Ni, Ki, st)
                   : pack_bits<bi::f16, 8>(group_size, w, scales, biases, packed, Ni, Ki, st);
}

extern "C" int bi_quantized_matmul_packed(const void* x, int64_t ldx, const uint32_t* w, const void* scales,
                                          const void* biases, const void* packed, void* out, int64_t M,
                                          int64_t N, int64_t K, int bits, int group_size, int dtype, void* ws,
                                          size_t ws_bytes, void* stream) {
  using namespace bi_host;
  if (!packed)
    return bi_quantized_matmul(x, ldx, w, scales, biases, out, M, N, K, bits, group_size, dtype, ws, ws_bytes,
                               stream);
  if ((dtype != BI_BF16 && dtype != BI_F16) || K % bi::kGroupK)
    return fail(BI_E_UNSUPPORTED,
                "bi_quantized_matmul_packed: a packed copy needs bf16 / fp16 and K %% 256 == 0 (dtype=%d K=%lld)",
                dtype, (long long)K);
  const int rc = qmm_check("bi_quantized_matmul_packed", x, ldx, w, scales, biases, out, M, N, K, bits, group_size,
                           dtype, ws, ws_bytes);
  if (rc) return rc == kQmmEmpty ? BI_OK : rc;
  if (!aligned16(packed)) return fail(BI_E_INVALID_ARG, "bi_quantized_matmul_packed: packed not 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int Mi = (int)M, Ni = (int)N, Ki = (int)K;
  if (dtype == BI_BF16)
    return bi::qmm_packed_bf16(bits, group_size, x, ldx, w, scales, biases, packed, out, Mi, Ni, Ki, ws, st);
  return bi::qmm_packed_f16(bits, group_size, x, ldx, w, scales, biases, packed, out, Mi, Ni, Ki, ws, st);
}

// ---------------------------------------------------------------------------
// The quantized op on a weight dequantized once (the large-M launch's B': the
// dequantized weight in the dense tile's k order, bi_qmm_big.h). With A
// reordered the same way, every dense launch puts in each MFMA slot exactly
// the product the quantized launches put there, so the result equals
// bi_quantized_matmul's bit for bit at every M; a caller that keeps B' skips
// the per-call dequantization of the large-M launch.
// ---------------------------------------------------------------------------
namespace {

template <typename T, int BITS>
int dequantize_bits(int gs, const uint32_t* w, const void* scales, const void* biases, void* bq, int N, int K,
                    hipStream_t st) {
  const int64_t nb = (int64_t)N * (K / 8);
  const unsigned grid = (unsigned)((nb + 255) / 256);
  const T* sc = static_cast<const T*>(scales);
  const T* bs = static_cast<const T*>(biases);
  T* out = static_cast<T*>(bq);
  if (gs == 32) bi::qmm_dequant_rows<T, BITS, 32><<<grid, 256, 0, st>>>(w, sc, bs, out, N, K);
  else if (gs == 64) bi::qmm_dequant_rows<T, BITS, 64><<<grid, 256, 0, st>>>(w, sc, bs, out, N, K);
  else bi::qmm_dequant_rows<T, BITS, 128><<<grid, 256, 0, st>>>(w, sc, bs, out, N, K);
  return bi_host::launch_status("bi_quantized_dequantize");
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

}  // namespace

extern "C" int bi_quantized_dequantize(const uint32_t* w, const void* scales, const void* biases, void* bq,
                                       int64_t N, int64_t K, int bits, int group_size, int dtype, void* stream) {
  using namespace bi_host;
  if ((bits != 4 && bits != 8) || (group_size != 32 && group_size != 64 && group_size != 128))
    return fail(BI_E_UNSUPPORTED, "bi_quantized_dequantize: bits=%d group_size=%d not in {4,8}x{32,64,128}", bits,
                group_size);
  if (dtype != BI_BF16 && dtype != BI_F16)
    return fail(BI_E_UNSUPPORTED, "bi_quantized_dequantize: dtype %d (bf16 and fp16 only)", dtype);
  if (N < 0 || K < 0 || N > 0x7fffffffLL || K > 0x7fffffffLL || K % bi::kGroupK || N * (K / 8) > ((int64_t)1 << 40))
    return fail(BI_E_INVALID_ARG, "bi_quantized_dequantize: N=%lld K=%lld (K a multiple of 256)", (long long)N,
                (long long)K);
  if (N == 0 || K == 0) return BI_OK;
  if (!w || !scales || !biases || !bq || !aligned16(bq))
    return fail(BI_E_INVALID_ARG, "bi_quantized_dequantize: null pointer, or bq not 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int Ni = (int)N, Ki = (int)K;
  if (dtype == BI_BF16)
    return bits == 4 ? dequantize_bits<bi::bf16, 4>(group_size, w, scales, biases, bq, Ni, Ki, st)
                     : dequantize_bits<bi::bf16, 8>(group_size, w, scales, biases, bq, Ni, Ki, st);
  return bits == 4 ? dequantize_bits<bi::f16, 4>(group_size, w, scales, biases, bq, Ni, Ki, st)
                   : dequantize_bits<bi::f16, 8>(group_size, w, scales, biases, bq, Ni, Ki, st);
}

extern "C" size_t bi_quantized_matmul_dequantized_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return align256((size_t)M * (size_t)K * 2) + split_ws_bytes(M, N, K, true);
}

extern "C" int bi_quantized_matmul_dequantized(const void* x, int64_t ldx, const void* bq, void* out, int64_t M,
                                               int64_t N, int64_t K, int dtype, void* ws, size_t ws_bytes,
                                               void* stream) {
  using namespace bi_host;
  if (dtype != BI_BF16 && dtype != BI_F16)
    return fail(BI_E_UNSUPPORTED, "bi_quantized_matmul_dequantized: dtype %d (bf16 and fp16 only)", dtype);
  if (M < 0 || N < 0 || K < 0 || M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL || K % bi::kGroupK)
    return fail(BI_E_INVALID_ARG, "bi_quantized_matmul_dequantized: M=%lld N=%lld K=%lld (K a multiple of 256)",
                (long long)M, (long long)N, (long long)K);
  if (M == 0 || N == 0) return BI_OK;
  if (K == 0) return fail(BI_E_INVALID_ARG, "bi_quantized_matmul_dequantized: K = 0");
  if (!x || !bq || !out || ldx % 8 || ldx < K || !aligned16(x) || !aligned16(bq))
    return fail(BI_E_INVALID_ARG,
                "bi_quantized_matmul_dequantized: needs ldx %% 8 == 0, ldx >= K, 16-byte aligned x and bq");
  const size_t a_bytes = align256((size_t)M * (size_t)K * 2);
  const size_t need = bi_quantized_matmul_dequantized_workspace_bytes(M, N, K);
  if (!ws || ws_bytes < need || !aligned16(ws))
    return fail(BI_E_WORKSPACE,
                "bi_quantized_matmul_dequantized: 16-byte aligned workspace of %zu bytes required, got %zu", need,
                ws ? ws_bytes : (size_t)0);
  int rc = check_common("bi_quantized_matmul_dequantized", M, N, K, out, static_cast<char*>(ws) + a_bytes,
                        ws_bytes - a_bytes, true);
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int Mi = (int)M, Ni = (int)N, Ki = (int)K;
  float* wsd = reinterpret_cast<float*>(static_cast<char*>(ws) + a_bytes);
  const int64_t na = (int64_t)M * (K / 8);
  auto go = [&](auto tag) {
    typedef decltype(tag) T;
    T* ap = static_cast<T*>(ws);
    bi::qmm_permute_a<T><<<(unsigned)((na + 255) / 256), 256, 0, st>>>(static_cast<const T*>(x), ldx, ap, Mi, Ki);
    bi::DenseB<T> db{static_cast<const T*>(bq), K, Ni, Ki};
    return bi::run_gemm<T, bi::DenseB<T>>(ap, K, db, static_cast<T*>(out), Mi, Ni, Ki, wsd, st,
                                          "bi_quantized_matmul_dequantized");
  };
  return dtype == BI_BF16 ? go(bi::bf16{}) : go(bi::f16{});
}
