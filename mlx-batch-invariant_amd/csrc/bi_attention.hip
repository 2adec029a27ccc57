// bi_attention.hip — batch-invariant split-KV decode and prefill attention.
//
// Reference: kernels/attention.py of mlx-batch-invariant — decode kernel
// :87-147 (one simdgroup per (batch, kv head, head chunk, split), partials per
// split), combine :149-171 (left fold of splits, precise divide), prefill
// :173-254 (queries share K/V rows, splits folded in registers, bottom-right
// causal mask nkeys = L - Tq + t + 1). Per-split arithmetic: bi_attn_common.h;
// kernels: bi_attn_mfma.h; launchers: bi_attn_launch.h, instantiated per element
// type in bi_attn_{bf16,f16,f32}.hip for head dims 32, 64, 96, 128, 192, 256.
//
// gfx950 launches:
//   decode  a resident grid of 256-thread workgroups walking the active items
//           (sequence, split, kv head, head chunk of GU <= 16 heads); each
//           item writes (m, l, acc) of its split.
//   combine one thread per (sequence, head, d); merges the sequence's own
//           ceil(len/256) splits left to right and divides.
//   prefill one 256-thread workgroup per (sequence, kv head, 64 (token, head)
//           rows, token-major), K/V streamed through LDS in 64-key chunks,
//           splits merged in registers.
#include <mutex>
#include <type_traits>

#include "bi_attn_api.h"

namespace bi {

// Calls fn(std::integral_constant<int, D>) for a supported head dim (checked
// by check_attn_shape before any launch).
template <class Fn>
static int with_head_dim(int D, Fn&& fn) {
  switch (D) {
    case 32: return fn(std::integral_constant<int, 32>());
    case 64: return fn(std::integral_constant<int, 64>());
    case 96: return fn(std::integral_constant<int, 96>());
    case 128: return fn(std::integral_constant<int, 128>());
    case 192: return fn(std::integral_constant<int, 192>());
    default: return fn(std::integral_constant<int, 256>());
  }
}

// The per-key kernels take every head dim D % 32 == 0 up to 512 (the
// reference's kernels accept any multiple of 32, kernels/attention.py:299-310);
// the six of with_head_dim, plus these.
template <class Fn>
static int with_head_dim_per_key(int D, Fn&& fn) {
  switch (D) {
    case 160: return fn(std::integral_constant<int, 160>());
    case 224: return fn(std::integral_constant<int, 224>());
    case 288: return fn(std::integral_constant<int, 288>());
    case 320: return fn(std::integral_constant<int, 320>());
    case 352: return fn(std::integral_constant<int, 352>());
    case 384: return fn(std::integral_constant<int, 384>());
    case 416: return fn(std::integral_constant<int, 416>());
    case 448: return fn(std::integral_constant<int, 448>());
    case 480: return fn(std::integral_constant<int, 480>());
    case 512: return fn(std::integral_constant<int, 512>());
    default: return with_head_dim(D, fn);
  }
}

}  // namespace bi

namespace {

int check_attn_shape(const char* what, int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t D,
                     bool per_key = false) {
  using namespace bi_host;
  if (B < 0 || Hq <= 0 || Hkv <= 0 || L <= 0 || D <= 0)
    return fail(BI_E_INVALID_ARG, "%s: bad shape B=%lld Hq=%lld Hkv=%lld L=%lld D=%lld", what,
                (long long)B, (long long)Hq, (long long)Hkv, (long long)L, (long long)D);
  if (Hq % Hkv) return fail(BI_E_INVALID_ARG, "%s: Hq=%lld not a multiple of Hkv=%lld", what,
                            (long long)Hq, (long long)Hkv);
  if (per_key && (D % 32 || D > 512))
    return fail(BI_E_UNSUPPORTED, "%s: head dim %lld (supported: multiples of 32 up to 512)", what, (long long)D);
  if (!per_key && D != 32 && D != 64 && D != 96 && D != 128 && D != 192 && D != 256)
    return fail(BI_E_UNSUPPORTED, "%s: head dim %lld (supported: 32, 64, 96, 128, 192, 256; any multiple of 32 "
                "up to 512 in the per-key order)", what, (long long)D);
  if (B > 65535 || Hkv > 65535 || L > 0x7fffffffLL - bi::kSplit || Hq > 0x7fffffffLL / 16)
    return fail(BI_E_UNSUPPORTED, "%s: shape exceeds the grid limits", what);
  return BI_OK;
}

}  // namespace

namespace {

// pm | pl | pacc | item counter (16 bytes), each 16-byte aligned, for splits of
// `split` keys.
size_t decode_ws_bytes(int64_t B, int64_t Hq, int64_t L, int64_t D, int64_t split) {
  if (B <= 0 || Hq <= 0 || L <= 0 || D <= 0 || split <= 0) return 0;
  const int64_t ns = (L + split - 1) / split;
  const int64_t bh = B * Hq * ns;
  auto up = [](int64_t x) { return (x + 3) / 4 * 4; };
  return (size_t)(up(bh) * 2 + bh * D + 4) * sizeof(float);
}

// Split sizes the per-key kernels take (the reference's split_size): any
// positive key count up to 2^20.
constexpr int64_t kMaxSplit = (int64_t)1 << 20;

}  // namespace

extern "C" size_t bi_attn_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t L, int64_t D) {
  return decode_ws_bytes(B, Hq, L, D, bi::kSplit);
}

extern "C" size_t bi_attn_decode_per_key_workspace_bytes(int64_t B, int64_t Hq, int64_t L, int64_t D,
                                                         int64_t split_size) {
  if (split_size <= 0 || split_size > kMaxSplit) return 0;
  return decode_ws_bytes(B, Hq, L, D, split_size);
}

namespace {

// Page table of a paged call: power-of-two page size, one row of
// table_stride >= ceil(L / page_size) page indices per sequence, a pool of
// 1 <= num_pages < 2^31 pages (the kernels clamp every table entry into it).
int check_pages(const char* what, const int32_t* table, int64_t table_stride, int64_t page_size, int64_t num_pages,
                int64_t L, int* shift) {
  using namespace bi_host;
  if (!table) return fail(BI_E_INVALID_ARG, "%s: null block table", what);
  if (num_pages <= 0 || num_pages > 0x7fffffffLL)
    return fail(BI_E_INVALID_ARG, "%s: num_pages %lld must be in [1, 2^31)", what, (long long)num_pages);
  if (page_size <= 0 || page_size > ((int64_t)1 << 24) || (page_size & (page_size - 1)))
    return fail(BI_E_INVALID_ARG, "%s: page size %lld must be a power of two in [1, 2^24]", what,
                (long long)page_size);
  if (table_stride < (L + page_size - 1) / page_size)
    return fail(BI_E_INVALID_ARG, "%s: table stride %lld < ceil(L / page size) = %lld", what,
                (long long)table_stride, (long long)((L + page_size - 1) / page_size));
  int sh = 0;
  while (((int64_t)1 << sh) < page_size) ++sh;
  *shift = sh;
  return BI_OK;
}

int decode_impl(const char* what, const void* q, const void* k, const void* v, const int32_t* kv_lens, void* out,
                int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t D, const int64_t* strides, float scale,
                int dtype, void* ws, size_t ws_bytes, void* stream, const int32_t* table, int64_t table_stride,
                int page_shift, int64_t num_pages, bool per_key = false, int64_t split = bi::kSplit) {
  using namespace bi_host;
  if (per_key && (split <= 0 || split > kMaxSplit))
    return fail(BI_E_INVALID_ARG, "%s: split_size %lld must be in [1, 2^20]", what, (long long)split);
  if (L > 0x7fffffffLL - split) return fail(BI_E_UNSUPPORTED, "%s: L + split_size exceeds 2^31", what);
  if (B == 0) return BI_OK;
  if (!q || !k || !v || !out || !strides)
    return fail(BI_E_INVALID_ARG, "%s: null pointer argument", what);
  const size_t need = decode_ws_bytes(B, Hq, L, D, split);
  if (!ws || ws_bytes < need)
    return fail(BI_E_WORKSPACE, "%s: workspace of %zu bytes required, got %zu", what, need,
                ws ? ws_bytes : (size_t)0);
  const size_t es = dtype_size(dtype);
  for (int i = 0; i < 8; ++i)
    if (strides[i] < 0 || ((strides[i] * (int64_t)es) % 16))
      return fail(BI_E_INVALID_ARG, "%s: stride %d (%lld) must be >= 0 and 16-byte aligned", what, i,
                  (long long)strides[i]);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(ws))
    return fail(BI_E_INVALID_ARG, "%s: q, k, v and workspace must be 16-byte aligned", what);
  // The contiguous-cache kernel addresses a split's 256 V rows with 32-bit
  // byte offsets.
  if (!table && !per_key && strides[7] * (int64_t)es >= ((int64_t)1 << 23))
    return fail(BI_E_UNSUPPORTED, "%s: V position stride (%lld elements) must stay below 2^23 bytes", what,
                (long long)strides[7]);
  bi::DecodeArgs a;
  a.q = q; a.k = k; a.v = v; a.kv_lens = kv_lens; a.out = out;
  a.table = table; a.table_stride = table_stride; a.page_shift = page_shift; a.num_pages = (int)num_pages;
  a.B = (int)B; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.L = (int)L;
  a.split = (int)split;
  a.nsplit = (int)((L + split - 1) / split);
  const int G = (int)(Hq / Hkv);
  a.GU = per_key ? bi::perkey_decode_nq(B, (int)Hq, (int)Hkv, a.nsplit) : bi::decode_gu(G);
  a.nchunk = G / a.GU;
  a.q_sb = strides[0]; a.q_sh = strides[1];
  a.k_sb = strides[2]; a.k_sh = strides[3]; a.k_sl = strides[4];
  a.v_sb = strides[5]; a.v_sh = strides[6]; a.v_sl = strides[7];
  a.scale_log2 = scale * bi::kLog2e;
  a.scale = scale;
  const int64_t bh = B * Hq * a.nsplit;
  const int64_t up = (bh + 3) / 4 * 4;
  a.pm = static_cast<float*>(ws);
  a.pl = a.pm + up;
  a.pacc = a.pl + up;
  a.ctr = reinterpret_cast<unsigned*>(a.pacc + bh * D);
  if ((int64_t)a.Hkv * a.nchunk > 65535 || a.nsplit > 0x7fffffff ||
      (per_key && bh / a.GU > ((int64_t)1 << 27)))  // per-key: 32 threads per unit, < 2^32 threads
    return fail(BI_E_UNSUPPORTED, "%s: grid too large", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
#define BI_DEC(TY)                                                                                          \
  if (per_key)                                                                                              \
    return bi::with_head_dim_per_key((int)D, [&](auto dd) { return bi::launch_decode_perkey<TY, dd.value>(a, st); }); \
  return bi::with_head_dim((int)D, [&](auto dd) { return bi::launch_decode<TY, dd.value>(a, st); });
  switch (dtype) {
    case BI_BF16: BI_DEC(bi::bf16)
    case BI_F16: BI_DEC(bi::f16)
    case BI_F32: BI_DEC(float)
    default: return fail(BI_E_UNSUPPORTED, "%s: unknown dtype %d", what, dtype);
  }
#undef BI_DEC
}

int prefill_impl(const char* what, const void* q, const void* k, const void* v, const int32_t* kv_lens,
                 void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t L, int64_t D,
                 const int64_t* strides, int causal, float scale, int dtype, void* stream, const int32_t* table,
                 int64_t table_stride, int page_shift, int64_t num_pages, bool per_key = false,
                 int64_t split = bi::kSplit) {
  using namespace bi_host;
  if (per_key && (split <= 0 || split > kMaxSplit))
    return fail(BI_E_INVALID_ARG, "%s: split_size %lld must be in [1, 2^20]", what, (long long)split);
  if (L > 0x7fffffffLL - split) return fail(BI_E_UNSUPPORTED, "%s: L + split_size exceeds 2^31", what);
  if (Tq <= 0) return fail(BI_E_INVALID_ARG, "%s: Tq=%lld", what, (long long)Tq);
  if (causal && Tq > L)
    return fail(BI_E_INVALID_ARG, "%s: causal needs Tq (%lld) <= L (%lld)", what, (long long)Tq, (long long)L);
  if (B == 0) return BI_OK;
  if (!q || !k || !v || !out || !strides) return fail(BI_E_INVALID_ARG, "%s: null pointer argument", what);
  const size_t es = dtype_size(dtype);
  for (int i = 0; i < 9; ++i)
    if (strides[i] < 0 || ((strides[i] * (int64_t)es) % 16))
      return fail(BI_E_INVALID_ARG, "%s: stride %d (%lld) must be >= 0 and 16-byte aligned", what, i,
                  (long long)strides[i]);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return fail(BI_E_INVALID_ARG, "%s: q, k, v, out must be 16-byte aligned", what);
  // The contiguous-cache kernel addresses the 64 rows of a key chunk with
  // 32-bit byte offsets.
  if (!table && !per_key && 64 * std::max(strides[5], strides[8]) * (int64_t)es >= ((int64_t)1 << 30))
    return fail(BI_E_UNSUPPORTED, "%s: K/V row strides (%lld, %lld elements) must stay below 2^24 bytes", what,
                (long long)strides[5], (long long)strides[8]);
  const int64_t wgs = (Tq * (Hq / Hkv) + 63) / 64;
  // The matrix-core kernel runs one 1-D grid over every (b, kv head, 64-pair
  // workgroup) item, padded to a multiple of 8.
  if (wgs > 0x7fffffffLL || Tq * (Hq / Hkv) > 0x7fffffffLL - 64 ||
      (!per_key && wgs * Hkv * B > 0x7fffffffLL - 8) ||
      (per_key && B * Hq * ((Tq + bi::pk_prefill_qb(D) - 1) / bi::pk_prefill_qb(D)) > ((int64_t)1 << 27)))
    return fail(BI_E_UNSUPPORTED, "%s: grid too large", what);
  bi::PrefillArgs a;
  a.q = q; a.k = k; a.v = v; a.kv_lens = kv_lens; a.out = out;
  a.table = table; a.table_stride = table_stride; a.page_shift = page_shift; a.num_pages = (int)num_pages;
  a.B = (int)B; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.Tq = (int)Tq; a.L = (int)L;
  a.causal = causal ? 1 : 0;
  a.q_sb = strides[0]; a.q_sh = strides[1]; a.q_st = strides[2];
  a.k_sb = strides[3]; a.k_sh = strides[4]; a.k_sl = strides[5];
  a.v_sb = strides[6]; a.v_sh = strides[7]; a.v_sl = strides[8];
  a.scale_log2 = scale * bi::kLog2e;
  a.scale = scale;
  a.split = (int)split;
  hipStream_t st = static_cast<hipStream_t>(stream);
#define BI_PRE(TY)                                                                                            \
  if (per_key)                                                                                                \
    return bi::with_head_dim_per_key((int)D, [&](auto dd) { return bi::launch_prefill_perkey<TY, dd.value>(a, st); }); \
  return bi::with_head_dim((int)D, [&](auto dd) { return bi::launch_prefill<TY, dd.value>(a, st); });
  switch (dtype) {
    case BI_BF16: BI_PRE(bi::bf16)
    case BI_F16: BI_PRE(bi::f16)
    case BI_F32: BI_PRE(float)
    default: return fail(BI_E_UNSUPPORTED, "%s: unknown dtype %d", what, dtype);
  }
#undef BI_PRE
}

}  // namespace

extern "C" int bi_attn_decode(const void* q, const void* k, const void* v, const int32_t* kv_lens,
                              void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t D,
                              const int64_t* strides, float scale, int dtype, void* ws,
                              size_t ws_bytes, void* stream) {
  int rc = check_attn_shape("bi_attn_decode", B, Hq, Hkv, L, D);
  if (rc) return rc;
  return decode_impl("bi_attn_decode", q, k, v, kv_lens, out, B, Hq, Hkv, L, D, strides, scale, dtype, ws,
                     ws_bytes, stream, nullptr, 0, 0, 0);
}

extern "C" int bi_attn_decode_paged(const void* q, const void* k_pages, const void* v_pages,
                                    const int32_t* block_table, int64_t table_stride, int64_t page_size,
                                    int64_t num_pages, const int32_t* kv_lens, void* out, int64_t B, int64_t Hq,
                                    int64_t Hkv, int64_t L, int64_t D, const int64_t* strides, float scale,
                                    int dtype, void* ws, size_t ws_bytes, void* stream) {
  int rc = check_attn_shape("bi_attn_decode_paged", B, Hq, Hkv, L, D);
  if (rc) return rc;
  int shift = 0;
  if (B > 0 &&
      (rc = check_pages("bi_attn_decode_paged", block_table, table_stride, page_size, num_pages, L, &shift)))
    return rc;
  return decode_impl("bi_attn_decode_paged", q, k_pages, v_pages, kv_lens, out, B, Hq, Hkv, L, D, strides, scale,
                     dtype, ws, ws_bytes, stream, block_table, table_stride, shift, num_pages);
}

extern "C" int bi_attn_prefill(const void* q, const void* k, const void* v, const int32_t* kv_lens,
                               void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t L,
                               int64_t D, const int64_t* strides, int causal, float scale, int dtype,
                               void* stream) {
  int rc = check_attn_shape("bi_attn_prefill", B, Hq, Hkv, L, D);
  if (rc) return rc;
  return prefill_impl("bi_attn_prefill", q, k, v, kv_lens, out, B, Hq, Hkv, Tq, L, D, strides, causal, scale,
                      dtype, stream, nullptr, 0, 0, 0);
}

extern "C" int bi_attn_prefill_paged(const void* q, const void* k_pages, const void* v_pages,
                                     const int32_t* block_table, int64_t table_stride, int64_t page_size,
                                     int64_t num_pages, const int32_t* kv_lens, void* out, int64_t B, int64_t Hq,
                                     int64_t Hkv, int64_t Tq, int64_t L, int64_t D, const int64_t* strides,
                                     int causal, float scale, int dtype, void* stream) {
  int rc = check_attn_shape("bi_attn_prefill_paged", B, Hq, Hkv, L, D);
  if (rc) return rc;
  int shift = 0;
  if (B > 0 &&
      (rc = check_pages("bi_attn_prefill_paged", block_table, table_stride, page_size, num_pages, L, &shift)))
    return rc;
  return prefill_impl("bi_attn_prefill_paged", q, k_pages, v_pages, kv_lens, out, B, Hq, Hkv, Tq, L, D, strides,
                      causal, scale, dtype, stream, block_table, table_stride, shift, num_pages);
}

// The reference's per-key order (bi_attn_perkey.h): the arguments of
// bi_attn_decode / bi_attn_prefill plus the split size.
extern "C" int bi_attn_decode_per_key(const void* q, const void* k, const void* v, const int32_t* kv_lens,
                                      void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t D,
                                      const int64_t* strides, float scale, int64_t split_size, int dtype, void* ws,
                                      size_t ws_bytes, void* stream) {
  int rc = check_attn_shape("bi_attn_decode_per_key", B, Hq, Hkv, L, D, true);
  if (rc) return rc;
  return decode_impl("bi_attn_decode_per_key", q, k, v, kv_lens, out, B, Hq, Hkv, L, D, strides, scale, dtype, ws,
                     ws_bytes, stream, nullptr, 0, 0, 0, true, split_size);
}

extern "C" int bi_attn_prefill_per_key(const void* q, const void* k, const void* v, const int32_t* kv_lens,
                                       void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t L,
                                       int64_t D, const int64_t* strides, int causal, float scale,
                                       int64_t split_size, int dtype, void* stream) {
  int rc = check_attn_shape("bi_attn_prefill_per_key", B, Hq, Hkv, L, D, true);
  if (rc) return rc;
  return prefill_impl("bi_attn_prefill_per_key", q, k, v, kv_lens, out, B, Hq, Hkv, Tq, L, D, strides, causal,
                      scale, dtype, stream, nullptr, 0, 0, 0, true, split_size);
}

// ---------------------------------------------------------------------------
// Decode without a caller workspace: the partials and the item counter live in
// one file-scope device array. Every GPU the library runs on holds its own copy
// from module load until the process ends; its address is looked up once per
// device (with that device current) and kept. Host code never passes the
// array's name to a kernel: in host code it is only a stand-in for the symbol.
// ---------------------------------------------------------------------------
static __device__ __align__(256) char scratch[BI_DECODE_SCRATCH_BYTES];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[bi::kMaxDev] = {};

// The scratch address of the current device. The kernels run on `stream`, so
// a stream of another device would have them write through this device's
// address: rejected. The address is resolved on the first call per device,
// which must not be under graph capture (the lookup is not a stream operation
// and is not recorded).
int scratch_of_current_device(const char* what, hipStream_t stream, void** out) {
  using namespace bi_host;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail((int)e, "%s: hipGetDevice failed: %s", what, hipGetErrorString(e));
  if (dev < 0 || dev >= bi::kMaxDev) return fail(BI_E_UNSUPPORTED, "%s: device %d out of range", what, dev);
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) return fail((int)e, "%s: hipStreamGetDevice failed: %s", what, hipGetErrorString(e));
    if (sdev != dev)
      return fail(BI_E_INVALID_ARG,
                  "%s: the stream belongs to device %d but device %d is current (the static scratch is the "
                  "current device's)",
                  what, (int)sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &cs);
    if (e != hipSuccess) return fail((int)e, "%s: hipStreamIsCapturing failed: %s", what, hipGetErrorString(e));
    if (cs != hipStreamCaptureStatusNone)
      return fail(BI_E_UNSUPPORTED,
                  "%s: the first call on device %d is under graph capture; make one call outside capture first "
                  "(it resolves the static scratch's address)",
                  what, dev);
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(e != hipSuccess ? (int)e : BI_E_UNSUPPORTED, "%s: hipGetSymbolAddress(scratch) failed: %s", what,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return BI_OK;
}

}  // namespace

extern "C" int bi_attn_decode_noalloc(const void* q, const void* k, const void* v, const int32_t* kv_lens,
                                      void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t D,
                                      const int64_t* strides, float scale, int dtype, void* stream) {
  const char* what = "bi_attn_decode_noalloc";
  int rc = check_attn_shape(what, B, Hq, Hkv, L, D);
  if (rc) return rc;
  if (B == 0) return BI_OK;
  const size_t need = bi_attn_decode_workspace_bytes(B, Hq, L, D);
  if (need > (size_t)BI_DECODE_SCRATCH_BYTES)
    return bi_host::fail(BI_E_WORKSPACE,
                         "%s: B=%lld Hq=%lld L=%lld D=%lld needs %zu bytes of partials; the static scratch holds "
                         "%zu (use bi_attn_decode with a workspace)",
                         what, (long long)B, (long long)Hq, (long long)L, (long long)D, need,
                         (size_t)BI_DECODE_SCRATCH_BYTES);
  void* ws = nullptr;
  if ((rc = scratch_of_current_device(what, static_cast<hipStream_t>(stream), &ws))) return rc;
  return decode_impl(what, q, k, v, kv_lens, out, B, Hq, Hkv, L, D, strides, scale, dtype, ws,
                     (size_t)BI_DECODE_SCRATCH_BYTES, stream, nullptr, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// The attention kernels' exponential as a standalone call (a diagnostic, no
// counterpart in the reference): y[i] = the hardware exp2 (v_exp_f32) of x[i],
// the instruction every split weight and merge factor above is computed with.
// The CPU emulation of the matrix-core order takes this function's values as
// its exp2, so the rest of that order can be checked bit for bit.
// ---------------------------------------------------------------------------
namespace bi {
__global__ __launch_bounds__(256) void exp2_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) y[i] = __builtin_amdgcn_exp2f(x[i]);
}
}  // namespace bi

extern "C" int bi_exp2_f32(const float* x, float* y, int64_t n, void* stream) {
  using namespace bi_host;
  if (n < 0 || n > ((int64_t)1 << 38)) return fail(BI_E_INVALID_ARG, "bi_exp2_f32: bad count %lld", (long long)n);
  if (n == 0) return BI_OK;
  if (!x || !y) return fail(BI_E_INVALID_ARG, "bi_exp2_f32: null pointer argument");
  bi::exp2_kernel<<<(unsigned)((n + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(x, y, n);
  return launch_status("bi_exp2_f32");
}
