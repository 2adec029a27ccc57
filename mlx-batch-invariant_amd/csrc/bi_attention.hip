// bi_attention.hip — batch-invariant split-KV decode and prefill attention.
//
// Reference: kernels/attention.py of mlx-batch-invariant — decode kernel
// :87-147 (one simdgroup per (batch, kv head, head chunk, split), partials per
// split), combine :149-171 (left fold of splits, precise divide), prefill
// :173-254 (queries share K/V rows, splits folded in registers, bottom-right
// causal mask nkeys = L - Tq + t + 1). Per-split arithmetic: bi_attn_common.h;
// kernels: bi_attn_mfma.h.
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
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "bi_attn_mfma.h"

namespace bi {

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
  // Splits merge strictly left to right; their partials are loaded eight
  // splits at a time ahead of the merges (the loads are independent).
  int i = 0;
  for (; i + 8 <= ns; i += 8) {
    float pm[8], pl[8], pa[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t po = bh * a.nsplit + i + j;
      pm[j] = a.pm[po];
      pl[j] = a.pl[po];
      pa[j] = a.pacc[po * D + d];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) merge_split<1>(M, Ls, &A, pm[j], pl[j], &pa[j]);
  }
  for (; i < ns; ++i) {
    const int64_t po = bh * a.nsplit + i;
    const float acc = a.pacc[po * D + d];
    merge_split<1>(M, Ls, &A, a.pm[po], a.pl[po], &acc);
  }
  // A sequence of length 0 has no split: Ls == 0 and its output is defined as 0.
  static_cast<T*>(a.out)[bh * D + d] = to_store<T>(Ls > 0.0f ? A / Ls : 0.0f);
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
static int decode_gu(int G) {
  for (int gu : {16, 8, 4, 2, 1})
    if (G % gu == 0) return gu;
  return 1;
}

// Workgroups of `kern` (256 threads) that the current device holds at once:
// compute units x resident workgroups per unit, queried once per device and
// kept in the caller's per-kernel cache.
constexpr int kMaxDev = 64;
template <typename K>
static int resident_grid(K kern, int (&cache)[kMaxDev]) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return 0;
  if (cache[dev] > 0) return cache[dev];  // benign race: every writer stores the same value
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, 0) != hipSuccess || cus <= 0 ||
      per_cu <= 0)
    return 0;
  cache[dev] = cus * per_cu;
  return cache[dev];
}

__global__ void zero_counter_kernel(unsigned* c) { *c = 0u; }

// With more possible items than DYN_MIN_ROUNDS rounds of the resident grid,
// items are handed out dynamically (one more tiny launch zeroes the counter:
// a fill kernel, not a memset, so the call can be captured into a graph);
// with fewer, the static order costs nothing extra.
constexpr int kDynMinRounds = 4;

// K/V addressing mode (bi_attn_common.h): contiguous, pages of >= 64 keys, or
// smaller pages.
template <class Args>
static int kv_mode(const Args& a) {
  return !a.table ? kKvContig : a.page_shift >= 6 ? kKvPaged : kKvRowPaged;
}

// Paged caches always take the dynamic item order (one instantiation each).
template <typename T, int D, int GU, int MODE>
static int launch_decode_paged(DecodeArgs& a, int64_t most, hipStream_t st) {
  static int cache[kMaxDev] = {};
  const int grid = resident_grid(attn_decode_mfma<T, D, GU, true, MODE>, cache);
  if (grid <= 0) return bi_host::fail(BI_E_UNSUPPORTED, "bi_attn_decode: device occupancy query failed");
  zero_counter_kernel<<<1, 1, 0, st>>>(a.ctr);
  attn_decode_mfma<T, D, GU, true, MODE><<<(int)std::min<int64_t>(grid, most), 256, 0, st>>>(a);
  return 0;
}

template <typename T, int D, int GU>
static int launch_decode_gu(DecodeArgs& a, hipStream_t st) {
  // Enough resident workgroups to fill the chip, never more than the number
  // of possible items (every sequence at full length).
  const int64_t most = (int64_t)a.B * a.nsplit * a.Hkv * a.nchunk;
  const int mode = kv_mode(a);
  if (mode == kKvPaged) return launch_decode_paged<T, D, GU, kKvPaged>(a, most, st);
  if (mode == kKvRowPaged) return launch_decode_paged<T, D, GU, kKvRowPaged>(a, most, st);
  static int cache[kMaxDev] = {};
  int grid = resident_grid(attn_decode_mfma<T, D, GU, true, kKvContig>, cache);
  if (grid <= 0) return bi_host::fail(BI_E_UNSUPPORTED, "bi_attn_decode: device occupancy query failed");
  if (most > (int64_t)kDynMinRounds * grid) {
    zero_counter_kernel<<<1, 1, 0, st>>>(a.ctr);
    attn_decode_mfma<T, D, GU, true, kKvContig><<<grid, 256, 0, st>>>(a);
  } else {
    grid = (int)std::min<int64_t>(grid, most);
    attn_decode_mfma<T, D, GU, false, kKvContig><<<grid, 256, 0, st>>>(a);
  }
  return 0;
}

template <typename T, int D>
static int launch_decode(DecodeArgs& a, hipStream_t st) {
  int rc0 = 0;
  switch (a.GU) {
    case 16: rc0 = launch_decode_gu<T, D, 16>(a, st); break;
    case 8: rc0 = launch_decode_gu<T, D, 8>(a, st); break;
    case 4: rc0 = launch_decode_gu<T, D, 4>(a, st); break;
    case 2: rc0 = launch_decode_gu<T, D, 2>(a, st); break;
    default: rc0 = launch_decode_gu<T, D, 1>(a, st); break;
  }
  if (rc0) return rc0;
  int rc = bi_host::launch_status("bi_attn_decode");
  if (rc) return rc;
  const int64_t n = (int64_t)a.B * a.Hq * D;
  attn_combine_kernel<T, D><<<(unsigned)((n + 255) / 256), 256, 0, st>>>(a);
  return bi_host::launch_status("bi_attn_decode(combine)");
}

template <typename T, int D>
static int launch_prefill(PrefillArgs& a, hipStream_t st) {
  const int G = a.Hq / a.Hkv;
  const int64_t wgs = ((int64_t)a.Tq * G + 63) / 64;
  dim3 grid((unsigned)wgs, a.Hkv, a.B);
  switch (kv_mode(a)) {
    case kKvPaged: attn_prefill_mfma<T, D, kKvPaged><<<grid, 256, 0, st>>>(a); break;
    case kKvRowPaged: attn_prefill_mfma<T, D, kKvRowPaged><<<grid, 256, 0, st>>>(a); break;
    default: attn_prefill_mfma<T, D, kKvContig><<<grid, 256, 0, st>>>(a); break;
  }
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
  // pm | pl | pacc | item counter (16 bytes), each 16-byte aligned
  auto up = [](int64_t x) { return (x + 3) / 4 * 4; };
  return (size_t)(up(bh) * 2 + bh * D + 4) * sizeof(float);
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
                int page_shift, int64_t num_pages) {
  using namespace bi_host;
  if (B == 0) return BI_OK;
  if (!q || !k || !v || !out || !strides)
    return fail(BI_E_INVALID_ARG, "%s: null pointer argument", what);
  const size_t need = bi_attn_decode_workspace_bytes(B, Hq, L, D);
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
  bi::DecodeArgs a;
  a.q = q; a.k = k; a.v = v; a.kv_lens = kv_lens; a.out = out;
  a.table = table; a.table_stride = table_stride; a.page_shift = page_shift; a.num_pages = (int)num_pages;
  a.B = (int)B; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.L = (int)L;
  a.nsplit = (int)((L + bi::kSplit - 1) / bi::kSplit);
  const int G = (int)(Hq / Hkv);
  a.GU = bi::decode_gu(G);
  a.nchunk = G / a.GU;
  a.q_sb = strides[0]; a.q_sh = strides[1];
  a.k_sb = strides[2]; a.k_sh = strides[3]; a.k_sl = strides[4];
  a.v_sb = strides[5]; a.v_sh = strides[6]; a.v_sl = strides[7];
  a.scale_log2 = scale * bi::kLog2e;
  const int64_t bh = B * Hq * a.nsplit;
  const int64_t up = (bh + 3) / 4 * 4;
  a.pm = static_cast<float*>(ws);
  a.pl = a.pm + up;
  a.pacc = a.pl + up;
  a.ctr = reinterpret_cast<unsigned*>(a.pacc + bh * D);
  if ((int64_t)a.Hkv * a.nchunk > 65535 || a.nsplit > 0x7fffffff)
    return fail(BI_E_UNSUPPORTED, "%s: grid too large", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
#define BI_DEC(TY)                                                         \
  return D == 64 ? bi::launch_decode<TY, 64>(a, st) : bi::launch_decode<TY, 128>(a, st);
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
                 int64_t table_stride, int page_shift, int64_t num_pages) {
  using namespace bi_host;
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
  const int64_t wgs = (Tq * (Hq / Hkv) + 63) / 64;
  if (wgs > 0x7fffffffLL || Tq * (Hq / Hkv) > 0x7fffffffLL - 64)
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
  hipStream_t st = static_cast<hipStream_t>(stream);
#define BI_PRE(TY)                                                           \
  return D == 64 ? bi::launch_prefill<TY, 64>(a, st) : bi::launch_prefill<TY, 128>(a, st);
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

int scratch_of_current_device(const char* what, void** out) {
  using namespace bi_host;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail((int)e, "%s: hipGetDevice failed: %s", what, hipGetErrorString(e));
  if (dev < 0 || dev >= bi::kMaxDev) return fail(BI_E_UNSUPPORTED, "%s: device %d out of range", what, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
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
  if ((rc = scratch_of_current_device(what, &ws))) return rc;
  return decode_impl(what, q, k, v, kv_lens, out, B, Hq, Hkv, L, D, strides, scale, dtype, ws,
                     (size_t)BI_DECODE_SCRATCH_BYTES, stream, nullptr, 0, 0, 0);
}
