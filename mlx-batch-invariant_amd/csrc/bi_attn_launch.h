// bi_attn_launch.h — host launchers of the attention kernels (decode items +
// combine, prefill), included by the per-element-type translation units
// bi_attn_{bf16,f16,f32}.hip, which instantiate them for every head dim; the
// C ABI in bi_attention.hip calls them through the declarations of
// bi_attn_api.h.
#pragma once

#include <algorithm>
#include <type_traits>

#include "bi_attn_api.h"
#include "bi_attn_mfma.h"
#include "bi_attn_perkey.h"

namespace bi {

template <typename T, int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(DecodeArgs a) {
  // Threads past the end compute element 0 and do not store it (no early
  // return: the kernel arguments are then read in one round).
  const int64_t gid0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)a.B * a.Hq * D;
  const bool live = gid0 < total;
  const int64_t gid = live ? gid0 : 0;
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
  if (live) static_cast<T*>(a.out)[bh * D + d] = to_store<T>(Ls > 0.0f ? A / Ls : 0.0f);
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------

// Workgroups of `kern` (256 threads) that the current device holds at once:
// compute units x resident workgroups per unit, queried once per device and
// kept in the caller's per-kernel cache.
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

template <typename U>
__global__ void zero_counter_kernel(U* c) { *c = 0u; }

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
int launch_decode(DecodeArgs& a, hipStream_t st) {
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
int launch_prefill(PrefillArgs& a, hipStream_t st) {
  const int G = a.Hq / a.Hkv;
  const int64_t wgs = ((int64_t)a.Tq * G + 63) / 64;
  const int64_t items = wgs * a.Hkv * a.B;     // the kernel maps blocks to items per XCD
  dim3 grid((unsigned)(8 * ((items + 7) / 8)));
  switch (kv_mode(a)) {
    case kKvPaged: attn_prefill_mfma<T, D, kKvPaged><<<grid, 256, 0, st>>>(a); break;
    case kKvRowPaged: attn_prefill_mfma<T, D, kKvRowPaged><<<grid, 256, 0, st>>>(a); break;
    default: attn_prefill_mfma<T, D, kKvContig><<<grid, 256, 0, st>>>(a); break;
  }
  return bi_host::launch_status("bi_attn_prefill");
}

#define BI_ATTN_INSTANTIATE_D(T, D)                                   \
  template int launch_decode<T, D>(DecodeArgs&, hipStream_t);        \
  template int launch_prefill<T, D>(PrefillArgs&, hipStream_t);      \
  template int launch_decode_perkey<T, D>(DecodeArgs&, hipStream_t); \
  template int launch_prefill_perkey<T, D>(PrefillArgs&, hipStream_t);
#define BI_ATTN_PERKEY_INSTANTIATE_D(T, D)                            \
  template int launch_decode_perkey<T, D>(DecodeArgs&, hipStream_t); \
  template int launch_prefill_perkey<T, D>(PrefillArgs&, hipStream_t);
// Head dims of the per-key kernels only (every multiple of 32 up to 512).
#define BI_ATTN_PERKEY_EXTRA(T)                                                                          \
  BI_ATTN_PERKEY_INSTANTIATE_D(T, 160) BI_ATTN_PERKEY_INSTANTIATE_D(T, 224)                             \
  BI_ATTN_PERKEY_INSTANTIATE_D(T, 288) BI_ATTN_PERKEY_INSTANTIATE_D(T, 320)                             \
  BI_ATTN_PERKEY_INSTANTIATE_D(T, 352) BI_ATTN_PERKEY_INSTANTIATE_D(T, 384)                             \
  BI_ATTN_PERKEY_INSTANTIATE_D(T, 416) BI_ATTN_PERKEY_INSTANTIATE_D(T, 448)                             \
  BI_ATTN_PERKEY_INSTANTIATE_D(T, 480) BI_ATTN_PERKEY_INSTANTIATE_D(T, 512)
#define BI_ATTN_INSTANTIATE(T)                                                                           \
  BI_ATTN_INSTANTIATE_D(T, 32) BI_ATTN_INSTANTIATE_D(T, 64) BI_ATTN_INSTANTIATE_D(T, 96)                \
  BI_ATTN_INSTANTIATE_D(T, 128) BI_ATTN_INSTANTIATE_D(T, 192) BI_ATTN_INSTANTIATE_D(T, 256)

}  // namespace bi
