// bi_abi.hip — library-wide C-ABI pieces: version, thread-local error text,
// launch-status plumbing.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>

#include "bi_common.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace bi_host {

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return (int)e;
  }
  return BI_OK;
}

}  // namespace bi_host

extern "C" int bi_abi_version(void) { return BI_ABI_VERSION; }
extern "C" const char* bi_last_error(void) { return g_last_error; }

// ---------------------------------------------------------------------------
// Achievable-bandwidth probe (a diagnostic, no counterpart in the reference):
// one pass over `bytes` of device memory, each wave reading whole 1 KB chunks
// (lane l: bytes 16 l .. 16 l + 15 of the chunk), up to kReadAhead chunks per
// wave requested before any is used. Nothing is written unless the xor of a
// thread's data equals `magic` (a value the caller picks), so the loads cannot
// be elided and the pass costs the reads alone.
// ---------------------------------------------------------------------------
namespace bi {
constexpr int kReadAhead = 8;
__global__ __launch_bounds__(512) void stream_read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                          uint32_t* __restrict__ sink, uint32_t magic) {
  const int64_t nwaves = (int64_t)gridDim.x * 8;
  const int64_t wave = (int64_t)blockIdx.x * 8 + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  uint32_t acc = 0;
  for (int64_t c0 = wave; c0 * 64 < n16; c0 += kReadAhead * nwaves) {
    u32x4 v[kReadAhead];
#pragma unroll
    for (int k = 0; k < kReadAhead; ++k) {
      const int64_t i = (c0 + k * nwaves) * 64 + lane;
      v[k] = src[i < n16 ? i : 0];
    }
#pragma unroll
    for (int k = 0; k < kReadAhead; ++k) acc ^= v[k][0] ^ v[k][1] ^ v[k][2] ^ v[k][3];
  }
  if (acc == magic) sink[0] = acc;
}
}  // namespace bi

namespace bi {
// One matrix-core step per block of the probe: lane (r, q) holds A row r and
// B row r (an output column) at k-slots 8 q .. 8 q + 7, and accumulator rows
// 4 q .. 4 q + 3 of column r, as in every matmul kernel of this library.
template <typename T>
__global__ __launch_bounds__(64) void mfma_step_probe_kernel(const T* __restrict__ a, const T* __restrict__ b,
                                                            const float* __restrict__ c, float* __restrict__ d) {
  const int64_t blk = blockIdx.x;
  const int lane = threadIdx.x, r = lane % 16, q = lane / 16;
  const typename Frag<T>::type af = frag_load(a + blk * 512 + r * 32 + 8 * q);
  const typename Frag<T>::type bf = frag_load(b + blk * 512 + r * 32 + 8 * q);
  f32x4 acc;
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] = c[blk * 256 + (4 * q + e) * 16 + r];
  acc = mfma_step(af, bf, acc);
#pragma unroll
  for (int e = 0; e < 4; ++e) d[blk * 256 + (4 * q + e) * 16 + r] = acc[e];
}
}  // namespace bi

extern "C" int bi_mfma_step_probe(const void* a, const void* b, const float* c, float* d, int64_t nblocks,
                                  int dtype, void* stream) {
  using namespace bi_host;
  if (nblocks < 0 || nblocks > ((int64_t)1 << 24))
    return fail(BI_E_INVALID_ARG, "bi_mfma_step_probe: block count %lld outside [0, 2^24]", (long long)nblocks);
  if (dtype != BI_BF16 && dtype != BI_F16 && dtype != BI_F32)
    return fail(BI_E_UNSUPPORTED, "bi_mfma_step_probe: unknown dtype %d", dtype);
  if (nblocks == 0) return BI_OK;
  if (!a || !b || !c || !d || !aligned16(a) || !aligned16(b))
    return fail(BI_E_INVALID_ARG, "bi_mfma_step_probe: null pointer, or a / b not 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned g = (unsigned)nblocks;
  const float* cf = c;
  if (dtype == BI_BF16)
    bi::mfma_step_probe_kernel<bi::bf16><<<g, 64, 0, st>>>(static_cast<const bi::bf16*>(a),
                                                            static_cast<const bi::bf16*>(b), cf, d);
  else if (dtype == BI_F16)
    bi::mfma_step_probe_kernel<bi::f16><<<g, 64, 0, st>>>(static_cast<const bi::f16*>(a),
                                                          static_cast<const bi::f16*>(b), cf, d);
  else
    bi::mfma_step_probe_kernel<float><<<g, 64, 0, st>>>(static_cast<const float*>(a), static_cast<const float*>(b),
                                                        cf, d);
  return launch_status("bi_mfma_step_probe");
}

extern "C" int bi_stream_read(const void* src, int64_t bytes, uint32_t* sink, uint32_t magic, void* stream) {
  using namespace bi_host;
  if (bytes < 0 || bytes % 16 || bytes > ((int64_t)1 << 40))
    return fail(BI_E_INVALID_ARG, "bi_stream_read: bytes (%lld) must be a multiple of 16 in [0, 2^40]", (long long)bytes);
  if (bytes == 0) return BI_OK;
  if (!src || !sink || !aligned16(src)) return fail(BI_E_INVALID_ARG, "bi_stream_read: null or unaligned pointer");
  const int64_t chunks = (bytes / 16 + 63) / 64;
  // about four chunks per wave: every wave resident at once for the sizes of
  // one weight matrix (33 MB: 1,010 workgroups of 8 waves)
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(65535, (chunks + 31) / 32));
  bi::stream_read_kernel<<<(unsigned)blocks, 512, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const bi::u32x4*>(src), bytes / 16, sink, magic);
  return launch_status("bi_stream_read");
}
