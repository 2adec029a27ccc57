// bi_rmsnorm.hip — batch-invariant RMSNorm for gfx950.
//
// Follows the reference kernel kernels/rmsnorm.py:19-47 (one 256-thread
// threadgroup per row, fixed-stride fp32 partials, fixed-shape tree,
// precise rsqrt, out = T((x * inv) * w)); re-laid for CDNA4:
//
//   * one 256-thread workgroup (4 wave64s) per row, whatever the row count;
//   * the row is cut into 8-element chunks (one 16-byte load of bf16/fp16);
//     thread t owns chunks t, t+256, t+512, ... and accumulates
//     ss = fmaf(v, v, ss) over its chunks in order, elements in order;
//   * each wave folds its 64 partials with a fixed xor butterfly
//     (offsets 32, 16, 8, 4, 2, 1), and the four wave sums are folded left to
//     right through LDS: ((S0 + S1) + S2) + S3;
//   * inv = 1 / sqrtf(ss / D + eps), both operations correctly rounded;
//   * out = T((float(x) * inv) * float(w)), rounded to nearest even.
//
// Nothing in that sequence depends on how many rows the launch holds, so a
// row's bits are the same alone or in a batch of thousands.
#include "bi_common.h"

namespace bi {

constexpr int kNormThreads = 256;
constexpr int kNormVec = 8;

// NC = chunks each thread keeps in registers (D <= NC * 2048); VECTOR selects
// 16-byte loads (needs D % 8 == 0 and 16-byte aligned rows). The scalar path
// walks exactly the same elements in the same order.
template <typename T, int NC, bool VECTOR>
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(
    const T* __restrict__ x, int64_t x_stride, const T* __restrict__ w,
    T* __restrict__ out, int D, float eps) {
  __shared__ float wave_sums[kNormThreads / kWave];
  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  const T* xr = x + row * x_stride;
  T* orow = out + row * (int64_t)D;
  const int nchunks = (D + kNormVec - 1) / kNormVec;

  float xv[NC][8];
  float wv[NC][8];
  float ss = 0.0f;
  if constexpr (VECTOR) {
    // Every thread loads a chunk (past the row's end: its last chunk, then
    // zeroed), and the weights are requested with x: no branch before the
    // first load and one memory round trip for x and w together. The sum
    // takes the same elements in the same order.
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int chunk = t + c * kNormThreads;
      const int base = min(chunk, nchunks - 1) * kNormVec;
      load8<T>(xr + base, xv[c]);
      if (w) load8<T>(w + base, wv[c]);
      else {
#pragma unroll
        for (int e = 0; e < 8; ++e) wv[c][e] = 1.0f;
      }
      if (chunk >= nchunks) {
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[c][e] = 0.0f;
      }
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (t + c * kNormThreads < nchunks) {
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(xv[c][e], xv[c][e], ss);
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int chunk = t + c * kNormThreads;
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[c][e] = 0.0f;
      if (chunk < nchunks) {
        const int base = chunk * kNormVec;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (base + e < D) xv[c][e] = (float)xr[base + e];
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(xv[c][e], xv[c][e], ss);
      }
    }
  }

  ss = wave_sum_butterfly(ss);
  const int wave = t / kWave;
  if ((t & (kWave - 1)) == 0) wave_sums[wave] = ss;
  __syncthreads();
  float total = wave_sums[0];
#pragma unroll
  for (int i = 1; i < kNormThreads / kWave; ++i) total = total + wave_sums[i];

  const float mean = total / (float)D;
  const float inv = 1.0f / sqrtf(mean + eps);

#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int chunk = t + c * kNormThreads;
    if (chunk < nchunks) {
      const int base = chunk * kNormVec;
      float o[8];
      if constexpr (VECTOR) {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (xv[c][e] * inv) * wv[c][e];
        store8<T>(orow + base, o);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (base + e < D) {
            const float wv = w ? (float)w[base + e] : 1.0f;
            orow[base + e] = to_store<T>((xv[c][e] * inv) * wv);
          }
        }
      }
    }
  }
}

// D above NC * 2048: same order, but the normalisation pass re-reads x.
template <typename T>
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel_long(
    const T* __restrict__ x, int64_t x_stride, const T* __restrict__ w,
    T* __restrict__ out, int D, float eps) {
  __shared__ float wave_sums[kNormThreads / kWave];
  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  const T* xr = x + row * x_stride;
  T* orow = out + row * (int64_t)D;
  const int nchunks = (D + kNormVec - 1) / kNormVec;
  float ss = 0.0f;
  for (int chunk = t; chunk < nchunks; chunk += kNormThreads) {
    const int base = chunk * kNormVec;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = (base + e < D) ? (float)xr[base + e] : 0.0f;
      ss = __builtin_fmaf(v, v, ss);
    }
  }
  ss = wave_sum_butterfly(ss);
  const int wave = t / kWave;
  if ((t & (kWave - 1)) == 0) wave_sums[wave] = ss;
  __syncthreads();
  float total = wave_sums[0];
#pragma unroll
  for (int i = 1; i < kNormThreads / kWave; ++i) total = total + wave_sums[i];
  const float mean = total / (float)D;
  const float inv = 1.0f / sqrtf(mean + eps);
  for (int i = t; i < D; i += kNormThreads) {
    const float wv = w ? (float)w[i] : 1.0f;
    orow[i] = to_store<T>(((float)xr[i] * inv) * wv);
  }
}

template <typename T>
static int launch_rms(const void* x, int64_t xs, const void* w, void* out, int64_t rows,
                      int64_t D, float eps, hipStream_t st) {
  const T* xp = static_cast<const T*>(x);
  const T* wp = static_cast<const T*>(w);
  T* op = static_cast<T*>(out);
  const bool vec = (D % kNormVec == 0) && (xs % kNormVec == 0) && bi_host::aligned16(x) &&
                   bi_host::aligned16(out) && (w == nullptr || bi_host::aligned16(w));
  dim3 grid((unsigned)rows), block(kNormThreads);
  const int Di = (int)D;
  const int nchunks = (int)((D + kNormVec - 1) / kNormVec);
  if (nchunks <= kNormThreads) {
    if (vec) rms_norm_kernel<T, 1, true><<<grid, block, 0, st>>>(xp, xs, wp, op, Di, eps);
    else rms_norm_kernel<T, 1, false><<<grid, block, 0, st>>>(xp, xs, wp, op, Di, eps);
  } else if (nchunks <= 2 * kNormThreads) {
    if (vec) rms_norm_kernel<T, 2, true><<<grid, block, 0, st>>>(xp, xs, wp, op, Di, eps);
    else rms_norm_kernel<T, 2, false><<<grid, block, 0, st>>>(xp, xs, wp, op, Di, eps);
  } else if (nchunks <= 4 * kNormThreads) {
    if (vec) rms_norm_kernel<T, 4, true><<<grid, block, 0, st>>>(xp, xs, wp, op, Di, eps);
    else rms_norm_kernel<T, 4, false><<<grid, block, 0, st>>>(xp, xs, wp, op, Di, eps);
  } else {
    rms_norm_kernel_long<T><<<grid, block, 0, st>>>(xp, xs, wp, op, Di, eps);
  }
  return bi_host::launch_status("bi_rms_norm");
}

}  // namespace bi

extern "C" int bi_rms_norm(const void* x, int64_t x_row_stride, const void* w, void* out,
                           int64_t rows, int64_t D, float eps, int dtype, void* stream) {
  using namespace bi_host;
  if (rows < 0 || D <= 0 || D > (int64_t)1 << 30)
    return fail(BI_E_INVALID_ARG, "bi_rms_norm: bad shape rows=%lld D=%lld", (long long)rows,
                (long long)D);
  if (rows > 0x7fffffffLL)
    return fail(BI_E_UNSUPPORTED, "bi_rms_norm: rows=%lld exceeds the grid limit",
                (long long)rows);
  if (rows == 0) return BI_OK;
  if (!x || !out) return fail(BI_E_INVALID_ARG, "bi_rms_norm: null x or out");
  if (x_row_stride < D)
    return fail(BI_E_INVALID_ARG, "bi_rms_norm: x_row_stride %lld < D %lld",
                (long long)x_row_stride, (long long)D);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case BI_BF16: return bi::launch_rms<bi::bf16>(x, x_row_stride, w, out, rows, D, eps, st);
    case BI_F16: return bi::launch_rms<bi::f16>(x, x_row_stride, w, out, rows, D, eps, st);
    case BI_F32: return bi::launch_rms<float>(x, x_row_stride, w, out, rows, D, eps, st);
    default: return fail(BI_E_UNSUPPORTED, "bi_rms_norm: unknown dtype %d", dtype);
  }
}
