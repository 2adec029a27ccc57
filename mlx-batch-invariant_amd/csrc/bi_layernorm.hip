// bi_layernorm.hip — batch-invariant LayerNorm over the last dimension for
// gfx950.
//
// The reference has no LayerNorm kernel: it lists "a batch-invariant
// mx.fast.layer_norm" as a roadmap item (README.md:257-260) and relies on the
// stock op for GPT-2 (README.md:250-251). This kernel gives LayerNorm the
// same kind of contract as RMSNorm (kernels/rmsnorm.py:19-47 there,
// bi_rmsnorm.hip here), with a two-pass canonical order:
//
//   * one 256-thread workgroup (4 wave64s) per row, whatever the row count;
//     the row is cut into 8-element chunks and thread t owns chunks t,
//     t+256, t+512, ... (elements in order within a chunk);
//   * pass 1: s = s + x over the thread's elements, each wave folds its 64
//     partials with the xor butterfly (offsets 32 .. 1), the four wave sums
//     are added left to right; mean = total / D;
//   * pass 2: d = x - mean, ss = fmaf(d, d, ss) over the same elements (only
//     k < D), the same tree; var = total / D (biased, as torch's);
//     inv = 1 / sqrtf(var + eps), correctly rounded division and square root;
//   * out = T(((x - mean) * inv) * w + b); the multiply by w and the add of b
//     are skipped when the tensor is absent; one round-to-nearest-even store.
//
// Nothing in that sequence depends on how many rows the launch holds.
#include "bi_common.h"

namespace bi {

constexpr int kLnThreads = 256;
constexpr int kLnVec = 8;

// Sum of one value per thread in the fixed order: butterfly per wave, then the
// four wave sums left to right. `slot` holds the wave sums; every thread gets
// the total.
__device__ __forceinline__ float ln_block_sum(float v, float* slot) {
  v = wave_sum_butterfly(v);
  const int t = threadIdx.x;
  if ((t & (kWave - 1)) == 0) slot[t / kWave] = v;
  __syncthreads();
  float total = slot[0];
#pragma unroll
  for (int i = 1; i < kLnThreads / kWave; ++i) total = total + slot[i];
  return total;
}

template <typename T>
__device__ __forceinline__ float ln_out(float d, float inv, const T* w, const T* b, int k) {
  float y = d * inv;
  if (w) y = y * (float)w[k];
  if (b) y = y + (float)b[k];
  return y;
}

// NC = chunks each thread keeps in registers (D <= NC * 2048); VECTOR selects
// 16-byte loads (D % 8 == 0, 16-byte aligned rows). The scalar path walks the
// same elements in the same order.
template <typename T, int NC, bool VECTOR>
__global__ __launch_bounds__(kLnThreads) void layer_norm_kernel(const T* __restrict__ x, int64_t x_stride,
                                                                const T* __restrict__ w,
                                                                const T* __restrict__ b, T* __restrict__ out,
                                                                int D, float eps) {
  __shared__ float sums[2][kLnThreads / kWave];
  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  const T* xr = x + row * x_stride;
  T* orow = out + row * (int64_t)D;
  const int nchunks = (D + kLnVec - 1) / kLnVec;

  float xv[NC][8];
  float wv[NC][8], bv[NC][8];
  float s = 0.0f;
  if constexpr (VECTOR) {
    // Every thread loads a chunk (past the row's end: its last chunk, then
    // zeroed) and the weight and bias chunks with it: no branch before the
    // first load and one memory round trip for x, w and b. The sums take the
    // same elements in the same order.
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int chunk = t + c * kLnThreads;
      const int base = min(chunk, nchunks - 1) * kLnVec;
      load8<T>(xr + base, xv[c]);
      if (w) load8<T>(w + base, wv[c]);
      if (b) load8<T>(b + base, bv[c]);
      if (chunk >= nchunks) {
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[c][e] = 0.0f;
      }
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (t + c * kLnThreads < nchunks) {
#pragma unroll
        for (int e = 0; e < 8; ++e) s = s + xv[c][e];
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int chunk = t + c * kLnThreads;
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[c][e] = 0.0f;
      if (chunk < nchunks) {
        const int base = chunk * kLnVec;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (base + e < D) xv[c][e] = (float)xr[base + e];
        // Elements past D are +0 here: adding them leaves s unchanged (s
        // starts at +0 and a round-to-nearest sum is never -0 unless both
        // terms are).
#pragma unroll
        for (int e = 0; e < 8; ++e) s = s + xv[c][e];
      }
    }
  }
  const float mean = ln_block_sum(s, sums[0]) / (float)D;

  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int chunk = t + c * kLnThreads;
    if (chunk < nchunks) {
      const int base = chunk * kLnVec;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = xv[c][e] - mean;
        if (VECTOR || base + e < D) ss = __builtin_fmaf(d, d, ss);
      }
    }
  }
  const float var = ln_block_sum(ss, sums[1]) / (float)D;
  const float inv = 1.0f / sqrtf(var + eps);

#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int chunk = t + c * kLnThreads;
    if (chunk < nchunks) {
      const int base = chunk * kLnVec;
      if constexpr (VECTOR) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float y = (xv[c][e] - mean) * inv;
          if (w) y = y * wv[c][e];
          if (b) y = y + bv[c][e];
          o[e] = y;
        }
        store8<T>(orow + base, o);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (base + e < D) orow[base + e] = to_store<T>(ln_out<T>(xv[c][e] - mean, inv, w, b, base + e));
      }
    }
  }
}

// D above NC * 2048: the same order, with x read again in each pass.
template <typename T>
__global__ __launch_bounds__(kLnThreads) void layer_norm_kernel_long(const T* __restrict__ x, int64_t x_stride,
                                                                     const T* __restrict__ w,
                                                                     const T* __restrict__ b,
                                                                     T* __restrict__ out, int D, float eps) {
  __shared__ float sums[2][kLnThreads / kWave];
  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  const T* xr = x + row * x_stride;
  T* orow = out + row * (int64_t)D;
  const int nchunks = (D + kLnVec - 1) / kLnVec;
  float s = 0.0f;
  for (int chunk = t; chunk < nchunks; chunk += kLnThreads) {
    const int base = chunk * kLnVec;
#pragma unroll
    for (int e = 0; e < 8; ++e) s = s + ((base + e < D) ? (float)xr[base + e] : 0.0f);
  }
  const float mean = ln_block_sum(s, sums[0]) / (float)D;
  float ss = 0.0f;
  for (int chunk = t; chunk < nchunks; chunk += kLnThreads) {
    const int base = chunk * kLnVec;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (base + e < D) {
        const float d = (float)xr[base + e] - mean;
        ss = __builtin_fmaf(d, d, ss);
      }
    }
  }
  const float var = ln_block_sum(ss, sums[1]) / (float)D;
  const float inv = 1.0f / sqrtf(var + eps);
  for (int i = t; i < D; i += kLnThreads) orow[i] = to_store<T>(ln_out<T>((float)xr[i] - mean, inv, w, b, i));
}

template <typename T>
static int launch_ln(const void* x, int64_t xs, const void* w, const void* b, void* out, int64_t rows,
                     int64_t D, float eps, hipStream_t st) {
  const T* xp = static_cast<const T*>(x);
  const T* wp = static_cast<const T*>(w);
  const T* bp = static_cast<const T*>(b);
  T* op = static_cast<T*>(out);
  const bool vec = (D % kLnVec == 0) && (xs % kLnVec == 0) && bi_host::aligned16(x) && bi_host::aligned16(out) &&
                   (w == nullptr || bi_host::aligned16(w)) && (b == nullptr || bi_host::aligned16(b));
  const dim3 grid((unsigned)rows), block(kLnThreads);
  const int Di = (int)D;
  const int nchunks = (int)((D + kLnVec - 1) / kLnVec);
  if (nchunks <= kLnThreads) {
    if (vec) layer_norm_kernel<T, 1, true><<<grid, block, 0, st>>>(xp, xs, wp, bp, op, Di, eps);
    else layer_norm_kernel<T, 1, false><<<grid, block, 0, st>>>(xp, xs, wp, bp, op, Di, eps);
  } else if (nchunks <= 2 * kLnThreads) {
    if (vec) layer_norm_kernel<T, 2, true><<<grid, block, 0, st>>>(xp, xs, wp, bp, op, Di, eps);
    else layer_norm_kernel<T, 2, false><<<grid, block, 0, st>>>(xp, xs, wp, bp, op, Di, eps);
  } else if (nchunks <= 4 * kLnThreads) {
    if (vec) layer_norm_kernel<T, 4, true><<<grid, block, 0, st>>>(xp, xs, wp, bp, op, Di, eps);
    else layer_norm_kernel<T, 4, false><<<grid, block, 0, st>>>(xp, xs, wp, bp, op, Di, eps);
  } else {
    layer_norm_kernel_long<T><<<grid, block, 0, st>>>(xp, xs, wp, bp, op, Di, eps);
  }
  return bi_host::launch_status("bi_layer_norm");
}

}  // namespace bi

extern "C" int bi_layer_norm(const void* x, int64_t x_row_stride, const void* w, const void* b, void* out,
                             int64_t rows, int64_t D, float eps, int dtype, void* stream) {
  using namespace bi_host;
  if (rows < 0 || D <= 0 || D > (int64_t)1 << 30)
    return fail(BI_E_INVALID_ARG, "bi_layer_norm: bad shape rows=%lld D=%lld", (long long)rows, (long long)D);
  if (rows > 0x7fffffffLL)
    return fail(BI_E_UNSUPPORTED, "bi_layer_norm: rows=%lld exceeds the grid limit", (long long)rows);
  if (rows == 0) return BI_OK;
  if (!x || !out) return fail(BI_E_INVALID_ARG, "bi_layer_norm: null x or out");
  if (x_row_stride < D)
    return fail(BI_E_INVALID_ARG, "bi_layer_norm: x_row_stride %lld < D %lld", (long long)x_row_stride,
                (long long)D);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case BI_BF16: return bi::launch_ln<bi::bf16>(x, x_row_stride, w, b, out, rows, D, eps, st);
    case BI_F16: return bi::launch_ln<bi::f16>(x, x_row_stride, w, b, out, rows, D, eps, st);
    case BI_F32: return bi::launch_ln<float>(x, x_row_stride, w, b, out, rows, D, eps, st);
    default: return fail(BI_E_UNSUPPORTED, "bi_layer_norm: unknown dtype %d", dtype);
  }
}
