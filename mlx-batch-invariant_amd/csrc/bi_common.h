// bi_common.h — shared device-side vocabulary of the gfx950 kernels:
// element types, 16-byte fragments, the one MFMA step every matmul tile uses,
// rounding helpers, and the host-side error plumbing of the C ABI.
//
// Numerics policy (applies to every kernel in this library; the build passes
// -ffp-contract=off and no fast-math flag):
//   * every fused multiply-add is written as an explicit __builtin_fmaf;
//   * fp32 division and sqrtf are IEEE correctly rounded (hipcc's default
//     -fhip-fp32-correctly-rounded-divide-sqrt); exp is the device library's
//     full-precision expf, or, for the attention weights and split merge, the
//     hardware exp2 (v_exp_f32) on log2-scaled scores — one fixed choice per
//     quantity, shared by every kernel that computes it;
//   * fp32 -> bf16 / fp16 conversion rounds to nearest even;
//   * denormals are kept (no flush-to-zero).
// This is the HIP counterpart of the reference's `metal::precise::` policy
// (kernels/__init__.py:12-17 of mlx-batch-invariant).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/bi_kernels.h"

namespace bi {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr int kGroupK = BI_GROUP_K;  // fixed K group of the matmul fold
constexpr int kSteps = 8;            // MFMA steps per K group (8 x 32 = 256)
constexpr int kSplit = BI_SPLIT_KEYS;

// ---------------------------------------------------------------------------
// Fragments. One MFMA "step" consumes, per lane, 8 consecutive-in-memory
// elements of A and 8 of B. For 16-bit types that is one 16-byte register
// quad and one v_mfma_f32_16x16x32_{bf16,f16}; for fp32 it is 32 bytes and a
// chain of eight v_mfma_f32_16x16x4_f32 (element e of every lane in sub-step e).
// ---------------------------------------------------------------------------
template <typename T> struct Frag;
template <> struct Frag<bf16> { typedef bf16x8 type; };
template <> struct Frag<f16> { typedef f16x8 type; };
struct f32x8 { f32x4 lo, hi; };
template <> struct Frag<float> { typedef f32x8 type; };

__device__ __forceinline__ f32x4 mfma_step(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_step(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_step(f32x8 a, f32x8 b, f32x4 c) {
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[0], b.lo[0], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[1], b.lo[1], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[2], b.lo[2], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[3], b.lo[3], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[0], b.hi[0], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[1], b.hi[1], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[2], b.hi[2], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[3], b.hi[3], c, 0, 0, 0);
  return c;
}

template <typename F> __device__ __forceinline__ F frag_zero();
template <> __device__ __forceinline__ bf16x8 frag_zero<bf16x8>() {
  u32x4 z = {0u, 0u, 0u, 0u};
  return __builtin_bit_cast(bf16x8, z);
}
template <> __device__ __forceinline__ f16x8 frag_zero<f16x8>() {
  u32x4 z = {0u, 0u, 0u, 0u};
  return __builtin_bit_cast(f16x8, z);
}
template <> __device__ __forceinline__ f32x8 frag_zero<f32x8>() {
  f32x8 z;
  z.lo = f32x4{0.f, 0.f, 0.f, 0.f};
  z.hi = z.lo;
  return z;
}

// Load 8 consecutive elements (16 or 32 bytes, naturally aligned).
__device__ __forceinline__ bf16x8 frag_load(const bf16* p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ f16x8 frag_load(const f16* p) {
  return __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ f32x8 frag_load(const float* p) {
  f32x8 r;
  r.lo = *reinterpret_cast<const f32x4*>(p);
  r.hi = *reinterpret_cast<const f32x4*>(p + 4);
  return r;
}

// ---------------------------------------------------------------------------
// Rounding. fp32 -> storage type, round to nearest even (hardware
// v_cvt_pk_bf16_f32 / v_cvt_f16_f32 on gfx950).
// ---------------------------------------------------------------------------
//
// The empty asm keeps the fp32 value materialised in a register, so the
// conversion rounds exactly that value. Without it the compiler may fold the
// producing fp32 multiply/add/fma into the conversion (v_fma_mixlo_f16 with a
// zero addend), rounding once where the canonical order rounds twice, and
// turning a -0 product into +0.
__device__ __forceinline__ float materialize(float x) {
  asm volatile("" : "+v"(x));
  return x;
}
template <typename T> __device__ __forceinline__ T to_store(float x);
template <> __device__ __forceinline__ bf16 to_store<bf16>(float x) { return (bf16)materialize(x); }
template <> __device__ __forceinline__ f16 to_store<f16>(float x) { return (f16)materialize(x); }
template <> __device__ __forceinline__ float to_store<float>(float x) { return x; }

template <typename T> __device__ __forceinline__ float to_f32(T x) { return (float)x; }

// Whole-wave reductions / scans over 64 lanes with a fixed butterfly shape.
__device__ __forceinline__ float wave_sum_butterfly(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off, kWave);
  return v;
}

// Eight consecutive elements of a row as fp32 (one 16-byte load for 2-byte
// types, two for fp32), and back with round-to-nearest-even stores.
template <typename T>
__device__ __forceinline__ void load8(const T* p, float* out) {
  if constexpr (sizeof(T) == 2) {
    u32x4 raw = *reinterpret_cast<const u32x4*>(p);
    const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = (float)e[i];
  } else {
    f32x4 a = *reinterpret_cast<const f32x4*>(p);
    f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[i] = a[i];
      out[4 + i] = b[i];
    }
  }
}

template <typename T>
__device__ __forceinline__ void store8(T* p, const float* in) {
  if constexpr (sizeof(T) == 2) {
    u32x4 raw;
    T* e = reinterpret_cast<T*>(&raw);
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = to_store<T>(in[i]);
    *reinterpret_cast<u32x4*>(p) = raw;
  } else {
    f32x4 a = {in[0], in[1], in[2], in[3]};
    f32x4 b = {in[4], in[5], in[6], in[7]};
    *reinterpret_cast<f32x4*>(p) = a;
    *reinterpret_cast<f32x4*>(p + 4) = b;
  }
}

// ---------------------------------------------------------------------------
// Direct global -> LDS copies (global_load_lds_dwordx4) and the barrier that
// waits for them.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void gbl_void_t;

// One 16-byte-per-lane copy global -> LDS; lane l lands at lds_block + 16 l.
__device__ __forceinline__ void copy_to_lds16(const void* src, void* lds_block) {
  __builtin_amdgcn_global_load_lds((gbl_void_t*)src, (lds_void_t*)lds_block, 16, 0, 0);
}

// The same copy through a buffer resource over [base, base + bytes): lane l
// reads base + voffset (zero past the range) and lands at lds_block + 16 l.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}
__device__ __forceinline__ void copy_to_lds16(__amdgpu_buffer_rsrc_t rs, int voffset, void* lds_block) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)lds_block, 16, voffset, 0, 0, 0);
}

// s_waitcnt vmcnt(N) lgkmcnt(0); the empty asm statements keep the compiler
// from moving memory accesses across it.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));
  asm volatile("" ::: "memory");
}

// Stage barrier: wait until at most N vector-memory operations of this wave
// are outstanding (vmcnt counts global_load_lds copies until their data is in
// LDS; they complete in issue order) and all of its LDS reads have returned,
// then s_barrier. Unlike __syncthreads() this does not drain the copies of
// later stages that are still in flight. The empty asm statements keep the
// compiler from moving memory accesses across the barrier.
template <int N>
__device__ __forceinline__ void stage_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("" ::: "memory");
  // gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace bi

// ---------------------------------------------------------------------------
// Host-side helpers shared by the C-ABI translation units.
// ---------------------------------------------------------------------------
namespace bi_host {
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int launch_status(const char* what);
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline size_t dtype_size(int dt) { return dt == BI_F32 ? 4 : 2; }
}  // namespace bi_host
