// bi_attn_api.h — the attention launchers the C ABI calls, one instantiation
// per (element type, head dim) in bi_attn_{bf16,f16,f32}.hip.
#pragma once

#include "bi_attn_common.h"

namespace bi {

// Query heads of one kv head that a decode work item scores together (the
// columns of its score tile): the largest of 16, 8, 4, 2, 1 dividing G.
inline int decode_gu(int G) {
  for (int gu : {16, 8, 4, 2, 1})
    if (G % gu == 0) return gu;
  return 1;
}

// Queries per per-key prefill unit: 4 up to D = 128, 2 up to 256, else 1 (a
// unit's rows and accumulators grow with D). A query's arithmetic does not
// depend on it (a query takes only its own keys and splits); the K / V rows
// of a key block are loaded and converted once for the unit's queries.
__host__ __device__ constexpr int pk_prefill_qb(int64_t D) { return D <= 128 ? 4 : D <= 256 ? 2 : 1; }

// Query heads a per-key decode unit scores together: 4, 2 or 1 (dividing G), and 1
// while the grid has fewer than 16384 (head, split) pairs, where every unit
// is wanted for parallelism.
inline int perkey_decode_nq(int64_t B, int Hq, int Hkv, int nsplit) {
  const int G = Hq / Hkv;
  if ((int64_t)B * Hq * nsplit < 16384) return 1;
  return G % 4 == 0 ? 4 : G % 2 == 0 ? 2 : 1;
}

template <typename T, int D>
int launch_decode(DecodeArgs& a, hipStream_t st);
template <typename T, int D>
int launch_prefill(PrefillArgs& a, hipStream_t st);
// The reference's per-key order on the vector ALUs (bi_attn_perkey.h).
template <typename T, int D>
int launch_decode_perkey(DecodeArgs& a, hipStream_t st);
template <typename T, int D>
int launch_prefill_perkey(PrefillArgs& a, hipStream_t st);

}  // namespace bi
