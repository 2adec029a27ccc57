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

template <typename T, int D>
int launch_decode(DecodeArgs& a, hipStream_t st);
template <typename T, int D>
int launch_prefill(PrefillArgs& a, hipStream_t st);

}  // namespace bi
