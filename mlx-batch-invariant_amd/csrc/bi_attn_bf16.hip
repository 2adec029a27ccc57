// bi_attn_bf16.hip — attention launchers and kernels for bf16 elements, every head dim.
#include "bi_attn_launch.h"

namespace bi {
BI_ATTN_INSTANTIATE(bf16)
}  // namespace bi
