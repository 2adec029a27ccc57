// bi_attn_f16.hip — attention launchers and kernels for f16 elements, every head dim.
#include "bi_attn_launch.h"

namespace bi {
BI_ATTN_INSTANTIATE(f16)
}  // namespace bi
