// bi_attn_f32.hip — attention launchers and kernels for f32 elements, every head dim.
#include "bi_attn_launch.h"

namespace bi {
BI_ATTN_INSTANTIATE(float)
}  // namespace bi
