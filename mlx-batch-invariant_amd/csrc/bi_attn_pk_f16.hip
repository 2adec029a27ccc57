// bi_attn_pk_f16.hip — the per-key attention launchers for f16 elements at the
// head dims only they take (multiples of 32 up to 512 beyond the six of the
// matrix-core kernels); their own translation unit so the build compiles them
// beside the others.
#include "bi_attn_launch.h"

namespace bi {
BI_ATTN_PERKEY_EXTRA(f16)
}  // namespace bi
