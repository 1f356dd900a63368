// The sampler kernel for fp32 logits and 1024-thread work-groups.
#include "spx_kernel.h"

SPX_KERNEL_VARIANT(float, 1024, f32_1024)
