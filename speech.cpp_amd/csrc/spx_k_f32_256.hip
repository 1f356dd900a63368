// The sampler kernel for fp32 logits and 256-thread work-groups.
#include "spx_kernel.h"

SPX_KERNEL_VARIANT(float, 256, f32_256)
