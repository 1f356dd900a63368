// The sampler kernel for bf16 logits and 256-thread work-groups.
#include "spx_kernel.h"

SPX_KERNEL_VARIANT(uint16_t, 256, bf16_256)
