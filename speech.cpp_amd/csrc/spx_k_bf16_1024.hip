// The sampler kernel for bf16 logits and 1024-thread work-groups.
#include "spx_kernel.h"

SPX_KERNEL_VARIANT(uint16_t, 1024, bf16_1024)
