// The sampler kernel for fp32 logits and 512-thread work-groups (batches of at least two rows per CU: two
// work-groups a CU, so that one row's fixed phases overlap the other's stream).
#include "spx_kernel.h"

SPX_SAMPLER_VARIANT(float, 512, f32_512)
