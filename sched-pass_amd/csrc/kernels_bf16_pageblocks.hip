// kernels_bf16_pageblocks.hip -- instantiates the decode kernels for bf16 KV, 32..256-token pages
// (the list is in kernel_set.h).
#include <hip/hip_runtime.h>

#include "kernel_set.h"

SCHED_PD_MFMA_BF16_PAGEBLOCKS()
