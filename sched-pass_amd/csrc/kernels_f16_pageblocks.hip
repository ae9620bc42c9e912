// kernels_f16_pageblocks.hip -- instantiates the decode kernels for fp16 KV
// with fp16 Q on pages of 32..256 tokens (the list is in kernel_set.h).
#include <hip/hip_runtime.h>

#include "kernel_set.h"

SCHED_PD_MFMA_F16_PAGEBLOCKS()
