// kernels_fp8.hip -- instantiates the decode kernels for fp8 e4m3fn KV, all page sizes
// (the list is in kernel_set.h).
#include <hip/hip_runtime.h>

#include "kernel_set.h"

SCHED_PD_MFMA_FP8()
