// kernels_fp8_tokmajor.hip -- instantiates the decode kernels for fp8 KV
// with a token-major V (the list is in kernel_set.h).
#include <hip/hip_runtime.h>

#include "kernel_set.h"

SCHED_PD_MFMA_FP8_TOKMAJOR()
