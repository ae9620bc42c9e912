// kernels_bf16_page16.hip -- instantiates the decode kernels for bf16 KV, 16-token pages (V d-major or token-major)
// (the list is in kernel_set.h).
#include <hip/hip_runtime.h>

#include "kernel_set.h"

SCHED_PD_MFMA_BF16_PAGE16()
