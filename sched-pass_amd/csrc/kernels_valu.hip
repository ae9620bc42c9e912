// kernels_valu.hip -- instantiates the decode kernels for the VALU kernels
// (the list is in kernel_set.h).
#include <hip/hip_runtime.h>

#include "kernel_set.h"

SCHED_PD_VALU_ALL()
