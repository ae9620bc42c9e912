// kernels_wave_groups.hip -- instantiates the one-wave-per-task decode
// kernels for 2 and 3 q-heads per kv-head (the list is in kernel_set.h).
#include <hip/hip_runtime.h>

#include "kernel_set.h"

SCHED_PD_WAVE_GROUPS()
