// kernels_wave.hip -- instantiates the one-wave-per-task decode kernels (the
// list is in kernel_set.h).
#include <hip/hip_runtime.h>

#include "kernel_set.h"

SCHED_PD_WAVE_ALL()
