// staging.hip -- host-to-device copies of a serving step's small arrays
// (lengths, split plan, block-table updates, orders, control rows).
//
// A step's arrays are staged in pinned host memory and copied to the device
// on the launch stream right before the kernels that read them. With
// hipMemcpyAsync the copy engine moves them: the engine waits for the
// previous kernel's completion signal, copies, and the next kernel then
// waits for the engine's signal, ~25-45 us per step on MI355X for a few KB.
// Memory from sched_pd_staging_alloc is mapped into the device's address
// space, so a small copy out of it runs as a kernel on the stream itself:
// one 8-byte (or 4-, or 1-byte, by alignment) system-scope load per lane
// over the host link, no hand-off between engines. Any other source takes
// hipMemcpyAsync.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "../../include/sched_pd.h"
#include "rt_internal.h"

namespace {

// Largest copy that runs as a kernel; larger ones are bandwidth work that
// the copy engine does better.
constexpr uint64_t kKernelCopyMax = 1ull << 20;
constexpr uint64_t kStagingMax = 1ull << 32;
constexpr int kMaxRegions = 64;

struct Region {
  uintptr_t host;
  uintptr_t dev;
  uint64_t bytes;
};

std::mutex g_mu;
Region g_regions[kMaxRegions];
int g_nregions = 0;

// Coherent (fine-grained) host memory is not cached by the device; the
// system-scope loads see the host's latest writes either way.
template <typename W>
__global__ void __launch_bounds__(256) staging_copy(W *__restrict__ dst, const W *__restrict__ src,
                                                    uint64_t nwords, uint8_t *__restrict__ dtail,
                                                    const uint8_t *__restrict__ stail,
                                                    uint32_t ntail) {
  const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (i < nwords)
    dst[i] = __hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  if (blockIdx.x == 0 && threadIdx.x < ntail)
    dtail[threadIdx.x] =
        __hip_atomic_load(stail + threadIdx.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Device address of [src, src + bytes) if the whole range lies in one
// staging region, else 0.
uintptr_t staged_device_address(const void *src, uint64_t bytes) {
  const uintptr_t s = reinterpret_cast<uintptr_t>(src);
  std::lock_guard<std::mutex> g(g_mu);
  for (int r = 0; r < g_nregions; ++r) {
    const Region &R = g_regions[r];
    if (s >= R.host && bytes <= R.bytes && s - R.host <= R.bytes - bytes)
      return R.dev + (s - R.host);
  }
  return 0;
}

// True when [p, p + bytes) lies in one device allocation. hipMemcpyAsync
// refuses a copy past its destination's allocation; the kernel would write
// past it, so it runs only where the range is known to fit.
bool fits_device_allocation(const void *p, uint64_t bytes) {
  hipPointerAttribute_t at;
  if (hipPointerGetAttributes(&at, p) != hipSuccess) {
    (void)hipGetLastError();       // an unknown pointer is an answer, not an error
    return false;
  }
  if (at.type != hipMemoryTypeDevice)
    return false;
  hipDeviceptr_t dp = reinterpret_cast<hipDeviceptr_t>(const_cast<void *>(p));
  uintptr_t start = 0;
  size_t size = 0;
  if (hipPointerGetAttribute(&start, HIP_POINTER_ATTRIBUTE_RANGE_START_ADDR, dp) != hipSuccess ||
      hipPointerGetAttribute(&size, HIP_POINTER_ATTRIBUTE_RANGE_SIZE, dp) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  const uintptr_t d = reinterpret_cast<uintptr_t>(p);
  return start != 0 && d >= start && bytes <= size && d - start <= size - bytes;
}

template <typename W>
hipError_t launch_copy(uintptr_t dst, uintptr_t src, uint64_t bytes, hipStream_t stream) {
  const uint64_t nwords = bytes / sizeof(W);
  const uint32_t ntail = (uint32_t)(bytes - nwords * sizeof(W));
  const uint64_t grid = nwords ? (nwords + 255) / 256 : 1;
  hipLaunchKernelGGL(staging_copy<W>, dim3((uint32_t)grid), dim3(256), 0, stream,
                     reinterpret_cast<W *>(dst), reinterpret_cast<const W *>(src), nwords,
                     reinterpret_cast<uint8_t *>(dst + nwords * sizeof(W)),
                     reinterpret_cast<const uint8_t *>(src + nwords * sizeof(W)), ntail);
  return hipGetLastError();
}

} // namespace

using schedpd::set_error;

void *sched_pd_staging_alloc(uint64_t bytes) {
  if (bytes == 0 || bytes > kStagingMax) {
    set_error(hipErrorInvalidValue, "sched_pd_staging_alloc: %llu bytes (1 to %llu)",
              (unsigned long long)bytes, (unsigned long long)kStagingMax);
    return nullptr;
  }
  std::lock_guard<std::mutex> g(g_mu);
  if (g_nregions == kMaxRegions) {
    set_error(hipErrorOutOfMemory, "sched_pd_staging_alloc: %d regions already held", kMaxRegions);
    return nullptr;
  }
  void *h = nullptr;
  hipError_t e = hipHostMalloc(&h, bytes,
                               hipHostMallocMapped | hipHostMallocPortable | hipHostMallocCoherent);
  if (e != hipSuccess || h == nullptr) {
    set_error(e != hipSuccess ? e : hipErrorOutOfMemory, "sched_pd_staging_alloc: hipHostMalloc: %s",
              hipGetErrorString(e));
    return nullptr;
  }
  void *d = nullptr;
  e = hipHostGetDevicePointer(&d, h, 0);
  if (e != hipSuccess || d == nullptr) {
    (void)hipHostFree(h);          // never read by a kernel
    set_error(e != hipSuccess ? e : hipErrorInvalidValue,
              "sched_pd_staging_alloc: hipHostGetDevicePointer: %s", hipGetErrorString(e));
    return nullptr;
  }
  g_regions[g_nregions++] = Region{reinterpret_cast<uintptr_t>(h), reinterpret_cast<uintptr_t>(d),
                                   bytes};
  return h;
}

int sched_pd_copy_to_device(void *dst, const void *src, uint64_t bytes, void *stream) {
  if (bytes == 0)
    return 0;
  if (dst == nullptr || src == nullptr)
    return set_error(hipErrorInvalidValue, "sched_pd_copy_to_device: NULL pointer");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const uintptr_t dsrc = bytes <= kKernelCopyMax ? staged_device_address(src, bytes) : 0;
  hipError_t e;
  if (dsrc != 0 && fits_device_allocation(dst, bytes)) {
    const uintptr_t d = reinterpret_cast<uintptr_t>(dst);
    if (((d | dsrc) & 7u) == 0)
      e = launch_copy<uint64_t>(d, dsrc, bytes, s);
    else if (((d | dsrc) & 3u) == 0)
      e = launch_copy<uint32_t>(d, dsrc, bytes, s);
    else
      e = launch_copy<uint8_t>(d, dsrc, bytes, s);
  } else {
    e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s);
  }
  if (e != hipSuccess)
    return set_error(e, "sched_pd_copy_to_device: %s", hipGetErrorString(e));
  return 0;
}
