// sched_rt.hip -- the runtime contract of reference runtime/sched_rt.h, as an
// exported C library on HIP.
//
// Same tables, layout and call semantics as the reference (file:line per
// function). Differences, all deliberate:
//   * the timer rows live in device memory (the reference maps pinned host
//     memory; its own measurement puts host-mapped atomics at +26.5% against
//     -0.5% for a device buffer, ROADMAP.md:1482-1488), so sched_rt_timer()
//     is a small device-to-host copy instead of a plain host read;
//   * the functions are exported, not `static inline` in a header, so the
//     state is one per process (the library), not one per translation unit;
//   * an external reader that wants the rows with no GPU call turns on the
//     host mirror: a pinned copy refreshed by an async copy after each launch
//     that uses these tables, published as timer_host_va;
//   * the kernels read the table pointers from the __sched_* slots at every
//     launch, so slots written directly on the device take effect.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unistd.h>

#include "../../include/sched_pd.h"
#include "rt_internal.h"

// --- device-side slots (reference runtime/sched_rt.h:88-94) ---------------
extern "C" {
__device__ int32_t *__sched_task_order = nullptr;
__device__ SchedCtrl *__sched_ctrl = nullptr;
__device__ unsigned long long *__sched_timer = nullptr;
__device__ uint32_t *__sched_queue = nullptr;
}

namespace {

struct RtState {
  int32_t *d_order = nullptr;
  SchedCtrl *d_ctrl = nullptr;
  unsigned long long *d_timer = nullptr;
  uint32_t *d_queue = nullptr;
  SchedCtrl h_ctrl;
  bool armed = false;
  // opt-in pinned host copy of the timer rows for external readers
  unsigned long long *h_timer = nullptr;
  bool mirror = false;
  // caller-owned tables in the slots (sched_rt_bind_tables): their pointers
  // and row count; the runtime's own buffers stay allocated meanwhile
  bool bound = false;
  const int32_t *b_order = nullptr;
  const void *b_ctrl = nullptr;
  unsigned long long *b_timer = nullptr;
  uint32_t *b_queue = nullptr;
  uint32_t b_rows = 0;
};

RtState g_rt;
thread_local std::string g_err;

// /tmp/sched_rt_<pid>.json (reference runtime/sched_rt.h:170-186): the table
// addresses, plus timer_host_va, the host copy of the timer rows an external
// reader can consume with no GPU call (0 unless the mirror is on).
// While caller tables are bound, the file names them and their row count
// (and no host copy: the mirror follows the runtime's own rows only).
void publish() {
  const RtState &S = g_rt;
  const bool b = S.bound;
  const uint32_t rows = b ? S.b_rows : (uint32_t)SCHED_MAX_TASKS;
  char path[256];
  std::snprintf(path, sizeof path, "/tmp/sched_rt_%d.json", (int)getpid());
  if (FILE *f = std::fopen(path, "w")) {
    std::fprintf(f,
                 "{\"pid\":%d,\"max_tasks\":%u,\"order_dev\":%llu,\"ctrl_dev\":%llu,"
                 "\"timer_dev\":%llu,\"timer_host_va\":%llu,\"timer_bytes\":%zu,"
                 "\"queue_dev\":%llu,\"bound\":%d}\n",
                 (int)getpid(), rows,
                 (unsigned long long)(uintptr_t)(b ? (const void *)S.b_order : S.d_order),
                 (unsigned long long)(uintptr_t)(b ? S.b_ctrl : (const void *)S.d_ctrl),
                 (unsigned long long)(uintptr_t)(b ? S.b_timer : S.d_timer),
                 (unsigned long long)(uintptr_t)(S.mirror && !b ? S.h_timer : nullptr),
                 (size_t)rows * sizeof(unsigned long long),
                 (unsigned long long)(uintptr_t)(b ? S.b_queue : S.d_queue), b ? 1 : 0);
    std::fclose(f);
  }
}

bool rt_check(hipError_t e, const char *what) {
  if (e == hipSuccess)
    return true;
  char buf[512];
  std::snprintf(buf, sizeof buf, "[sched_rt] %s failed: %s", what, hipGetErrorString(e));
  schedpd::set_error_text(buf);
  return false;
}

#define RT_CHECK(call)                                                         \
  do {                                                                         \
    if (!rt_check((call), #call))                                              \
      return false;                                                            \
  } while (0)

bool write_slots(const int32_t *order, const void *ctrl, unsigned long long *timer,
                 uint32_t *queue) {
  RT_CHECK(hipMemcpyToSymbol(HIP_SYMBOL(__sched_task_order), &order, sizeof(void *)));
  RT_CHECK(hipMemcpyToSymbol(HIP_SYMBOL(__sched_ctrl), &ctrl, sizeof(void *)));
  RT_CHECK(hipMemcpyToSymbol(HIP_SYMBOL(__sched_timer), &timer, sizeof(void *)));
  RT_CHECK(hipMemcpyToSymbol(HIP_SYMBOL(__sched_queue), &queue, sizeof(void *)));
  return true;
}

} // namespace

namespace schedpd {

void set_error_text(const char *text) {
  g_err = text;
  std::fprintf(stderr, "%s\n", text);
}

int set_error(int code, const char *fmt, ...) {
  char buf[512];
  int n = std::snprintf(buf, sizeof buf, "[sched_pd] ");
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf + n, sizeof buf - n, fmt, ap);
  va_end(ap);
  set_error_text(buf);
  return code;
}

bool rt_slot_addresses(uint64_t out[4]) {
  constexpr int kMaxDev = 64;
  static uint64_t cache[kMaxDev][4];
  static bool have[kMaxDev];
  static std::mutex mu;
  int dev = 0;
  if (!rt_check(hipGetDevice(&dev), "hipGetDevice"))
    return false;
  if (dev < 0 || dev >= kMaxDev) {
    set_error_text("[sched_rt] device index beyond the runtime's table");
    return false;
  }
  // threads making their first launch on a device at once fill the entry
  // under the lock, so none reads it half written
  std::lock_guard<std::mutex> lock(mu);
  if (!have[dev]) {
    void *p[4] = {nullptr, nullptr, nullptr, nullptr};
    if (!rt_check(hipGetSymbolAddress(&p[0], HIP_SYMBOL(__sched_task_order)),
                  "hipGetSymbolAddress(__sched_task_order)") ||
        !rt_check(hipGetSymbolAddress(&p[1], HIP_SYMBOL(__sched_ctrl)),
                  "hipGetSymbolAddress(__sched_ctrl)") ||
        !rt_check(hipGetSymbolAddress(&p[2], HIP_SYMBOL(__sched_timer)),
                  "hipGetSymbolAddress(__sched_timer)") ||
        !rt_check(hipGetSymbolAddress(&p[3], HIP_SYMBOL(__sched_queue)),
                  "hipGetSymbolAddress(__sched_queue)"))
      return false;
    for (int i = 0; i < 4; ++i)
      cache[dev][i] = (uint64_t)(uintptr_t)p[i];
    have[dev] = true;
  }
  for (int i = 0; i < 4; ++i)
    out[i] = cache[dev][i];
  return true;
}

int rt_after_launch(void *stream) {
  if (!g_rt.mirror || g_rt.h_timer == nullptr || !g_rt.armed || g_rt.bound)
    return 0;
  hipError_t e = hipMemcpyAsync(g_rt.h_timer, g_rt.d_timer,
                                SCHED_MAX_TASKS * sizeof(unsigned long long),
                                hipMemcpyDeviceToHost, (hipStream_t)stream);
  if (e != hipSuccess)
    return set_error(e, "timer mirror copy failed: %s", hipGetErrorString(e));
  return 0;
}

RtSnapshot rt_snapshot() {
  RtSnapshot s{};
  s.armed = g_rt.armed || g_rt.bound;
  s.rows = SCHED_MAX_TASKS;
  s.num_tasks_known = true;
  if (g_rt.bound) {
    s.order = g_rt.b_order;
    s.ctrl = g_rt.b_ctrl;
    s.timer = g_rt.b_timer;
    s.queue = g_rt.b_queue;
    s.rows = g_rt.b_rows;
    s.num_tasks_known = false; // the tables' owner pushes num_tasks
  } else if (g_rt.armed) {
    s.order = g_rt.d_order;
    s.ctrl = g_rt.d_ctrl;
    s.timer = g_rt.d_timer;
    s.queue = g_rt.d_queue;
  }
  s.num_tasks = g_rt.h_ctrl.num_tasks;
  return s;
}

} // namespace schedpd

extern "C" {

const char *sched_pd_last_error(void) { return g_err.c_str(); }

// reference runtime/sched_rt.h:121-189
bool sched_rt_init(void) {
  RtState &S = g_rt;
  if (S.armed && !S.bound)
    return true;
  if (S.d_order == nullptr) {
    RT_CHECK(hipMalloc(&S.d_order, SCHED_MAX_TASKS * sizeof(int32_t)));
    int32_t *ident = (int32_t *)std::malloc(SCHED_MAX_TASKS * sizeof(int32_t));
    for (int i = 0; i < SCHED_MAX_TASKS; ++i)
      ident[i] = i;
    hipError_t e = hipMemcpy(S.d_order, ident, SCHED_MAX_TASKS * sizeof(int32_t),
                             hipMemcpyHostToDevice);
    std::free(ident);
    RT_CHECK(e);
    // Neutral policy: lambda = 0, q = 0 -> score = -H < 0 -> stock action.
    std::memset(&S.h_ctrl, 0, sizeof(SchedCtrl));
    RT_CHECK(hipMalloc(&S.d_ctrl, sizeof(SchedCtrl)));
    RT_CHECK(hipMemcpy(S.d_ctrl, &S.h_ctrl, sizeof(SchedCtrl), hipMemcpyHostToDevice));
    RT_CHECK(hipMalloc(&S.d_timer, SCHED_MAX_TASKS * sizeof(unsigned long long)));
    RT_CHECK(hipMemset(S.d_timer, 0, SCHED_MAX_TASKS * sizeof(unsigned long long)));
    RT_CHECK(hipMalloc(&S.d_queue, sizeof(uint32_t)));
    RT_CHECK(hipMemset(S.d_queue, 0, sizeof(uint32_t)));
  }
  if (!write_slots(S.d_order, S.d_ctrl, S.d_timer, S.d_queue))
    return false;
  S.bound = false;
  S.armed = true;
  publish();
  return true;
}

// reference runtime/sched_rt.h:192-203
bool sched_rt_disarm(void) {
  if (!write_slots(nullptr, nullptr, nullptr, nullptr))
    return false;
  g_rt.armed = false;
  g_rt.bound = false;
  return true;
}

// No counterpart in the reference, whose Python plane bakes its table
// addresses into a JIT-compiled kernel (python/sched_rt.py:489-555): here
// the plane's tables go into the slots the launchers read at every launch.
bool sched_rt_bind_tables(const int32_t *order, const void *ctrl, unsigned long long *timer,
                          uint32_t *queue, uint32_t max_tasks) {
  if (max_tasks > SCHED_RT_BIND_MAX_TASKS) {
    char buf[160];
    std::snprintf(buf, sizeof buf,
                  "[sched_rt] sched_rt_bind_tables failed: max_tasks %u > %u", max_tasks,
                  (unsigned)SCHED_RT_BIND_MAX_TASKS);
    schedpd::set_error_text(buf);
    return false;
  }
  if (!write_slots(order, ctrl, timer, queue))
    return false;
  RtState &S = g_rt;
  S.b_order = order;
  S.b_ctrl = ctrl;
  S.b_timer = timer;
  S.b_queue = queue;
  S.b_rows = max_tasks;
  S.bound = true;
  S.armed = false;
  publish();
  return true;
}

// reference runtime/sched_rt.h:206-212
bool sched_rt_set_order(const int32_t *order, unsigned n) {
  if (g_rt.d_order == nullptr) {
    schedpd::set_error_text("[sched_rt] sched_rt_set_order failed: runtime not initialised");
    return false;
  }
  if (n > SCHED_MAX_TASKS)
    n = SCHED_MAX_TASKS;
  RT_CHECK(hipMemcpy(g_rt.d_order, order, n * sizeof(int32_t), hipMemcpyHostToDevice));
  return true;
}

// reference runtime/sched_rt.h:214-249
void sched_rt_set_lambda(float bw, float l2, float smem, float comp) {
  g_rt.h_ctrl.lambda[0] = bw;
  g_rt.h_ctrl.lambda[1] = l2;
  g_rt.h_ctrl.lambda[2] = smem;
  g_rt.h_ctrl.lambda[3] = comp;
}
void sched_rt_set_task(unsigned i, float q, uint16_t tau, uint8_t hint) {
  if (i >= SCHED_MAX_TASKS)
    return;
  g_rt.h_ctrl.task[i].q = q;
  g_rt.h_ctrl.task[i].tau = tau;
  g_rt.h_ctrl.task[i].hint = hint;
  g_rt.h_ctrl.task[i]._pad = 0;
}
void sched_rt_set_tau(unsigned i, uint16_t tau) {
  if (i < SCHED_MAX_TASKS)
    g_rt.h_ctrl.task[i].tau = tau;
}
void sched_rt_set_num_tasks(uint32_t n) { g_rt.h_ctrl.num_tasks = n; }
void sched_rt_set_order_size(uint32_t n) { g_rt.h_ctrl.order_size = n; }
void sched_rt_set_timer_enabled(bool on) {
  if (on)
    g_rt.h_ctrl.flags &= ~SCHED_CTRL_FLAG_TIMER_OFF;
  else
    g_rt.h_ctrl.flags |= SCHED_CTRL_FLAG_TIMER_OFF;
}

// reference runtime/sched_rt.h:252-257
bool sched_rt_push_ctrl(void) {
  if (g_rt.d_ctrl == nullptr) {
    schedpd::set_error_text("[sched_rt] sched_rt_push_ctrl failed: runtime not initialised");
    return false;
  }
  g_rt.h_ctrl.generation++;
  RT_CHECK(hipMemcpy(g_rt.d_ctrl, &g_rt.h_ctrl, sizeof(SchedCtrl), hipMemcpyHostToDevice));
  return true;
}

// reference runtime/sched_rt.h:261-265
bool sched_rt_queue_reset(uint32_t workers) {
  if (g_rt.d_queue == nullptr) {
    schedpd::set_error_text("[sched_rt] sched_rt_queue_reset failed: runtime not initialised");
    return false;
  }
  RT_CHECK(hipMemcpy(g_rt.d_queue, &workers, sizeof(uint32_t), hipMemcpyHostToDevice));
  return true;
}

// reference runtime/sched_rt.h:267-275
unsigned long long sched_rt_timer(unsigned i) {
  if (i >= SCHED_MAX_TASKS || g_rt.d_timer == nullptr)
    return 0ull;
  unsigned long long v = 0;
  if (!rt_check(hipMemcpy(&v, g_rt.d_timer + i, sizeof v, hipMemcpyDeviceToHost),
                "hipMemcpy(timer row)"))
    return 0ull;
  return v;
}
void sched_rt_timer_clear(void) {
  if (g_rt.d_timer)
    rt_check(hipMemset(g_rt.d_timer, 0, SCHED_MAX_TASKS * sizeof(unsigned long long)),
             "hipMemset(timer)");
  if (g_rt.h_timer)
    std::memset(g_rt.h_timer, 0, SCHED_MAX_TASKS * sizeof(unsigned long long));
}

bool sched_rt_set_timer_host_mirror(bool on) {
  RtState &S = g_rt;
  if (on && S.h_timer == nullptr) {
    void *p = nullptr;
    RT_CHECK(hipHostMalloc(&p, SCHED_MAX_TASKS * sizeof(unsigned long long),
                           hipHostMallocDefault));
    S.h_timer = static_cast<unsigned long long *>(p);
    std::memset(S.h_timer, 0, SCHED_MAX_TASKS * sizeof(unsigned long long));
  }
  S.mirror = on;
  if (S.armed)
    publish();
  return true;
}

bool sched_rt_slot_addresses(uint64_t addrs[4]) {
  if (addrs == nullptr) {
    schedpd::set_error_text("[sched_rt] sched_rt_slot_addresses failed: addrs is NULL");
    return false;
  }
  return schedpd::rt_slot_addresses(addrs);
}

uint64_t sched_rt_timer_host_va(void) {
  return g_rt.mirror ? (uint64_t)(uintptr_t)g_rt.h_timer : 0u;
}

bool sched_rt_timer_read(unsigned long long *dst, unsigned n) {
  if (g_rt.d_timer == nullptr || dst == nullptr) {
    schedpd::set_error_text("[sched_rt] sched_rt_timer_read failed: runtime not initialised");
    return false;
  }
  if (n > SCHED_MAX_TASKS)
    n = SCHED_MAX_TASKS;
  RT_CHECK(hipMemcpy(dst, g_rt.d_timer, n * sizeof(unsigned long long), hipMemcpyDeviceToHost));
  return true;
}

bool sched_rt_slots(uint64_t slots[4]) {
  void *p[4] = {nullptr, nullptr, nullptr, nullptr};
  RT_CHECK(hipMemcpyFromSymbol(&p[0], HIP_SYMBOL(__sched_task_order), sizeof(void *)));
  RT_CHECK(hipMemcpyFromSymbol(&p[1], HIP_SYMBOL(__sched_ctrl), sizeof(void *)));
  RT_CHECK(hipMemcpyFromSymbol(&p[2], HIP_SYMBOL(__sched_timer), sizeof(void *)));
  RT_CHECK(hipMemcpyFromSymbol(&p[3], HIP_SYMBOL(__sched_queue), sizeof(void *)));
  for (int i = 0; i < 4; ++i)
    slots[i] = (uint64_t)(uintptr_t)p[i];
  return true;
}

} // extern "C"
