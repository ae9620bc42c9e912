// rt_internal.h -- what the launcher needs from the C runtime: the tables the
// __sched_* slots point at right now, and error reporting shared by both
// translation units.
#pragma once

#include <stdint.h>

namespace schedpd {

struct RtSnapshot {
  const int32_t *order;
  const void *ctrl;
  unsigned long long *timer;
  uint32_t *queue;
  uint32_t num_tasks;   // host mirror of ctrl.num_tasks as last pushed
  uint32_t rows;        // rows of order / ctrl / timer (the kernels' task bound)
  bool num_tasks_known; // false while caller tables are bound (their owner pushes it)
  bool armed;           // the slots hold tables (the runtime's own or bound ones)
};

RtSnapshot rt_snapshot();

// Device addresses of the four __sched_* slots (order, ctrl, timer, queue) on
// the current device; false (with the error recorded) if they cannot be had.
bool rt_slot_addresses(uint64_t out[4]);

// The runtime's host mirror of the timer rows, if enabled: enqueue its refresh
// on `stream` after a launch that used the runtime's tables.
int rt_after_launch(void *stream);

// Record and print an error ("[sched_pd] ..."); returns `code`.
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void set_error_text(const char *text);

} // namespace schedpd
