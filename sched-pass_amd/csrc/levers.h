// levers.h -- device side of the five scheduling levers, hand-written for
// gfx950 (one workgroup = one task at a time, wave64).
//
// Each lever reads the table pointers in LeverTables; a NULL pointer is that
// lever's stock behaviour. The decisions follow the reference weave exactly
// (file:line of the reference cited per function); only the mechanism is
// native (no IR weaving: the kernels call these helpers directly).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sched_pd.h"

namespace schedpd {

struct LeverTables {
  const int32_t *order;      // pi
  const uint8_t *ctrl;       // SchedCtrl bytes
  unsigned long long *timer; // residency rows
  uint32_t *queue;           // ticket counter
  uint32_t max_tasks;        // rows in order/ctrl/timer
  uint32_t nitems;           // work items of this launch (static grid size)
  uint32_t wq;               // 1 = launched as W persistent workers
  uint32_t workers;          // W of a work-queue launch (per-wave kernels)
  uint32_t spread;           // per-wave kernels, static grid: workgroups resident at once
                             // (0 or 1: positions row-major, wave-minor)
  uint32_t wallclock;        // timer source: 1 = s_memrealtime, 0 = s_memtime
  float dT, dR, H;           // policy marginal-exchange constants
  // Runtime mode (SCHED_PD_FLAG_RT_TABLES): the device addresses of the four
  // __sched_* slots; the kernel reads the table pointers they hold (lt_order,
  // lt_ctrl, lt_timer, lt_queue), so a slot written directly on the device
  // takes effect at the next launch.
  uint64_t rt_slot[4];
  uint32_t rt;
};

struct TaskPolicy {
  bool urgent;
  bool polite;
  uint32_t budget; // tokens; 0xFFFFFFFF = no cap
};

// The table pointers a kernel uses: the launch's own, or (runtime mode) the
// ones the __sched_* slots hold, read with a scalar load at each use (no
// kernel writes the slots, so every read of a launch sees the same pointer,
// and the loads hit the scalar cache).
typedef const __attribute__((address_space(4))) uint64_t slot_u64;
// A 64-bit value every lane holds alike, kept wave-uniform for the compiler
// (so what is derived from it stays in scalar registers).
__device__ __forceinline__ uint64_t uniform_u64(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t slot_or(const LeverTables &L, int k, const void *own) {
  return L.rt ? uniform_u64(*(slot_u64 *)L.rt_slot[k]) : (uint64_t)(uintptr_t)own;
}
__device__ __forceinline__ const int32_t *lt_order(const LeverTables &L) {
  return reinterpret_cast<const int32_t *>(slot_or(L, 0, L.order));
}
__device__ __forceinline__ const uint8_t *lt_ctrl(const LeverTables &L) {
  return reinterpret_cast<const uint8_t *>(slot_or(L, 1, L.ctrl));
}
__device__ __forceinline__ unsigned long long *lt_timer(const LeverTables &L) {
  return reinterpret_cast<unsigned long long *>(slot_or(L, 2, L.timer));
}
__device__ __forceinline__ uint32_t *lt_queue(const LeverTables &L) {
  return reinterpret_cast<uint32_t *>(slot_or(L, 3, L.queue));
}

// Fields of the control block and entries of pi: the same for every lane of a
// workgroup (task-uniform), kept in scalar registers (the tables may come from
// loaded slot pointers, where the compiler could not otherwise tell).
__device__ __forceinline__ uint32_t ld_u32(const uint8_t *p) {
  return __builtin_amdgcn_readfirstlane(*reinterpret_cast<const uint32_t *>(p));
}
__device__ __forceinline__ float ld_f32(const uint8_t *p) {
  return __uint_as_float(ld_u32(p));
}

__device__ __forceinline__ unsigned long long read_clock(uint32_t wallclock) {
  return wallclock ? __builtin_amdgcn_s_memrealtime() : __builtin_amdgcn_s_memtime();
}

// pi on the static grid (reference lib/SchedWeave.cpp:444-526):
//   task = order[pid] if order is armed, pid < max, order[pid] < nctaid and
//   ctrl.order_size in {0, nctaid} (ctrl unarmed = unchecked); else pid.
__device__ __forceinline__ uint32_t remap_static(const LeverTables &L, uint32_t pid,
                                                 uint32_t nctaid) {
  const int32_t *order = lt_order(L);
  if (order == nullptr || pid >= L.max_tasks)
    return pid;
  uint32_t mapped = __builtin_amdgcn_readfirstlane((uint32_t)order[pid]);
  bool size_ok = true;
  if (const uint8_t *ctrl = lt_ctrl(L)) {
    uint32_t osz = ld_u32(ctrl + SCHED_CTRL_ORDER_SIZE_OFF);
    size_ok = (osz == 0u) || (osz == nctaid);
  }
  return (mapped < nctaid && size_ok) ? mapped : pid;
}

// pi inside the work-queue loop (reference lib/SchedWorkQueue.cpp:305-343):
// bounded by num_tasks (this claim wave's range) with order_size in
// {0, num_tasks}. ctrl is armed on this path (the driver checked it).
__device__ __forceinline__ uint32_t remap_wq(const LeverTables &L, uint32_t raw,
                                             uint32_t num_tasks) {
  const int32_t *order = lt_order(L);
  if (order == nullptr || raw >= L.max_tasks)
    return raw;
  uint32_t mapped = __builtin_amdgcn_readfirstlane((uint32_t)order[raw]);
  uint32_t osz = ld_u32(lt_ctrl(L) + SCHED_CTRL_ORDER_SIZE_OFF);
  bool ok = mapped < num_tasks && (osz == 0u || osz == num_tasks);
  return ok ? mapped : raw;
}

// Policy flags and shed budget of one task (reference lib/SchedWeave.cpp:
// 532-581 and :585-614). Task-uniform: every lane computes the same values
// from scalar loads.
__device__ __forceinline__ TaskPolicy task_policy(const LeverTables &L, uint32_t task) {
  TaskPolicy P{false, false, 0xFFFFFFFFu};
  const uint8_t *ctrl = lt_ctrl(L);
  if (ctrl == nullptr || task >= L.max_tasks)
    return P;
  const uint8_t *row = ctrl + SCHED_CTRL_ROWS_OFF + (size_t)task * SCHED_CTRL_ROW_SIZE;
  float lam = ld_f32(ctrl + SCHED_CTRL_LAMBDA_OFF);
  float q = ld_f32(row);
  uint32_t w1 = ld_u32(row + 4); // tau (u16) | hint (u8) << 16
  uint32_t tau = w1 & 0xFFFFu;
  uint32_t hint = (w1 >> 16) & 0xFFu;
  float score = (q * L.dT - lam * L.dR) - L.H;
  P.urgent = hint == SCHED_HINT_URGENT || (hint == SCHED_HINT_AUTO && score > 0.f);
  P.polite = hint == SCHED_HINT_POLITE;
  P.budget = tau ? tau : 0xFFFFFFFFu;
  return P;
}

// Timer-off gate latched at kernel entry (reference lib/SchedWeave.cpp:
// 346-356, 979-1002): ctrl unarmed -> timer on.
__device__ __forceinline__ bool timer_off_latched(const LeverTables &L) {
  const uint8_t *ctrl = lt_ctrl(L);
  return ctrl != nullptr && (ld_u32(ctrl + SCHED_CTRL_FLAGS_OFF) & SCHED_CTRL_FLAG_TIMER_OFF);
}

// Epilogue of one task body (reference lib/SchedWeave.cpp:1004-1049): lane 0
// of the workgroup adds the residency delta into timer[task], relaxed, device
// scope; rows accumulate until cleared.
__device__ __forceinline__ void timer_commit(const LeverTables &L, bool off, uint32_t task,
                                             unsigned long long t0) {
  unsigned long long *timer = lt_timer(L);
  if (threadIdx.x == 0 && timer != nullptr && task < L.max_tasks && !off) {
    unsigned long long dt = read_clock(L.wallclock) - t0;
    __hip_atomic_fetch_add(timer + task, dt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Task acquisition: the static grid or the ticket work queue (reference
// lib/SchedWorkQueue.cpp:345-448). `body(task)` runs one task with the whole
// workgroup and must end with every thread past its last LDS use.
//
// Static launch (wq == 0): one task per workgroup, task = remap_static(ctaid)
// with the launch's item count as the grid bound (the host launches one
// workgroup per item).
// The body gets the item and whether it is a queue worker's last (the
// launch's run-down).
// Work-queue launch (wq == 1, grid = W workers):
//   stock path if queue or ctrl is NULL, the grid is not 1-D, or num_tasks==0;
//   otherwise raw = ctaid (exit if >= num_tasks), then loop: body(remap(raw)),
//   barrier, lane 0 claims raw = atomicAdd(queue, 1), barrier, until
//   raw >= num_tasks. The claim comes after the body (late binding).
// On the stock path pi stays live with the static-grid bound (the reference's
// stated intent, test/hetero_batch.cu:220-225; its num_tasks-bounded remap
// there degrades to identity, which changes no output).
// The worker that takes the launch's last ticket (W + num_tasks - 1) stores W
// back into the counter: every other worker has already made its last claim,
// so the next launch with the same W needs no host-side reset.
// Claim rounds at the end of a queue launch whose items the body is told
// are late (the MFMA kernel streams them with its deep ring): measured on
// the heterogeneous, shed and fp8 queue launches, 1 is best (2 and 3 slow
// the fp8 and shed launches by 2-6%).
#ifndef SCHED_PD_LATE_ROUNDS
#define SCHED_PD_LATE_ROUNDS 1u
#endif
template <class Body>
__device__ __forceinline__ void run_tasks(const LeverTables &L, Body &&body) {
  const uint32_t pid = blockIdx.x;
  uint32_t ntasks = 0u;
  if (L.wq) {
    const bool grid1d = gridDim.y == 1 && gridDim.z == 1;
    const bool armed = lt_queue(L) != nullptr && lt_ctrl(L) != nullptr && grid1d;
    ntasks = armed ? ld_u32(lt_ctrl(L) + SCHED_CTRL_NUM_TASKS_OFF) : 0u;
  }
  const bool queue = ntasks != 0u;
  if (queue && pid >= ntasks)
    return;
  __shared__ uint32_t s_next;
  const uint32_t last_ticket = gridDim.x + ntasks - 1u;
  // Static grid (or the stock path of a queue launch): items pid, pid + grid,
  // ... -- one per workgroup when the grid covers the items, as it does for
  // a static launch; a queue grid whose tables were disarmed on the device
  // still covers every item.
  uint32_t raw = pid;
  // One call site of the body (it is large: inlining it once keeps the
  // kernel's code and register allocation that of a single task body).
  while (true) {
    if (!queue && raw >= L.nitems)
      return;
    // the item is the same on every lane: keep it (and the addresses derived
    // from it) in scalar registers
    // a queue worker's last item (fewer tickets left than workers, on a
    // launch of at least twice as many items as workers, so that most items
    // stream in full rounds): the launch's run-down, where the item streams
    // with fewer and fewer others beside it
    const bool last_round = queue && ntasks >= 2u * gridDim.x &&
                            raw + SCHED_PD_LATE_ROUNDS * gridDim.x >= ntasks;
    body(__builtin_amdgcn_readfirstlane(queue ? remap_wq(L, raw, ntasks)
                                              : remap_static(L, raw, L.nitems)),
         last_round);
    if (!queue) {
      raw += gridDim.x;
      if (raw < L.nitems)
        __syncthreads();
      continue;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t t = __hip_atomic_fetch_add(lt_queue(L), 1u, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
      if (t == last_ticket)
        __hip_atomic_store(lt_queue(L), gridDim.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_next = t;
    }
    __syncthreads();
    raw = __builtin_amdgcn_readfirstlane(s_next);
    if (raw >= ntasks)
      return;
  }
}

} // namespace schedpd
