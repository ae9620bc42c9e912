/* sched_pd.h -- C ABI of the MI355X (gfx950) paged-KV decode hot path with the
 * sched-pass scheduling levers built into hand-written HIP kernels.
 *
 * Three groups of entry points, all plain C (no HIP or torch types):
 *
 *   1. The runtime contract of reference runtime/sched_rt.h:54-275: the
 *      SchedPolicyRow / SchedCtrl layout with its pinned offsets, and the
 *      sched_rt_* host API (init/arm, disarm, setters, push, queue reset,
 *      timer read/clear). The reference defines these `static inline` in a
 *      header; here they are exported from libschedpd.so.
 *   2. The decode launcher: sched_paged_decode(const SchedDecodeArgs*, stream).
 *      One call runs one decode step over a paged batch, with the five levers
 *      (pi, policy/prefetch, shed, timer, ticket work queue) read from the
 *      table pointers in the argument block. A NULL table is the stock path.
 *   3. The reference's JIT-kernel launcher, same name and signature:
 *      launch_paged_softmax (reference python/kernels/paged_softmax.cu:47-54)
 *      and paged_softmax_occupancy (:61-67).
 *
 * Errors: entry points that return int return 0 on success and a nonzero
 * hipError_t code on failure; entry points returning bool return false. In
 * both cases a line "[sched_rt] <call> failed: <reason>" or
 * "[sched_pd] <reason>" goes to stderr, and sched_pd_last_error() returns the
 * same text. Nothing aborts.
 */
#ifndef SCHED_PD_H
#define SCHED_PD_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- 1. runtime contract (reference runtime/sched_rt.h) ------------------ */

/* Rows in the order / ctrl / timer tables of the C runtime. Same knob and
 * default as reference runtime/sched_rt.h:50-52. */
#ifndef SCHED_MAX_TASKS
#define SCHED_MAX_TASKS 4096
#endif

/* Per-task policy row, 8 bytes (reference runtime/sched_rt.h:54-59). */
typedef struct SchedPolicyRow {
  float q;        /* urgency, >= 0 */
  uint16_t tau;   /* shed budget in tokens (0 = unbounded) */
  uint8_t hint;   /* SCHED_HINT_* */
  uint8_t _pad;
} SchedPolicyRow;

/* Per-step control block (reference runtime/sched_rt.h:61-74). The kernels
 * read num_tasks, lambda[0], flags, order_size and the rows; generation is
 * written by push and read by no kernel. */
typedef struct SchedCtrl {
  uint32_t generation;
  uint32_t num_tasks;   /* work-queue bound; 0 = stock static path */
  float lambda[4];      /* shadow prices {bw, l2, smem, comp}; kernels read [0] */
  uint32_t flags;       /* bit0 = SCHED_CTRL_FLAG_TIMER_OFF */
  uint32_t order_size;  /* task count the installed pi was built for; 0 = unchecked */
  SchedPolicyRow task[SCHED_MAX_TASKS];
} SchedCtrl;

#define SCHED_CTRL_FLAG_TIMER_OFF 1u

/* Byte offsets (reference lib/SchedUtil.h:96-123, python/sched_rt.py:52-61). */
#define SCHED_CTRL_NUM_TASKS_OFF 4
#define SCHED_CTRL_LAMBDA_OFF 8
#define SCHED_CTRL_FLAGS_OFF 24
#define SCHED_CTRL_ORDER_SIZE_OFF 28
#define SCHED_CTRL_ROWS_OFF 32
#define SCHED_CTRL_ROW_SIZE 8
#define SCHED_CTRL_ROW_TAU_OFF 4
#define SCHED_CTRL_ROW_HINT_OFF 6

/* Hints (reference lib/SchedUtil.h:119-122). */
#define SCHED_HINT_AUTO 0   /* urgent iff q*dT - lambda_bw*dR - H > 0 */
#define SCHED_HINT_URGENT 1 /* deeper KV prefetch ring (pf_dist pages in flight) */
#define SCHED_HINT_POLITE 2 /* non-temporal KV loads always; stock tasks load the
                               same way except items longer than 256 pages, which
                               stream with ordinary loads on the deepest ring */

#ifdef __cplusplus
static_assert(offsetof(SchedCtrl, num_tasks) == SCHED_CTRL_NUM_TASKS_OFF, "sched ABI: num_tasks");
static_assert(offsetof(SchedCtrl, lambda) == SCHED_CTRL_LAMBDA_OFF, "sched ABI: lambda");
static_assert(offsetof(SchedCtrl, flags) == SCHED_CTRL_FLAGS_OFF, "sched ABI: flags");
static_assert(offsetof(SchedCtrl, order_size) == SCHED_CTRL_ORDER_SIZE_OFF, "sched ABI: order_size");
static_assert(offsetof(SchedCtrl, task) == SCHED_CTRL_ROWS_OFF, "sched ABI: rows offset");
static_assert(sizeof(SchedPolicyRow) == SCHED_CTRL_ROW_SIZE, "sched ABI: row size");
static_assert(offsetof(SchedPolicyRow, tau) == SCHED_CTRL_ROW_TAU_OFF, "sched ABI: row tau");
static_assert(offsetof(SchedPolicyRow, hint) == SCHED_CTRL_ROW_HINT_OFF, "sched ABI: row hint");
#endif

/* Replaces reference runtime/sched_rt.h:121-189 (sched_rt_init): allocate the
 * tables once (identity pi, neutral ctrl, zeroed device-memory timer, queue),
 * arm the __sched_* device slots, publish /tmp/sched_rt_<pid>.json.
 * Idempotent; re-arming after disarm reuses the buffers. */
bool sched_rt_init(void);
/* runtime/sched_rt.h:192-203: null the slots, keep the buffers. */
bool sched_rt_disarm(void);
/* runtime/sched_rt.h:206-212: write order[0..n) (n clamped to the table size),
 * synchronously. */
bool sched_rt_set_order(const int32_t *order, unsigned n);
/* runtime/sched_rt.h:214-249: host-mirror setters; effective at the next push. */
void sched_rt_set_lambda(float bw, float l2, float smem, float comp);
void sched_rt_set_task(unsigned i, float q, uint16_t tau, uint8_t hint);
void sched_rt_set_tau(unsigned i, uint16_t tau);
void sched_rt_set_num_tasks(uint32_t n);
void sched_rt_set_order_size(uint32_t n);
void sched_rt_set_timer_enabled(bool on);
/* runtime/sched_rt.h:252-257: generation++, then copy the whole struct. */
bool sched_rt_push_ctrl(void);
/* runtime/sched_rt.h:261-265: prime the ticket counter to `workers`. */
bool sched_rt_queue_reset(uint32_t workers);
/* runtime/sched_rt.h:267-275: timer row read / clear. The rows live in device
 * memory, so these synchronise with the device. */
unsigned long long sched_rt_timer(unsigned i);
void sched_rt_timer_clear(void);

/* Rows a caller's tables may hold for sched_rt_bind_tables: the reference
 * plane's per-table window (python/sched_rt.py:89). */
#define SCHED_RT_BIND_MAX_TASKS 16384

/* Point the four __sched_* slots at caller-owned device tables instead of the
 * runtime's own, no counterpart in the reference: its Python plane
 * (python/sched_rt.py:489-555) bakes the addresses of its arena into a
 * JIT-compiled kernel, so that kernel's levers follow the plane. Here the
 * launchers that take their levers from the slots (launch_paged_softmax, and
 * sched_paged_decode with SCHED_PD_FLAG_RT_TABLES) then run with these
 * tables: order i32[max_tasks], ctrl in the SchedCtrl layout with max_tasks
 * rows, timer u64[max_tasks], queue one u32. Any pointer may be NULL (that
 * lever's stock behaviour). Task ids >= max_tasks (at most
 * SCHED_RT_BIND_MAX_TASKS) get no levers. The tables' owner writes them
 * (e.g. SchedPlane.push): the sched_rt_set_* / push / timer calls keep
 * working on the runtime's own tables, which stay allocated. A queue launch
 * over bound tables starts `workers` workgroups whatever num_tasks the owner
 * pushed (the kernels take the stock path when it is 0). sched_rt_init()
 * puts the runtime's own tables back, sched_rt_disarm() nulls the slots.
 * Synchronous; returns false on error. */
bool sched_rt_bind_tables(const int32_t *order, const void *ctrl, unsigned long long *timer,
                          uint32_t *queue, uint32_t max_tasks);

/* Introspection, no counterpart in the reference (its tables are static
 * globals of the including translation unit): the device addresses the
 * __sched_* slots hold right now (0 when disarmed), read back from the device
 * symbols. slots[0..3] = order, ctrl, timer, queue. Returns false on error. */
bool sched_rt_slots(uint64_t slots[4]);
/* Device addresses of the __sched_* slots themselves (addrs[0..3] = order,
 * ctrl, timer, queue), no counterpart in the reference: its slots are symbols
 * of the including translation unit, written with cudaMemcpyToSymbol; here
 * they live in the library's code object, so a caller that writes a slot
 * directly copies the 8-byte table pointer to this address (hipMemcpy). The
 * kernels read the slots at every launch with SCHED_PD_FLAG_RT_TABLES.
 * Returns false on error. */
bool sched_rt_slot_addresses(uint64_t addrs[4]);
/* Bulk timer read, no counterpart in the reference (its rows are host-mapped
 * and read in place): copies rows [0, n) (n clamped) into dst. */
bool sched_rt_timer_read(unsigned long long *dst, unsigned n);
/* The reference's host-mapped timer readout (runtime/sched_rt.h:150-156,
 * :178-181), opt-in: on = keep a pinned host copy of the timer rows, refreshed
 * by an async device-to-host copy on the launch's stream after every
 * sched_paged_decode launch with SCHED_PD_FLAG_RT_TABLES, and publish its
 * address as timer_host_va in /tmp/sched_rt_<pid>.json, so a separate process
 * can read the rows with no GPU call (they trail the device rows by the copy).
 * The kernels add into device memory either way. Off by default. */
bool sched_rt_set_timer_host_mirror(bool on);
/* Address of the host copy of the timer rows (0 while the mirror is off). */
uint64_t sched_rt_timer_host_va(void);

/* ---- 2. decode launcher --------------------------------------------------- */

#define SCHED_PD_ABI_VERSION 1u

/* mode */
#define SCHED_PD_SOFTMAX 0u /* out[r][hq][:] = softmax(scale*q.K^T) V   (online softmax) */
#define SCHED_PD_LINEAR 1u  /* out[r][hkv][:] = sum_t w[t] V[t]         (linear contraction) */

/* dtypes */
#define SCHED_PD_F32 0u
#define SCHED_PD_BF16 1u
#define SCHED_PD_FP8_E4M3 2u /* OCP e4m3fn, per-(page, kv-head) fp32 scales */
#define SCHED_PD_F16 3u      /* IEEE binary16 (FlashInfer's fp16 caches, Q, output) */

/* tau scope: prefix = the first tau tokens of the request; per_page = the first
 * tau tokens of every page, the counter of the reference fixtures' woven
 * innermost loop (test/paged_decode.cu:103,136) */
#define SCHED_PD_TAU_PREFIX 0u
#define SCHED_PD_TAU_PER_PAGE 1u

/* split-KV tile row formats (tile_format) */
#define SCHED_PD_TILES_PAIRS 0u  /* (task, chunk); chunks of tile_pages pages */
#define SCHED_PD_TILES_RANGED 1u /* (task, chunk | nchunks << 16, p0, p1) */

/* flags */
#define SCHED_PD_FLAG_RT_TABLES 0x1u    /* take order/ctrl/timer/queue from the C runtime's
                                           __sched_* slots: the kernel reads the pointers the
                                           device slots hold when it starts; whether a queue
                                           grid of `workers` is launched follows what
                                           sched_rt_* last armed and pushed */
#define SCHED_PD_FLAG_WALLCLOCK 0x2u    /* timer counts s_memrealtime (100 MHz) instead of s_memtime */
#define SCHED_PD_FLAG_FORCE_VALU 0x4u   /* use the general VALU kernel (one workgroup per
                                           work item) even where another kernel applies */
#define SCHED_PD_FLAG_CTX_IN_PAGES 0x8u /* ctx_lens counts full pages, not tokens */
#define SCHED_PD_FLAG_SHED_LOADS 0x10u  /* load shed tokens and mask them (reference weave,
                                           lib/SchedWeave.cpp:646-651) instead of skipping
                                           the pages past a prefix budget; same output */
#define SCHED_PD_FLAG_NO_WAVE 0x20u     /* do not use the one-wave-per-item kernel (G <= 3):
                                           take the MFMA kernel where it applies, else the
                                           general VALU kernel */
#define SCHED_PD_FLAG_NO_MFMA 0x40u     /* do not use the MFMA kernel: the one-wave-per-item
                                           kernel where it applies, else the VALU kernel */

/* One decode step. Element (page, kv-head h, token t, dim j) of the pools:
 *   K: k_pool + page*k_page_stride + h*k_head_stride + t*k_tok_stride + j
 *   V: v_pool + page*v_page_stride + h*v_head_stride + t*v_tok_stride + j*v_dim_stride
 * (strides in elements). Request r's page b is block_table[r*bt_stride + b],
 * or block_table[page_indptr[r] + b] when page_indptr is not NULL. Page
 * ids are not bounds-checked on the device (as in the reference's kernels):
 * every page a request's context reaches must lie in the pools (the Python
 * layer's check_tables verifies this on the host).
 * Task id = r*num_kv_heads + h; the lever tables are indexed by task. */
typedef struct SchedDecodeArgs {
  uint32_t abi_version; /* SCHED_PD_ABI_VERSION */
  uint32_t mode;
  uint32_t kv_dtype;    /* F32, BF16, F16 or FP8_E4M3 */
  uint32_t q_dtype;     /* F32, BF16 or F16 (softmax mode) */
  uint32_t o_dtype;     /* F32, BF16 or F16 */
  uint32_t num_requests;
  uint32_t num_q_heads;  /* softmax: multiple of num_kv_heads */
  uint32_t num_kv_heads;
  uint32_t head_dim;     /* 32, 64 or 128 */
  uint32_t page_size;    /* tokens per page, multiple of 16, <= 256 */
  uint32_t bt_stride;
  uint32_t tau_scope;
  uint32_t workers;      /* 0 = static grid (one workgroup per task); W = ticket queue */
  uint32_t pf_dist;      /* pages of loads an urgent task's waves keep in flight: 0 = the
                            selected kernel's deepest ring, else a depth it serves
                            (sched_paged_decode_prefetch_range; other values are
                            rejected with hipErrorInvalidValue) */
  uint32_t flags;
  uint32_t max_tasks;    /* rows of order/ctrl/timer; task ids >= max_tasks get no levers */
  float sm_scale;        /* 0 = 1/sqrt(head_dim) */
  float policy_dT, policy_dR, policy_H; /* urgent iff q*dT - lambda_bw*dR - H > 0 */
  uint32_t lin_w_period; /* linear mode: w index = pos % period (0 = pos) */
  uint32_t tile_pages;   /* split-KV tile size in pages (pair rows, see tiles) */
  const void *q;         /* [num_requests][num_q_heads][head_dim] */
  void *out;             /* softmax: [R][Hq][d]; linear: [R][Hkv][d] */
  const void *k_pool;
  const void *v_pool;
  int64_t k_page_stride, k_head_stride, k_tok_stride;
  int64_t v_page_stride, v_head_stride, v_tok_stride, v_dim_stride;
  const float *k_scale;  /* fp8: [num_pages*num_kv_heads], index page*Hkv + h */
  const float *v_scale;
  const int32_t *block_table;
  const int32_t *page_indptr; /* NULL = 2-D block table */
  const int32_t *ctx_lens;    /* [num_requests] tokens (or pages, see flags) */
  const float *lin_w;         /* linear mode weights */
  /* lever tables; NULL = that lever's stock behaviour */
  const int32_t *order;       /* i32[max_tasks] pi */
  const void *ctrl;           /* SchedCtrl layout, rows[max_tasks] */
  unsigned long long *timer;  /* u64[max_tasks] residency accumulators */
  uint32_t *queue;            /* ticket counter */
  /* Split-KV work items (NULL = one work item per task), in one of two row
   * formats (tile_format):
   * SCHED_PD_TILES_PAIRS: tiles[2*i], tiles[2*i+1] = (task, chunk) of work
   *   item i; chunk c of a task covers its pages [c*tile_pages,
   *   (c+1)*tile_pages). A task has ceil(ceil(ctx/page_size)/tile_pages)
   *   chunks (at least 1).
   * SCHED_PD_TILES_RANGED: tiles[4*i .. 4*i+3] = (task, chunk | nchunks << 16,
   *   p0, p1): chunk `chunk` of the task's `nchunks` covers its pages
   *   [p0, p1), so chunk sizes may differ (tile_pages is unused). The ranges
   *   of a task's chunks are contiguous from page 0 (chunk c+1's p0 = chunk
   *   c's p1), every row of a task carries the same nchunks (1..65535), and
   *   the last range ends at or past the context's last page; a range past
   *   the context reads nothing.
   * Either list is task-major: the chunks of a task are consecutive and in
   * chunk order. pi, num_tasks, order_size and the ticket queue count work
   * items; policy rows and timer rows stay per task. Plan the list from the
   * ctx_lens of the launch: chunks a shorter context does not reach add
   * nothing (the result is unchanged), but a task whose context reaches past
   * the list's last chunk is stale -- its output rows are written as NaN and
   * it is counted in the workspace's stale counter. A list that is not
   * task-major (chunks out of order, a task's rows not consecutive, ranged
   * rows disagreeing on nchunks) gives undefined output rows and may leave
   * arrival counters nonzero: zero the workspace before its next use. The
   * kernels read and write nothing outside the tables, the workspace and
   * the output either way. */
  const int32_t *tiles;
  uint32_t num_tiles;
  uint32_t tile_format;  /* SCHED_PD_TILES_PAIRS (0) or SCHED_PD_TILES_RANGED */
  /* Device scratch for split tasks (sched_paged_decode_workspace_bytes),
   * 256-byte aligned: bytes [0, 4) a u32 stale-plan counter (tasks found
   * stale, see tiles; the launcher only adds to it: read it after the launch
   * and zero it to reset), then from byte 256 the per-task arrival counters,
   * then per-work-item partial results. The arrival counters must be zero
   * before the first launch; each launch leaves them zero (a stale task's
   * counter is never touched). Launches sharing one workspace must not
   * overlap (use one workspace per stream). */
  void *workspace;
  uint64_t workspace_bytes;
} SchedDecodeArgs;

/* Fill *a with defaults (ABI version, F32, prefix tau, dT=dR=1, H=0.25,
 * max_tasks=SCHED_MAX_TASKS, everything else 0/NULL). */
void sched_pd_default_args(SchedDecodeArgs *a);

/* Run one decode step on `stream` (a hipStream_t; NULL = default stream).
 * Asynchronous. Replaces the launch sites of the reference's decode kernels
 * (test/paged_decode.cu:207-213, test/hetero_batch.cu:130-134,
 * python/kernels/paged_softmax.cu:47-54). */
int sched_paged_decode(const SchedDecodeArgs *a, void *stream);

/* sched_paged_decode without any allocation, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc); it has no counterpart in the reference. Same
 * arguments, except that a->workspace must be NULL and workspace_bytes 0: a
 * split launch (tiles != NULL) uses the library's own scratch, a 16 MiB
 * device array per GPU held until the process ends, and is rejected with
 * hipErrorInvalidValue when it needs more (sched_paged_decode_workspace_bytes
 * above 16 MiB). Before each split launch one small kernel on `stream` zeroes
 * the scratch's stale counter and this launch's arrival counters. Calls on one
 * GPU share its scratch: calls that overlap on one GPU (two streams, two
 * threads) race. Without tiles it is sched_paged_decode. Returns 0 or a
 * hipError_t code. */
int sched_paged_decode_noalloc(const SchedDecodeArgs *a, void *stream);

/* Bytes of workspace a launch with these arguments needs (0 without tiles,
 * or -1 on invalid arguments). */
int64_t sched_paged_decode_workspace_bytes(const SchedDecodeArgs *a);

/* Work items resident per CU for the kernel `a` selects (workgroups per CU,
 * times the tasks a workgroup of the one-wave-per-task kernel runs; 0 =
 * unknown). Counterpart of reference paged_softmax_occupancy
 * (python/kernels/paged_softmax.cu:61-67), whose CTAs are tasks. */
int sched_paged_decode_occupancy(const SchedDecodeArgs *a);

/* Policy lever depths of the kernel a launch with a nonzero pf_dist selects
 * (a->pf_dist ignored; the one-wave kernel, which has no ring, is set aside): *stock =
 * pages of loads in flight per wave for stock and polite tasks, *deepest = the
 * deepest ring an urgent task may use (its default); pf_dist may be 0 or any
 * value in [*stock, *deepest]. Both 0 for the VALU kernel, which has no ring
 * (pf_dist must be 0 there). The counterpart of the reference's SCHED_PF_DIST
 * (lib/SchedUtil.cpp:48), a per-build constant there and a per-launch choice
 * among compiled depths here. Returns 0 or a hipError_t code. */
int sched_paged_decode_prefetch_range(const SchedDecodeArgs *a, uint32_t *stock,
                                      uint32_t *deepest);

/* Which kernel `a` selects: 0 = the general VALU kernel (one workgroup per
 * work item), 1 = MFMA, 2 = one wave per work item (softmax over token-major
 * K and V rows, 1..3 q-heads per kv-head), -1 = invalid args. Selection: the
 * one-wave kernel at one q-head per kv-head wherever it applies (unless
 * pf_dist asks for the MFMA kernel's prefetch ring), else the MFMA kernel
 * where it applies, else the one-wave kernel where it applies, else the
 * VALU kernel. */
int sched_paged_decode_kernel_kind(const SchedDecodeArgs *a);

/* Compute-unit count of the current device (0 on error). */
int sched_pd_cu_count(void);

/* Host-to-device copy of `bytes` from `src` to `dst` on `stream`. No
 * counterpart in the reference: the Python layer stages each step's small
 * host arrays (lengths, split plan, block-table update, order, control rows)
 * in a pinned ring and copies them with this call. When `src..src+bytes`
 * lies in memory from sched_pd_staging_alloc, `dst..dst+bytes` lies in one
 * device allocation and `bytes` is at most 1 MiB, a kernel on `stream` does
 * the copy, reading the host memory directly (no hand-off to the copy
 * engine and back); otherwise hipMemcpyAsync (asynchronous when `src` is
 * pinned). Either way the bytes are read when the copy runs on the stream,
 * not at the call. Returns 0 or a hipError_t code. */
int sched_pd_copy_to_device(void *dst, const void *src, uint64_t bytes, void *stream);

/* Pinned host memory of `bytes` (1 B to 4 GiB), mapped into every device's
 * address space and coherent, for staging uploads that
 * sched_pd_copy_to_device runs as a kernel. No counterpart in the
 * reference. Held until the process ends (at most 64 regions). NULL on
 * error (sched_pd_last_error). */
void *sched_pd_staging_alloc(uint64_t bytes);

/* Streaming-read ceiling probe, no counterpart in the reference: reads
 * `bytes` (16-byte aligned) of `buf` once on `stream`, writes nothing (sink
 * may be NULL). Timing it gives the device's achievable read bandwidth, the
 * measured peak beside the vendor figure. Returns 0 or a hipError_t code. */
int sched_pd_read_probe(const void *buf, uint64_t bytes, void *sink, void *stream);

/* Random-block read ceiling, no counterpart in the reference: reads blocks
 * block_ids[0..nblocks) of block_bytes each (16-byte multiple) from `buf`
 * (`bytes` long; ids outside it are skipped) with non-temporal loads, the
 * access pattern of a decode over scattered (page, kv-head) blocks. Writes
 * nothing (sink may be NULL). Returns 0 or a hipError_t code. */
int sched_pd_read_probe_blocks(const void *buf, uint64_t bytes, const int32_t *block_ids,
                               uint32_t nblocks, uint32_t block_bytes, void *sink, void *stream);

/* Last error text of this thread ("" if none). */
const char *sched_pd_last_error(void);

/* ---- 3. reference JIT-kernel launcher ------------------------------------ */

/* reference python/kernels/paged_softmax.cu:47-54: fp32 online-softmax decode,
 * one task per request, head dim 32, page layout [token][64] with K in
 * elements 0..31 and V in 32..63, score scale 0.125, nbl[seq] full pages per
 * request. Levers come from the C runtime's slots (sched_rt_init); tau counts
 * tokens within each page, as the reference's woven innermost loop does. */
void launch_paged_softmax(const void *kv, const void *bt, const void *nbl,
                          const void *q, void *out, int nseq, int bt_stride,
                          int page_tokens, void *stream);
/* python/kernels/paged_softmax.cu:61-67: workgroups per CU, 0 = unknown. */
int paged_softmax_occupancy(void);

#ifdef __cplusplus
}
#endif

#endif /* SCHED_PD_H */
