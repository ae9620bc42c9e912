/* sched_kv.h -- paged KV-cache writer for the decode pools of sched_pd.h.
 *
 * The reference has no writer of its own: its decode paths read caches that
 * FlashInfer (flashinfer-python==0.6.12, requirements.txt:6) or the serving
 * engine filled, in the CSR format its tests build (kv_indptr, kv_indices,
 * last_page_len; test/py/eval_pi_makespan.py:46-60). sched_kv_append is the
 * counterpart of FlashInfer's append_paged_kv_cache with its
 * (append_indptr, seq_lens) position rule, writing the pools in the layout
 * the decode kernels read, and quantising on write for an fp8 cache.
 *
 * Append rule. Request r appends n_r = append_indptr[r+1] - append_indptr[r]
 * tokens, source rows append_indptr[r] .. append_indptr[r+1]-1, at token
 * positions ctx_lens[r] - n_r .. ctx_lens[r] - 1 (ctx_lens counts tokens
 * after the append). Position p lives in page table entry p / page_size,
 * slot p % page_size; the page table is the decode's (block_table with
 * bt_stride, or CSR through page_indptr).
 *
 * fp8 cache (OCP e4m3fn). Every (page, kv-head) has one fp32 scale for K and
 * one for V (index page*num_kv_heads + h); stored code c means c * scale.
 * Scales are powers of two: for the amax a of the tokens an append writes
 * into a (page, head), P(a) = the least 2^k (k >= -126) with a <= 448 * 2^k,
 * and P(0) = 0. A page's first append (it writes slot 0) sets scale = P(a);
 * a later append sets scale = max(old, P(a)), and when that grows the scale
 * the page's earlier codes are re-encoded at the new scale, which for a
 * power-of-two ratio moves only their exponent (exact unless a code drops
 * into e4m3's subnormal range). Each value x is written as
 * e4m3(clamp(x * (1/scale), -448, 448)), round-to-nearest-even; 1/0 counts
 * as 0. Non-finite inputs are not supported.
 *
 * bf16 / fp32 caches: values are converted (fp32 -> bf16 round-to-nearest-
 * even) and scales are not touched.
 */
#ifndef SCHED_KV_H
#define SCHED_KV_H

#include <stdint.h>

#include "sched_pd.h"

#ifdef __cplusplus
extern "C" {
#endif

#define SCHED_KV_ABI_VERSION 1u

/* Element (page, kv-head h, slot t, dim j) of the pools, strides in elements:
 *   K: k_pool + page*k_page_stride + h*k_head_stride + t*k_tok_stride + j
 *   V: v_pool + page*v_page_stride + h*v_head_stride + t*v_tok_stride + j*v_dim_stride
 * with v_tok_stride == 1 (d-major V, the MFMA kernel's layout) or
 * v_dim_stride == 1 (token-major V). A d-major V is written in groups of 4
 * slots: the unused slots after a request's last token, up to its group's
 * end, are written as zero. Source row i, head h, dim j:
 *   k_src[i*src_tok_stride + h*src_head_stride + j] (v_src alike). */
typedef struct SchedKvAppendArgs {
  uint32_t abi_version;   /* SCHED_KV_ABI_VERSION */
  uint32_t src_dtype;     /* SCHED_PD_F32, SCHED_PD_BF16 or SCHED_PD_F16 */
  uint32_t kv_dtype;      /* SCHED_PD_F32, SCHED_PD_BF16, SCHED_PD_F16 or SCHED_PD_FP8_E4M3 */
  uint32_t num_requests;
  uint32_t num_kv_heads;
  uint32_t head_dim;      /* multiple of 4, <= 256 */
  uint32_t page_size;     /* multiple of 4, <= 256 */
  uint32_t bt_stride;     /* 2-D block table row stride (page_indptr == NULL) */
  uint32_t max_append;    /* >= every n_r (sizes the grid; 0 = num_tokens) */
  uint32_t num_tokens;    /* source rows = append_indptr[num_requests] */
  uint64_t num_pages;     /* pool pages; ids outside [0, num_pages) are errors */
  const void *k_src;
  const void *v_src;
  int64_t src_tok_stride, src_head_stride;
  const int32_t *append_indptr; /* [num_requests + 1] */
  const int32_t *ctx_lens;      /* [num_requests], tokens after the append */
  const int32_t *block_table;
  const int32_t *page_indptr;   /* NULL = 2-D block table */
  void *k_pool;
  void *v_pool;
  int64_t k_page_stride, k_head_stride, k_tok_stride;
  int64_t v_page_stride, v_head_stride, v_tok_stride, v_dim_stride;
  float *k_scale;         /* fp8: [num_pages * num_kv_heads], read and written */
  float *v_scale;
  /* Optional u32 error counter (NULL = none): the kernel adds one per
   * (token, kv-head) it could not write (a page id outside the pool, a table
   * entry past the request's pages, or n_r > ctx_lens[r]) and skips it. */
  uint32_t *errors;
  /* kv-heads one workgroup writes (divides num_kv_heads, <= 64); 0 = chosen
   * from the append size. Does not change the result. */
  uint32_t heads_per_group;
  uint32_t _pad0;
} SchedKvAppendArgs;

/* Fill *a with defaults (ABI version, BF16 source and cache, the rest 0/NULL). */
void sched_kv_default_args(SchedKvAppendArgs *a);

/* Append on `stream` (hipStream_t; NULL = default). Asynchronous; returns 0,
 * or -1 with sched_pd_last_error() set for invalid arguments. Pages written
 * by one call must belong to one request each; calls that write the same
 * pages must be stream-ordered. Replaces FlashInfer's append_paged_kv_cache
 * at the serving engine's cache-write site (no call site in the reference's
 * own tree). */
int sched_kv_append(const SchedKvAppendArgs *a, void *stream);

/* One decode step that also appends the step's token of every request: the
 * same result, pools and output, as sched_kv_append(w) followed by
 * sched_paged_decode(a) on the same stream, in one launch. The decode
 * kernel's work item that holds request r's last position (ctx_lens[r] - 1)
 * writes source row r's K and V for each kv-head into it before reading it;
 * for an fp8 cache it applies the writer's scale rule above to that
 * (page, kv-head) first (grow the scale, re-encode the page's earlier slots
 * when it grew, store the scales). No counterpart in the reference (its
 * decode reads caches an engine filled); for serving loops, where the
 * separate append is a small, launch-bound kernel per step. Supported:
 * softmax decode on the MFMA kernel (head dim 128, bf16, fp16 or fp8 cache,
 * token-major V) or the one-wave kernel (the same with a 16-bit cache), the
 * kernel the decode alone would select, so the bits are those of the two
 * calls; one token per request (w->num_tokens == w->num_requests;
 * source row r belongs to request r; append_indptr is not read), source
 * dtype fp32 or the cache's (fp32, bf16 or fp16 for fp8); w's pools,
 * strides, page table, ctx_lens (and fp8 scales) must be a's. Anything else
 * returns hipErrorInvalidValue with sched_pd_last_error() set: d-major V
 * takes the two calls. The page written must exist (ctx_lens[r] >= 1 and its
 * table entry valid); the writer's error counter is not used. */
int sched_paged_decode_append(const SchedDecodeArgs *a, const SchedKvAppendArgs *w,
                              void *stream);

/* Block-table update on `stream`: table[row * width + col] = val for each of
 * the n (row, col, val) triples, packed in device memory as n rows, then n
 * cols, then n vals (int32). Entries outside [0, num_rows) x [0, width) are
 * ignored. One small launch; n == 0 launches nothing. Returns 0, or -1 with
 * sched_pd_last_error() set. No counterpart in the reference (its engine
 * owns the block table): it is how PagedKvCache adds a step's new pages to
 * the device table it keeps between steps. */
int sched_kv_table_update(int32_t *table, int64_t num_rows, int64_t width,
                          const int32_t *updates, uint32_t n, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SCHED_KV_H */
