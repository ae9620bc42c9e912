// combine.h -- end of one work item: merge the wave states of the workgroup
// (fixed wave order), then either write the task's output (the task is one
// work item) or publish the work item's partial and, in the work item that
// completes the task, merge all partials of the task in chunk order.
//
// The merge order depends only on the task's chunking, never on which
// workgroup finished last, so split tasks stay bit-reproducible under any pi
// or work-queue schedule.
//
// Cross-XCD handoff without L2 maintenance: partials are written and read
// with agent-scope relaxed atomic stores / loads (sc1: coherent at device
// scope, so the per-XCD L2s are not involved), and each wave waits for its
// stores to complete (s_waitcnt vmcnt(0)) before the barrier that precedes the
// arrival atomic; the reading work item issues its loads only after its
// arrival atomic has returned. This is an ordering the hardware provides (a
// completed sc1 store is visible at the device coherence point), not one the
// HIP memory model states for relaxed atomics: that needs a release/acquire
// edge, i.e. an acq_rel arrival atomic, which on gfx950 writes back and
// invalidates the XCD's L2 once per work item. Measured with that one change
// on a queue launch over 128-page tiles (256 requests of the Llama-3-8B shape,
// lognormal contexts, median 1024): 378 -> 478 us; on the fp8 Qwen2-7B queue
// launch: 356 -> 431 us. The other way the memory model allows without L2
// maintenance -- every published value in a 64-bit word with a "published"
// tag that the merging item validates word by word and then clears, so that
// no ordering between words is needed -- was built and measured on the same
// batch's queue launch over the graded plan: 366 -> 404 us (8-byte words
// +9 us, the per-word checks +12 us, the clears +17 us). The
// arrival counter is reset to 0 by the work item that completes the task:
// every other chunk has already arrived.
#pragma once

#include "common.h"

namespace schedpd {

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima), GFX9 encoding.
constexpr int kWaitVmcnt0 = 0x0F70;

template <typename T> __device__ __forceinline__ T ld_coherent(const T *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Build-time choice of the handoff's ordering (above), for measurement: 0 =
// relaxed arrival (the default); 1 = a release arrival and, in the item that
// merges, an acquire fence (the HIP memory model's edge); 2 = the release
// alone; 3 = the acquire alone.
#ifndef SCHED_PD_HANDOFF_RELACQ
#define SCHED_PD_HANDOFF_RELACQ 0
#endif

// One work item's arrival at its task's counter (one thread); true in the
// item that completes the task, which resets the counter for the next launch
// (every other chunk has already arrived).
__device__ __forceinline__ bool arrive(uint32_t *count, uint32_t nchunks) {
  constexpr int kMode = SCHED_PD_HANDOFF_RELACQ;
  const uint32_t old = (kMode == 1 || kMode == 2)
                           ? __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELEASE,
                                                    __HIP_MEMORY_SCOPE_AGENT)
                           : __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
  const bool last = old == nchunks - 1u;
  if (last) {
    __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (kMode == 1 || kMode == 3)
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  return last;
}

// The merge of a task's partials, in the work item that completes it: the
// partials of chunks 0 .. nchunks-1 (work items base .. base + nchunks - 1)
// read in chunk order, outputs (orow + g) * D + j for g < G (linear: orow * D
// + j). Threads tid, tid + nthreads, ... take the G * D outputs. The loads go
// out kMergeBatch chunks at a time (chunk indices past the last are clamped
// to it and their terms dropped by a select), so a task of N chunks costs
// about N / kMergeBatch memory round trips; the sums run in chunk order.
template <int D, typename AccT, bool LINEAR>
__device__ __forceinline__ void merge_partials(const KParams &P, uint32_t base, uint32_t nchunks,
                                               uint32_t G, int64_t orow, uint32_t tid,
                                               uint32_t nthreads) {
  constexpr uint32_t kMergeBatch = 8;
  const uint32_t clast = nchunks - 1u;
  for (uint32_t idx = tid; idx < G * D; idx += nthreads) {
    const uint32_t g = idx / D, j = idx % D;
    if (LINEAR) {
      const AccT *acc = static_cast<const AccT *>(P.ws_acc) + (size_t)base * G * D + j;
      AccT a = 0;
      for (uint32_t c0 = 0; c0 < nchunks; c0 += kMergeBatch) {
        AccT v[kMergeBatch];
#pragma unroll
        for (uint32_t k = 0; k < kMergeBatch; ++k)
          v[k] = ld_coherent(acc + (size_t)min(c0 + k, clast) * G * D);
#pragma unroll
        for (uint32_t k = 0; k < kMergeBatch; ++k)
          a = c0 + k < nchunks ? a + v[k] : a;
      }
      store_out(P, orow * D + j, (float)a);
    } else {
      // (m, l) of a chunk as one 8-byte load
      const uint64_t *ml = reinterpret_cast<const uint64_t *>(P.ws_ml + (size_t)base * G * 2) + g;
      const AccT *acc = static_cast<const AccT *>(P.ws_acc) + (size_t)base * G * D + g * D + j;
      const size_t stride_ml = G; // u64 words per chunk
      const size_t stride_acc = (size_t)G * D;
      // one pass: each batch's (m, l) and accumulators load together; the
      // running max moves per batch and rescales the sums (for up to
      // kMergeBatch chunks the arithmetic is that of a max pass followed by
      // a sum pass)
      float M = 0.f, Lt = 0.f, A = 0.f;
      for (uint32_t c0 = 0; c0 < nchunks; c0 += kMergeBatch) {
        uint64_t w[kMergeBatch];
        AccT v[kMergeBatch];
#pragma unroll
        for (uint32_t k = 0; k < kMergeBatch; ++k) {
          const size_t c = min(c0 + k, clast);
          w[k] = ld_coherent(ml + c * stride_ml);
          v[k] = ld_coherent(acc + c * stride_acc);
        }
        // a clamped repeat of the last chunk leaves the max unchanged
        float Mb = __uint_as_float((uint32_t)w[0]);
#pragma unroll
        for (uint32_t k = 1; k < kMergeBatch; ++k)
          Mb = fmaxf(Mb, __uint_as_float((uint32_t)w[k]));
        if (c0 == 0u) {
          M = Mb;
        } else if (Mb > M) {
          const float cf = __builtin_amdgcn_exp2f(M - Mb);
          Lt *= cf;
          A *= cf;
          M = Mb;
        }
#pragma unroll
        for (uint32_t k = 0; k < kMergeBatch; ++k) {
          const float e = __builtin_amdgcn_exp2f(__uint_as_float((uint32_t)w[k]) - M);
          const float lt = Lt + __uint_as_float((uint32_t)(w[k] >> 32)) * e;
          const float at = A + (float)v[k] * e;
          const bool in = c0 + k < nchunks;
          Lt = in ? lt : Lt;
          A = in ? at : A;
        }
      }
      store_out(P, (orow + g) * D + j, A / Lt);
    }
  }
}

// Softmax: acc is unnormalised with running max m and sum l per head.
// Linear: acc is a plain sum (m, l unused).
template <int NW, int GMAX, int D, typename AccT, bool LINEAR>
__device__ __forceinline__ void finish_item(const KParams &P, uint32_t wi, uint32_t task,
                                            uint32_t chunk, uint32_t nchunks, uint32_t r,
                                            uint32_t h, uint32_t G, AccT (*s_acc)[GMAX][D],
                                            float (*s_m)[GMAX], float (*s_l)[GMAX]) {
  constexpr uint32_t NT = NW * 64;
  const int64_t orow = LINEAR ? ((int64_t)r * P.Hkv + h) : ((int64_t)r * P.Hq + h * G);
  if (nchunks <= 1) {
    for (uint32_t idx = threadIdx.x; idx < G * D; idx += NT) {
      const uint32_t g = idx / D, j = idx % D;
      if (LINEAR) {
        AccT a = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w)
          a += s_acc[w][0][j];
        store_out(P, orow * D + j, (float)a);
      } else {
        float M = s_m[0][g];
#pragma unroll
        for (int w = 1; w < NW; ++w)
          M = fmaxf(M, s_m[w][g]);
        float Lt = 0.f, A = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const float e = __builtin_amdgcn_exp2f(s_m[w][g] - M);
          Lt += s_l[w][g] * e;
          A += (float)s_acc[w][g][j] * e;
        }
        store_out(P, (orow + g) * D + j, A / Lt);
      }
    }
    return;
  }

  // Publish this work item's partial.
  AccT *pacc = static_cast<AccT *>(P.ws_acc) + (size_t)wi * G * D;
  float *pml = P.ws_ml + (size_t)wi * G * 2;
  for (uint32_t idx = threadIdx.x; idx < G * D; idx += NT) {
    const uint32_t g = idx / D, j = idx % D;
    if (LINEAR) {
      AccT a = 0;
#pragma unroll
      for (int w = 0; w < NW; ++w)
        a += s_acc[w][0][j];
      __hip_atomic_store(pacc + j, a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      float M = s_m[0][g];
#pragma unroll
      for (int w = 1; w < NW; ++w)
        M = fmaxf(M, s_m[w][g]);
      float Lt = 0.f, A = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float e = __builtin_amdgcn_exp2f(s_m[w][g] - M);
        Lt += s_l[w][g] * e;
        A += (float)s_acc[w][g][j] * e;
      }
      __hip_atomic_store(pacc + g * D + j, (AccT)A, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (j == 0) {
        __hip_atomic_store(pml + 2 * g, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(pml + 2 * g + 1, Lt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();
  __shared__ uint32_t s_last;
  if (threadIdx.x == 0)
    s_last = arrive(P.ws_count + task, nchunks) ? 1u : 0u;
  __syncthreads();
  if (!s_last)
    return;
  merge_partials<D, AccT, LINEAR>(P, wi - chunk, nchunks, G, orow, threadIdx.x, NT);
}

// A work item's plan row. Pair rows (task, chunk) cover pages
// [chunk * tile_pages, (chunk + 1) * tile_pages) of the task, the chunk count
// following from the context length. Ranged rows (task, chunk | nchunks << 16,
// p0, p1) carry the task's chunk count and the chunk's page range, so the
// chunks of one task may differ in size. Without a list, work item = task.
struct ItemRow {
  uint32_t task, chunk, nchunks, p0, p1;
};

__device__ __forceinline__ ItemRow item_row(const KParams &P, uint32_t wi) {
  ItemRow I{wi, 0u, 1u, 0u, 0u};
  if (P.tiles == nullptr)
    return I;
  if (P.tile_ranged) {
    const int32_t *row = P.tiles + 4 * (size_t)wi;
    I.task = __builtin_amdgcn_readfirstlane((uint32_t)row[0]);
    const uint32_t cc = __builtin_amdgcn_readfirstlane((uint32_t)row[1]);
    I.chunk = cc & 0xFFFFu;
    I.nchunks = cc >> 16;
    I.p0 = __builtin_amdgcn_readfirstlane((uint32_t)row[2]);
    I.p1 = __builtin_amdgcn_readfirstlane((uint32_t)row[3]);
  } else {
    I.task = __builtin_amdgcn_readfirstlane((uint32_t)P.tiles[2 * wi]);
    I.chunk = __builtin_amdgcn_readfirstlane((uint32_t)P.tiles[2 * wi + 1]);
  }
  return I;
}

// The task's chunk count and the page range [p0, p1) the item reads, within
// the npages_load pages of the task that are read at all (n context tokens).
struct ItemRange {
  uint32_t nchunks, p0, p1;
};

__device__ __forceinline__ ItemRange item_range(const KParams &P, const ItemRow &I, uint32_t n,
                                                uint32_t npages_load) {
  if (P.tiles == nullptr)
    return ItemRange{1u, 0u, npages_load};
  ItemRange it;
  if (P.tile_ranged) {
    it.nchunks = I.nchunks;
    it.p1 = min(I.p1, npages_load);
    it.p0 = min(I.p0, it.p1);
    return it;
  }
  const uint32_t npages_ctx = (n + P.ps - 1) / P.ps;
  it.nchunks = npages_ctx ? (npages_ctx + P.tile_pages - 1) / P.tile_pages : 1u;
  it.p0 = min(I.chunk * P.tile_pages, npages_load);
  it.p1 = min(it.p0 + P.tile_pages, npages_load);
  return it;
}

// What a work item does, decided from the plan and the launch's context
// length. It runs (streams its pages and takes part in the task's merge)
// unless
//   - it is skipped: a pair-row chunk the context does not reach (the plan
//     was built for a longer context; the task's other chunks cover it), or
//     a chunk index that cannot be task-major;
//   - its task is stale: the plan does not cover the context (pair rows: the
//     row of chunk nchunks-1 is not where the task's chunk 0 puts it;
//     ranged rows: that row is missing or its range ends before the
//     context's last page). No item of such a task merges or touches its
//     arrival counter: chunk 0 writes the task's output rows as NaN and
//     counts the task in the workspace's stale counter.
// A ranged chunk past the context reads no page and merges an empty
// partial. Every item of a task reads the same rows and lengths, so they all
// decide alike. The merge only ever reads items [wi - chunk, wi - chunk +
// nchunks), which a running item keeps inside the list.
__device__ __forceinline__ bool item_skip(const KParams &P, uint32_t wi, const ItemRow &I,
                                         const ItemRange &R) {
  return P.tiles != nullptr && (I.chunk > wi || I.chunk >= R.nchunks);
}

// One tile-row load, issued when the item starts and consumed at its merge.
__device__ __forceinline__ bool item_stale(const KParams &P, uint32_t wi, const ItemRow &I,
                                           const ItemRange &R, uint32_t n) {
  if (P.tiles == nullptr)
    return false;
  if (P.tile_ranged) {
    const uint32_t npages_ctx = (n + P.ps - 1) / P.ps;
    if (R.nchunks == 1u)
      return I.p1 < npages_ctx;
    const uint32_t last = wi - I.chunk + R.nchunks - 1u;
    if (last >= P.L.nitems)
      return true;
    const int32_t *row = P.tiles + 4 * (size_t)last;
    const uint32_t lt = __builtin_amdgcn_readfirstlane((uint32_t)row[0]);
    const uint32_t lc = __builtin_amdgcn_readfirstlane((uint32_t)row[1]);
    const uint32_t lp1 = __builtin_amdgcn_readfirstlane((uint32_t)row[3]);
    return !(lt == I.task && lc == ((R.nchunks << 16) | (R.nchunks - 1u)) && lp1 >= npages_ctx);
  }
  if (R.nchunks == 1u)
    return false;
  const uint32_t last = wi - I.chunk + R.nchunks - 1u;
  if (last >= P.L.nitems)
    return true;
  const int32_t lt = __builtin_amdgcn_readfirstlane(P.tiles[2 * last]);
  const int32_t lc = __builtin_amdgcn_readfirstlane(P.tiles[2 * last + 1]);
  return !((uint32_t)lt == I.task && (uint32_t)lc == R.nchunks - 1u);
}

// A stale task's signal: output rows NaN (chunk 0's item writes them), one
// count in the workspace's stale counter.
template <int NW, int D, bool LINEAR>
__device__ __forceinline__ void mark_stale(const KParams &P, uint32_t chunk, uint32_t r,
                                           uint32_t h, uint32_t G) {
  if (chunk != 0u)
    return;
  constexpr uint32_t NT = NW * 64;
  const int64_t orow = LINEAR ? ((int64_t)r * P.Hkv + h) : ((int64_t)r * P.Hq + h * G);
  for (uint32_t idx = threadIdx.x; idx < G * D; idx += NT)
    store_out(P, orow * D + idx, __builtin_nanf(""));
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(P.ws_stale, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

} // namespace schedpd
