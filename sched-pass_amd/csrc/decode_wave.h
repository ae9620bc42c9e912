// decode_wave.h -- one wave per work item for 1-3 q-heads per kv-head (G):
// the shape of the reference's JIT kernel (python/kernels/paged_softmax.cu:
// 14-45, fp32, head dim 32, [token][K|V] pages) and of caches with
// token-major rows that the MFMA kernel does not take (fp32 KV or Q, head
// dim 32 / 64, pages that are not a power of two); fp32 / bf16 / fp16 KV,
// head dim 32 (fp32) / 64 / 128, softmax mode.
//
// With G = 1 a task is one (request, head) stream of K and V rows and little
// arithmetic, so what bounds it is how many bytes are in flight and how long
// the chain ctx -> page id -> KV takes, not compute. A workgroup of NWT waves
// runs NWT independent tasks (no LDS, no barrier), so many tasks' chains
// overlap and each wave keeps DEPTH 16-token chunks of loads in flight. One
// wave per workgroup is the default: a wave that finishes a short task frees
// its slot for the next workgroup at once, instead of waiting for the
// longest task of its group.
//
// Lane layout: a K or V row of D elements is LPR = D / VN lanes of 16-byte
// loads (VN elements each); lane = ts * LPR + ds holds dims ds*VN..+VN-1 of
// token slot ts, so one load instruction covers TPI = 64 / LPR tokens and a
// 16-token chunk takes NI = 16 / TPI instructions per tensor. The score of
// a token is the lane's partial dot product summed over its LPR lanes with
// DPP (quad_perm, row_half_mirror, row_mirror; a row swap for 32 lanes), so
// every lane of the slot holds the same bits. Each token slot keeps its own
// online softmax state (m, l, acc) over the tokens it sees (token t of a
// chunk goes to slot t % TPI), with no cross-slot reduction per chunk; the
// TPI slot states merge once per task with lane shuffles. Which slot
// sees a token depends only on the token's position, so the result bits do
// not depend on pi, the work queue or which wave ran the task.
//
// Levers per wave: pi remaps the wave's virtual workgroup id (blockIdx * NWT
// + wave) over the launch's work items; the ticket queue hands tasks to
// waves; the timer row is added by lane 0 of the wave. The shed masks scores
// to -inf (and skips chunks past a prefix budget, as the other kernels do).
// The policy lever has no action here (no prefetch ring choice).
#pragma once

#include <type_traits>

#include "combine.h"

namespace schedpd {

// KV bytes each wave keeps in flight (a build-time tuning knob).
#ifndef SCHED_PD_WAVE_BYTES
#define SCHED_PD_WAVE_BYTES 16384
#endif
// Waves (tasks) per workgroup.
#ifndef SCHED_PD_WAVE_NWT
#define SCHED_PD_WAVE_NWT 1
#endif

typedef __attribute__((ext_vector_type(4))) unsigned wave_u4;

template <typename KVT> struct WaveElem;
template <> struct WaveElem<float> { static constexpr int VN = 4; };
template <> struct WaveElem<uint16_t> { static constexpr int VN = 8; };  // bf16
template <> struct WaveElem<_Float16> { static constexpr int VN = 8; };

// 16 bytes of KV as VN floats.
__device__ __forceinline__ void wave_cvt(const wave_u4 &r, float *f, float) {
  f[0] = __uint_as_float(r.x);
  f[1] = __uint_as_float(r.y);
  f[2] = __uint_as_float(r.z);
  f[3] = __uint_as_float(r.w);
}
__device__ __forceinline__ void wave_cvt(const wave_u4 &r, float *f, uint16_t) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    f[2 * k] = __uint_as_float(w[k] << 16);
    f[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
  }
}
__device__ __forceinline__ void wave_cvt(const wave_u4 &r, float *f, _Float16) {
  typedef __attribute__((ext_vector_type(2))) _Float16 h2;
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const h2 v = __builtin_bit_cast(h2, w[k]);
    f[2 * k] = (float)v.x;
    f[2 * k + 1] = (float)v.y;
  }
}

// DPP controls (GFX9): quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror,
// row_mirror, row_ror:8.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140,
              kDppRor8 = 0x128;

template <int CTRL> __device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over the LPR consecutive lanes of a token slot; every lane of the slot
// ends with the same bits (each step adds a value and its partner's, and
// a + b == b + a).
template <int LPR> __device__ __forceinline__ float slot_sum(float x) {
  if constexpr (LPR >= 2)
    x += dpp_f<kDppXor1>(x);
  if constexpr (LPR >= 4)
    x += dpp_f<kDppXor2>(x);
  if constexpr (LPR >= 8)
    x += dpp_f<kDppHalfMirror>(x);
  if constexpr (LPR >= 16)
    x += dpp_f<kDppMirror>(x);
  if constexpr (LPR >= 32) {
    const unsigned u = __float_as_uint(x);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  }
  return x;
}

// Online softmax state of one token slot (uniform over its LPR lanes) and
// the lane's VN dims of the unnormalised output.
template <int VN> struct WaveState {
  float m, l;
  float acc[VN];
};

// Merge the state of the slot S lanes away into this one (both partners end
// with the same bits: max and the sum of two products commute). Once per
// task, so the exchange is a plain lane shuffle.
template <int S, int VN>
__device__ __forceinline__ void merge_partner(WaveState<VN> &st) {
  const float mo = __shfl_xor(st.m, S), lo = __shfl_xor(st.l, S);
  float ao[VN];
#pragma unroll
  for (int e = 0; e < VN; ++e)
    ao[e] = __shfl_xor(st.acc[e], S);
  const float mn = fmaxf(st.m, mo);
  const float cs = __builtin_amdgcn_exp2f(st.m - mn), co = __builtin_amdgcn_exp2f(mo - mn);
  st.l = st.l * cs + lo * co;
#pragma unroll
  for (int e = 0; e < VN; ++e)
    st.acc[e] = st.acc[e] * cs + ao[e] * co;
  st.m = mn;
}

template <typename KVT, int D> struct WaveShape {
  static constexpr int VN = WaveElem<KVT>::VN;
  static constexpr int LPR = D / VN;        // lanes per K / V row
  static constexpr int TPI = 64 / LPR;      // token slots (tokens per load instruction)
  static constexpr int NI = 16 / TPI;       // load instructions per tensor per 16-token chunk
  // chunks in flight per wave: SCHED_PD_WAVE_BYTES of KV, at least two
  static constexpr int CHUNK_BYTES = 16 * D * (int)sizeof(KVT) * 2;
  static constexpr int DEPTH =
      SCHED_PD_WAVE_BYTES / CHUNK_BYTES >= 2 ? SCHED_PD_WAVE_BYTES / CHUNK_BYTES : 2;
  static_assert(LPR >= 2 && LPR <= 32 && TPI * LPR == 64 && NI * TPI == 16, "wave shape");
};

template <typename KVT, int D> struct WaveChunk {
  wave_u4 k[WaveShape<KVT, D>::NI];
  wave_u4 v[WaveShape<KVT, D>::NI];
};

// Work items of one wave: the static grid (virtual workgroup id = blockIdx *
// NWT + wave, remapped by pi over the launch's items) or the ticket queue
// (W worker waves; claim after the body, lane 0's atomic, broadcast by
// readfirstlane). Same decisions as run_tasks, per wave.
template <int NWT, class Body>
__device__ __forceinline__ void run_wave_tasks(const LeverTables &L, Body &&body) {
  const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t pid = blockIdx.x * NWT + w;
  uint32_t ntasks = 0u;
  if (L.wq) {
    const bool armed = lt_queue(L) != nullptr && lt_ctrl(L) != nullptr && gridDim.y == 1 &&
                       gridDim.z == 1;
    ntasks = armed ? ld_u32(lt_ctrl(L) + SCHED_CTRL_NUM_TASKS_OFF) : 0u;
  }
  if (ntasks == 0u) {
    // Static grid (or a queue grid disarmed on the device): every position
    // once. Within each round of `spread` workgroups (those resident at
    // once) positions run wave-major: wave w of the round's j-th workgroup
    // takes position w * (round size) + j, so consecutive positions of pi
    // (the longest tasks first, under LPT) land in different workgroups and
    // CUs instead of sharing the first workgroup's four waves. Positions of
    // a later round start after those of an earlier one, as with the
    // one-task-per-workgroup kernels.
    uint32_t v0 = pid;
    if (L.spread > 1u) {
      const uint32_t R = L.spread, g = blockIdx.x / R, j = blockIdx.x % R;
      const uint32_t Rg = min(R, gridDim.x - g * R);
      v0 = g * R * NWT + w * Rg + j;
    }
    for (uint32_t v = v0; v < L.nitems; v += gridDim.x * NWT)
      body(remap_static(L, v, L.nitems));
    return;
  }
  const uint32_t W = L.workers;
  if (pid >= W || pid >= ntasks)
    return;
  const uint32_t last_ticket = W + ntasks - 1u;
  const uint32_t lane = threadIdx.x & 63u;
  uint32_t raw = pid;
  while (true) {
    body(remap_wq(L, raw, ntasks));
    uint32_t t = 0u;
    if (lane == 0u) {
      t = __hip_atomic_fetch_add(lt_queue(L), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (t == last_ticket)
        __hip_atomic_store(lt_queue(L), W, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    raw = __builtin_amdgcn_readfirstlane(t);
    if (raw >= ntasks)
      return;
  }
}

// End of one work item of the one-wave kernel, per head g: the wave's merged
// state (lanes of token slot 0 hold dims ds*VN..+VN-1 of acc; m and l are
// the same on every lane) -> the task's output rows, or this item's partial
// and, in the item that completes the task, the merge of the task's
// partials in chunk order (merge_partials, all 64 lanes). The wave waits for
// its partial's stores before its arrival atomic; the reading item loads
// only after its own arrival has returned (see the handoff note at the top
// of combine.h).
template <int G, int VN, int D>
__device__ __forceinline__ void finish_wave_item(const KParams &P, uint32_t wi, uint32_t task,
                                                 uint32_t chunk, uint32_t nchunks, uint32_t r,
                                                 uint32_t h, const WaveState<VN> (&st)[G],
                                                 uint32_t lane, uint32_t ts, uint32_t ds) {
  const int64_t orow = (int64_t)r * P.Hq + (int64_t)h * G;
  if (nchunks <= 1u) {
    if (ts == 0u) {
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < VN; ++e)
          store_out(P, (orow + g) * D + ds * VN + e, st[g].acc[e] / st[g].l);
    }
    return;
  }
  float *pacc = static_cast<float *>(P.ws_acc) + (size_t)wi * G * D;
  float *pml = P.ws_ml + (size_t)wi * G * 2;
  if (ts == 0u) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < VN; ++e)
        __hip_atomic_store(pacc + g * D + ds * VN + e, st[g].acc[e], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  }
  if (lane == 0u) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      __hip_atomic_store(pml + 2 * g, st[g].m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(pml + 2 * g + 1, st[g].l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  uint32_t last = 0u;
  if (lane == 0u)
    last = arrive(P.ws_count + task, nchunks) ? 1u : 0u;
  if (__builtin_amdgcn_readfirstlane(last))
    merge_partials<D, float, false>(P, wi - chunk, nchunks, G, orow, lane, 64u);
}

template <typename KVT, int D, int NWT, int G>
__global__ void __launch_bounds__(NWT * 64) decode_wave(KParams P) {
  using S = WaveShape<KVT, D>;
  constexpr int VN = S::VN, LPR = S::LPR, TPI = S::TPI, NI = S::NI, DEPTH = S::DEPTH;
  constexpr uint32_t EB = sizeof(KVT);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t ts = lane / LPR, ds = lane % LPR;
  const bool toff = timer_off_latched(P.L);

  run_wave_tasks<NWT>(P.L, [&](uint32_t wi) __attribute__((always_inline)) {
    if (wi >= P.L.nitems)
      return;
    const unsigned long long t0 = read_clock(P.L.wallclock);
    const ItemRow I = item_row(P, wi);
    const uint32_t task = I.task;
    if (task >= P.ntasks)
      return;
    const uint32_t r = task / P.Hkv, h = task % P.Hkv;
    const TaskPolicy pol = task_policy(P.L, task);
    const uint32_t n = ctx_tokens(P, r);
    const uint32_t nload = load_extent(P, n, pol.budget);
    const uint32_t ps = P.ps, cpp = ps / 16u; // 16-token chunks per page
    const ItemRange R = item_range(P, I, n, (nload + ps - 1u) / ps);
    if (item_skip(P, wi, I, R))
      return;
    const bool stale = item_stale(P, wi, I, R, n);
    // the item's 16-token chunks [c_begin, c_end) of those read
    const uint32_t nchunks = (nload + 15u) / 16u;
    const uint32_t c_end = min(R.p1 * cpp, nchunks), c_begin = min(R.p0 * cpp, c_end);
    const int64_t row = P.indptr ? (int64_t)__builtin_amdgcn_readfirstlane(P.indptr[r])
                                 : (int64_t)r * P.bt_stride;
    // fused append (16-bit caches, head dim 128): the item holding the
    // step's token writes it before streaming, as in the MFMA kernel (a
    // stale plan's chunk 0 too)
    bool wrote = false;
    if constexpr (!std::is_same<KVT, float>::value && D == 128) {
      if (P.app_k != nullptr && n > 0u) {
        const uint32_t pos = n - 1u, pg = pos / ps;
        const bool holds =
            P.tiles == nullptr ||
            (P.tile_ranged ? pg >= I.p0 && pg < I.p1 : I.chunk == pg / P.tile_pages);
        if (holds || (stale && I.chunk == 0u)) {
          append_token<std::is_same<KVT, _Float16>::value>(
              P, r, h, __builtin_amdgcn_readfirstlane(P.bt[row + pg]), pos % ps, lane);
          wrote = true;
        }
      }
    }

    // the lane's VN dims of each head's q, pre-scaled into the exp2 domain
    float q[G][VN];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < VN; ++e)
        q[g][e] = load_q(P, ((int64_t)r * P.Hq + h * G + g) * D + ds * VN + e) * P.scale_log2;

    WaveState<VN> st[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      st[g].m = kMInit;
      st[g].l = 0.f;
#pragma unroll
      for (int e = 0; e < VN; ++e)
        st[g].acc[e] = 0.f;
    }

    // uniform (scalar) page bases; each lane adds a 32-bit offset (its token
    // slot's row and its 16 bytes of the row), so the loads take the
    // scalar-base + vector-offset form
    const uint8_t *kb = static_cast<const uint8_t *>(P.k_pool) + (int64_t)h * P.khs * EB;
    const uint8_t *vb = static_cast<const uint8_t *>(P.v_pool) + (int64_t)h * P.vhs * EB;
    const int64_t kps = P.kps * EB, vps = P.vps * EB;
    const int64_t kstep = (int64_t)TPI * P.kts * EB, vstep = (int64_t)TPI * P.vts * EB;
    const int64_t krow = P.kts * EB, vrow = P.vts * EB;
    const uint32_t klane = ts * (uint32_t)krow + ds * 16u, vlane = ts * (uint32_t)vrow + ds * 16u;
    const bool prefix = P.tau_scope == SCHED_PD_TAU_PREFIX;
    const uint32_t budget = pol.budget;

    // Page ids in windows of 64 pages: lane i holds the id of window page i
    // (one vector load per window), read back per chunk with readlane, so a
    // chunk's KV loads never wait on a page-table load.
    int32_t win = 0;
    uint32_t w0 = 0;
    auto issue = [&](uint32_t c, WaveChunk<KVT, D> &B) __attribute__((always_inline)) {
      const uint32_t b = c / cpp, o = (c % cpp) * 16u;
      const int64_t page = __builtin_amdgcn_readlane(win, (int)(b - w0));
      const uint8_t *kp = kb + page * kps + (int64_t)o * krow;
      const uint8_t *vp = vb + page * vps + (int64_t)o * vrow;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        B.k[i] = __builtin_nontemporal_load(
            reinterpret_cast<const wave_u4 *>(kp + i * kstep + (uint64_t)klane));
        B.v[i] = __builtin_nontemporal_load(
            reinterpret_cast<const wave_u4 *>(vp + i * vstep + (uint64_t)vlane));
      }
    };
    auto compute = [&](uint32_t c, const WaveChunk<KVT, D> &B) __attribute__((always_inline)) {
      const uint32_t pos0 = c * 16u, o = (c % cpp) * 16u; // o: chunk offset in its page
      float s[G][NI];
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        float f[VN];
        wave_cvt(B.k[i], f, KVT());
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float dot = 0.f;
#pragma unroll
          for (int e = 0; e < VN; ++e)
            dot = __builtin_fmaf(q[g][e], f[e], dot);
          s[g][i] = slot_sum<LPR>(dot);
        }
      }
      // the mask is a select per token, with no test for a chunk that needs
      // none (an unshed budget is 0xFFFFFFFF): a branch here splits the
      // steady loop's body into blocks, the compiler then moves the softmax
      // and PV of every chunk below the reloads, and the ring's old V
      // registers are copied at the back edge after waiting for their loads
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const uint32_t k = i * TPI + ts; // token in the chunk
        const bool keep = (pos0 + k < n) & ((prefix ? pos0 + k : o + k) < budget);
#pragma unroll
        for (int g = 0; g < G; ++g)
          s[g][i] = keep ? s[g][i] : kNegInf;
      }
      float p[G][NI];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float mc = s[g][0];
#pragma unroll
        for (int i = 1; i < NI; ++i)
          mc = fmaxf(mc, s[g][i]);
        const float mn = fmaxf(st[g].m, mc);
        const float cf = __builtin_amdgcn_exp2f(st[g].m - mn);
        float lsum = 0.f;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          p[g][i] = __builtin_amdgcn_exp2f(s[g][i] - mn);
          lsum += p[g][i];
        }
        st[g].l = st[g].l * cf + lsum;
#pragma unroll
        for (int e = 0; e < VN; ++e)
          st[g].acc[e] *= cf;
        st[g].m = mn;
      }
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        float f[VN];
        wave_cvt(B.v[i], f, KVT());
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int e = 0; e < VN; ++e)
            st[g].acc[e] = __builtin_fmaf(p[g][i], f[e], st[g].acc[e]);
      }
    };

    // The prologue's and the tail's loads: buffer loads over the chunk's own
    // rows, with an empty range for a chunk past the segment, whose loads
    // then return 0 and read nothing (the buffer range check). Every path
    // issues the same loads, with no branch and no re-read: a conditional
    // load makes the compiler's vmcnt waits drain the ring. Offsets are 32
    // bits (a chunk's 16 rows span less than 2 GiB; the launcher checks).
    const uint32_t kstep32 = (uint32_t)kstep, vstep32 = (uint32_t)vstep;
    auto issue_or_skip = [&](uint32_t c, bool live, uint32_t cfirst,
                             WaveChunk<KVT, D> &B) __attribute__((always_inline)) {
      const uint32_t cc = live ? c : cfirst; // a chunk of the window, for the page id
      const uint32_t b = cc / cpp, o = (cc % cpp) * 16u;
      const int64_t page = __builtin_amdgcn_readlane(win, (int)(b - w0));
      const int nrec = live ? 0x7FFFFFFF : 0;
      const auto rk = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint8_t *>(kb + page * kps + (int64_t)o * krow), (short)0, nrec, kBufWord3);
      const auto rv = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint8_t *>(vb + page * vps + (int64_t)o * vrow), (short)0, nrec, kBufWord3);
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        B.k[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, klane + i * kstep32, 0, kBufNT);
        B.v[i] = __builtin_amdgcn_raw_buffer_load_b128(rv, vlane + i * vstep32, 0, kBufNT);
      }
    };

    // Segments of up to 64 pages: load the window, then stream its chunks
    // through a ring of DEPTH chunks -- a prologue, a branch-free steady
    // loop, so the compiler's vmcnt waits keep DEPTH-1 chunks in flight, and
    // a tail of fewer than 2 DEPTH chunks with the same waits.
    // the appended token is read back from the cache: its stores complete
    // first
    if (wrote)
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    const uint32_t pg_end = (c_end + cpp - 1u) / cpp;
    for (w0 = c_begin / cpp; w0 < pg_end; w0 += 64u) {
      const uint32_t wn = min(pg_end - w0, 64u);
      win = lane < wn ? P.bt[row + w0 + lane] : 0;
      const uint32_t c0 = max(w0 * cpp, c_begin);
      const uint32_t c1 = min((w0 + wn) * cpp, c_end);
      const uint32_t cnt = c1 - c0;
      WaveChunk<KVT, D> buf[DEPTH];
#pragma unroll
      for (int sl = 0; sl < DEPTH; ++sl)
        issue_or_skip(c0 + sl, sl < cnt, c0, buf[sl]);
      uint32_t j = 0;
      for (; j + 2u * DEPTH <= cnt; j += DEPTH) {
#pragma unroll
        for (int sl = 0; sl < DEPTH; ++sl) {
          compute(c0 + j + sl, buf[sl]);
          // the slot's reload after its last use, so that it takes the same
          // registers (a hoisted load needs others and a copy on the back edge)
          __builtin_amdgcn_sched_barrier(0);
          issue(c0 + j + DEPTH + sl, buf[sl]);
        }
      }
      // tail: a round that computes DEPTH chunks and issues the rest (empty
      // ranges past the segment) when more than DEPTH are left, then a round
      // that computes what is left; either way the last DEPTH chunks' loads
      // are outstanding in slot order at the join
      if (j + DEPTH < cnt) {
#pragma unroll
        for (int sl = 0; sl < DEPTH; ++sl) {
          compute(c0 + j + sl, buf[sl]);
          __builtin_amdgcn_sched_barrier(0);
          issue_or_skip(c0 + j + DEPTH + sl, j + DEPTH + sl < cnt, c0, buf[sl]);
        }
        j += DEPTH;
      }
#pragma unroll
      for (int sl = 0; sl < DEPTH; ++sl)
        if (j + sl < cnt)
          compute(c0 + j + sl, buf[sl]);
    }

    // merge the TPI token slots (lanes LPR, 2 LPR, ... apart)
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if constexpr (TPI >= 8)
        merge_partner<8, VN>(st[g]);
      if constexpr (TPI >= 4)
        merge_partner<16, VN>(st[g]);
      if constexpr (TPI >= 2)
        merge_partner<32, VN>(st[g]);
    }
    if (stale) {
      // the plan does not cover the context: chunk 0's item writes the
      // task's rows as NaN and counts the task; nothing merges
      if (I.chunk == 0u) {
        const int64_t orow = (int64_t)r * P.Hq + (int64_t)h * G;
        for (uint32_t idx = lane; idx < (uint32_t)(G * D); idx += 64u)
          store_out(P, orow * D + idx, __builtin_nanf(""));
        if (lane == 0u)
          __hip_atomic_fetch_add(P.ws_stale, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    } else {
      finish_wave_item<G, VN, D>(P, wi, task, I.chunk, R.nchunks, r, h, st, lane, ts, ds);
    }
    unsigned long long *timer = lt_timer(P.L);
    if (lane == 0u && timer != nullptr && task < P.L.max_tasks && !toff) {
      const unsigned long long dt = read_clock(P.L.wallclock) - t0;
      __hip_atomic_fetch_add(timer + task, dt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  });
}

} // namespace schedpd
