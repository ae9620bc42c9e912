// paged_decode.hip -- the C-ABI launchers: sched_paged_decode (one decode
// step over a paged batch with the levers), its occupancy query, and the
// reference's launch_paged_softmax / paged_softmax_occupancy
// (python/kernels/paged_softmax.cu:47-67). The kernels are instantiated in
// kernels_*.hip (kernel_set.h lists them).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>

#include "kernel_set.h"
#include "../../include/sched_kv.h"
#include "rt_internal.h"

SCHED_PD_DECLARE_ALL_KERNELS

using namespace schedpd;

namespace {

// Fewest q-heads per kv-head that the MFMA kernel takes when the one-wave
// kernel also applies. Measured on the 64 x 2048-token bf16 step (Hkv 8,
// token-major V): one wave per item runs 4.0-4.6% behind the MFMA kernel at
// one q-head per kv-head (2.7-3.2% with a 24 KB ring), 25% at two and 55%
// at three (its VALU work grows with the group; the MFMA kernel's does not),
// so the MFMA kernel takes every group it applies to and the one-wave kernel
// the shapes it does not (fp32 KV or Q, head dim 32 / 64, pages that are not
// a power of two).
constexpr uint32_t kMfmaMinGroup = 1;

typedef void (*KernelFn)(KParams);

struct Selected {
  KernelFn fn;
  int block;
  int mfma;     // kernel kind: 0 general VALU, 1 MFMA, 2 one wave per task
  int per_block; // work items a workgroup runs at once
};

template <typename KVT, int D> KernelFn valu_kernel(bool linear, uint32_t G) {
  if (linear)
    return decode_valu<KVT, D, 1, true>;
  if (G <= 1)
    return decode_valu<KVT, D, 1, false>;
  if (G <= 4)
    return decode_valu<KVT, D, 4, false>;
  return decode_valu<KVT, D, 16, false>;
}

template <bool FP8, bool VT = false, bool PG = false>
KernelFn mfma_kernel(uint32_t G, bool linear) {
  constexpr int NW = SCHED_PD_MFMA_NW, DS = mfma_ds(FP8), DU = mfma_du(FP8, VT, PG);
  if (linear)
    return decode_mfma<FP8, NW, 4, DS, DU, true, VT, PG, false>;
  if (G <= 4)
    return decode_mfma<FP8, NW, 4, DS, DU, false, VT, PG, false>;
  if (G <= 8)
    return decode_mfma<FP8, NW, 8, DS, DU, false, VT, PG, false>;
  return decode_mfma<FP8, NW, 16, DS, DU, false, VT, PG, false>;
}

uint32_t elem_bytes(uint32_t dt) {
  return dt == SCHED_PD_F32 ? 4u : (dt == SCHED_PD_BF16 || dt == SCHED_PD_F16) ? 2u : 1u;
}

// fp16 cache with fp16 Q: 16-byte page-16 layouts, softmax mode.
template <bool VT, bool PG = false> KernelFn mfma_kernel_f16(uint32_t G) {
  constexpr int NW = SCHED_PD_MFMA_NW, DS = mfma_ds(false), DU = mfma_du(false, VT, PG, true);
  if (G <= 4)
    return decode_mfma<false, NW, 4, DS, DU, false, VT, PG, true>;
  if (G <= 8)
    return decode_mfma<false, NW, 8, DS, DU, false, VT, PG, true>;
  return decode_mfma<false, NW, 16, DS, DU, false, VT, PG, true>;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

uint64_t round256(uint64_t x) { return (x + 255u) & ~uint64_t(255); }

// Workspace layout for split tasks: [stale-plan counter: u32][counters:
// ntasks u32][(m, l): items x G x 2 f32][partials: items x G x d x (f32
// softmax | f64 linear)], each region 256-byte aligned.
struct WsLayout {
  uint64_t stale_off, count_off, ml_off, acc_off, total;
};

WsLayout ws_layout(const SchedDecodeArgs *a) {
  const bool linear = a->mode == SCHED_PD_LINEAR;
  const uint64_t G = linear ? 1u : a->num_q_heads / a->num_kv_heads;
  const uint64_t ntasks = (uint64_t)a->num_requests * a->num_kv_heads;
  WsLayout L;
  L.stale_off = 0;
  L.count_off = 256;
  L.ml_off = L.count_off + round256(ntasks * 4u);
  L.acc_off = L.ml_off + round256((uint64_t)a->num_tiles * G * 8u);
  L.total = L.acc_off + (uint64_t)a->num_tiles * G * a->head_dim * (linear ? 8u : 4u);
  return L;
}

// V token-major (dims contiguous, aligned token rows).
bool v_token_major(const SchedDecodeArgs *a) {
  return a->v_dim_stride == 1 && a->v_tok_stride != 1;
}

// The MFMA kernel's shape: bf16/fp8 KV with bf16 Q (or fp16 KV with fp16 Q,
// softmax), d 128, pages of 16..256 tokens (a power of two), K rows
// dims-contiguous, V d-major rows of one page (or token-major rows),
// G <= 16, 16-byte aligned pools.
bool mfma_applies(const SchedDecodeArgs *a) {
  if (a->flags & SCHED_PD_FLAG_FORCE_VALU)
    return false;
  const bool linear = a->mode == SCHED_PD_LINEAR;
  if (a->kv_dtype == SCHED_PD_F16) {
    if (linear || a->q_dtype != SCHED_PD_F16)
      return false;
  } else {
    if (!linear && a->q_dtype != SCHED_PD_BF16)
      return false;
    if (a->kv_dtype != SCHED_PD_BF16 && a->kv_dtype != SCHED_PD_FP8_E4M3)
      return false;
  }
  const uint32_t G = linear ? 1u : a->num_q_heads / a->num_kv_heads;
  const uint32_t ps = a->page_size;
  if (a->head_dim != 128 || ps < 16 || ps > 256 || (ps & (ps - 1)) || G > 16)
    return false;
  const int64_t eb = elem_bytes(a->kv_dtype);
  if (v_token_major(a)) {
    // token rows start 16-byte (16-bit V) or 8-byte (fp8 V) aligned
    if ((a->v_tok_stride * eb) % (a->kv_dtype == SCHED_PD_FP8_E4M3 ? 8 : 16))
      return false;
  } else if (a->v_tok_stride != 1 || a->v_dim_stride != (int64_t)ps) {
    return false;
  }
  if ((a->k_tok_stride * eb) % 16 || (a->k_page_stride * eb) % 16 || (a->k_head_stride * eb) % 16)
    return false;
  if ((a->v_page_stride * eb) % 16 || (a->v_head_stride * eb) % 16)
    return false;
  if (linear)
    return aligned16(a->v_pool);
  return aligned16(a->k_pool) && aligned16(a->v_pool) && aligned16(a->q);
}

// Ring depths (pages in flight per wave) of the MFMA kernel `a` selects:
// stock, and the deepest an urgent task may use (its default). 0, 0 for the
// VALU kernel, which has no ring.
void ring_depths(const SchedDecodeArgs *a, bool mfma, uint32_t *ds, uint32_t *du) {
  if (!mfma) {
    *ds = *du = 0;
    return;
  }
  const bool fp8 = a->kv_dtype == SCHED_PD_FP8_E4M3;
  *ds = (uint32_t)mfma_ds(fp8);
  *du = (uint32_t)mfma_du(fp8, v_token_major(a), a->page_size > 16,
                          a->kv_dtype == SCHED_PD_F16);
}

// The one-wave-per-item kernel's shape: softmax, 1..3 q-heads per kv-head,
// fp32 KV (head dim 32/64/128) or bf16 / fp16 KV (64/128), K and V
// token-major rows (dims contiguous), 16-byte aligned pools and strides.
bool wave_applies(const SchedDecodeArgs *a) {
  if (a->flags & (SCHED_PD_FLAG_FORCE_VALU | SCHED_PD_FLAG_NO_WAVE))
    return false;
  if (a->mode != SCHED_PD_SOFTMAX || a->num_q_heads > 3u * a->num_kv_heads)
    return false;
  const uint32_t d = a->head_dim;
  if (a->kv_dtype == SCHED_PD_F32) {
    if (d != 32 && d != 64 && d != 128)
      return false;
  } else if (a->kv_dtype == SCHED_PD_BF16 || a->kv_dtype == SCHED_PD_F16) {
    if (d != 64 && d != 128)
      return false;
  } else {
    return false;
  }
  if (a->v_dim_stride != 1)
    return false;
  const int64_t eb = elem_bytes(a->kv_dtype);
  if ((a->k_tok_stride * eb) % 16 || (a->k_page_stride * eb) % 16 || (a->k_head_stride * eb) % 16)
    return false;
  if ((a->v_tok_stride * eb) % 16 || (a->v_page_stride * eb) % 16 || (a->v_head_stride * eb) % 16)
    return false;
  // a lane's offset into a 16-token chunk is 32 bits (buffer loads)
  const int64_t span = 16 * std::max(a->k_tok_stride, a->v_tok_stride) * eb + d * eb;
  if (a->k_tok_stride < 0 || a->v_tok_stride < 0 || span > INT32_MAX)
    return false;
  return aligned16(a->k_pool) && aligned16(a->v_pool);
}

template <int G> KernelFn wave_kernel_g(const SchedDecodeArgs *a) {
  constexpr int NWT = SCHED_PD_WAVE_NWT;
  if (a->kv_dtype == SCHED_PD_F32)
    return a->head_dim == 32   ? decode_wave<float, 32, NWT, G>
           : a->head_dim == 64 ? decode_wave<float, 64, NWT, G>
                               : decode_wave<float, 128, NWT, G>;
  if (a->kv_dtype == SCHED_PD_BF16)
    return a->head_dim == 64 ? decode_wave<uint16_t, 64, NWT, G>
                             : decode_wave<uint16_t, 128, NWT, G>;
  return a->head_dim == 64 ? decode_wave<_Float16, 64, NWT, G>
                           : decode_wave<_Float16, 128, NWT, G>;
}

KernelFn wave_kernel(const SchedDecodeArgs *a) {
  const uint32_t G = a->num_q_heads / a->num_kv_heads;
  return G == 1 ? wave_kernel_g<1>(a) : G == 2 ? wave_kernel_g<2>(a) : wave_kernel_g<3>(a);
}

// Validate `a`; on success fill *kp (tables resolved) and *sel.
int prepare(const SchedDecodeArgs *a, KParams *kp, Selected *sel) {
  if (a == nullptr)
    return set_error(hipErrorInvalidValue, "args is NULL");
  if (a->abi_version != SCHED_PD_ABI_VERSION)
    return set_error(hipErrorInvalidValue, "abi_version %u, library speaks %u", a->abi_version,
                     SCHED_PD_ABI_VERSION);
  if (a->mode > SCHED_PD_LINEAR)
    return set_error(hipErrorInvalidValue, "unknown mode %u", a->mode);
  auto qo_ok = [](uint32_t dt) {
    return dt == SCHED_PD_F32 || dt == SCHED_PD_BF16 || dt == SCHED_PD_F16;
  };
  if (a->kv_dtype > SCHED_PD_F16 || !qo_ok(a->q_dtype) || !qo_ok(a->o_dtype))
    return set_error(hipErrorInvalidValue, "unsupported dtype (kv %u, q %u, out %u)", a->kv_dtype,
                     a->q_dtype, a->o_dtype);
  if (a->num_kv_heads == 0)
    return set_error(hipErrorInvalidValue, "num_kv_heads is 0");
  const bool linear = a->mode == SCHED_PD_LINEAR;
  if (!linear && (a->num_q_heads == 0 || a->num_q_heads % a->num_kv_heads))
    return set_error(hipErrorInvalidValue, "num_q_heads %u is not a multiple of num_kv_heads %u",
                     a->num_q_heads, a->num_kv_heads);
  const uint32_t G = linear ? 1u : a->num_q_heads / a->num_kv_heads;
  if (G > 16)
    return set_error(hipErrorInvalidValue, "%u q-heads per kv-head, at most 16 supported", G);
  if (a->head_dim != 32 && a->head_dim != 64 && a->head_dim != 128)
    return set_error(hipErrorInvalidValue, "head_dim %u (supported: 32, 64, 128)", a->head_dim);
  if (a->head_dim == 32 && a->kv_dtype != SCHED_PD_F32)
    return set_error(hipErrorInvalidValue, "head_dim 32 is supported for fp32 KV only");
  if (a->page_size == 0 || a->page_size % 16 || a->page_size > 256)
    return set_error(hipErrorInvalidValue, "page_size %u (multiple of 16, at most 256)",
                     a->page_size);
  if (a->tau_scope > SCHED_PD_TAU_PER_PAGE)
    return set_error(hipErrorInvalidValue, "unknown tau_scope %u", a->tau_scope);
  if (!a->out || !a->v_pool || !a->block_table || !a->ctx_lens)
    return set_error(hipErrorInvalidValue, "out, v_pool, block_table and ctx_lens are required");
  if (!linear && (!a->q || !a->k_pool))
    return set_error(hipErrorInvalidValue, "softmax mode needs q and k_pool");
  if (linear && !a->lin_w)
    return set_error(hipErrorInvalidValue, "linear mode needs lin_w");
  if (!a->page_indptr && a->bt_stride == 0)
    return set_error(hipErrorInvalidValue, "bt_stride is 0 with a 2-D block table");

  const int64_t eb = elem_bytes(a->kv_dtype);
  // The matrix cores wherever the MFMA kernel applies (a d-major V included:
  // the general VALU kernel reads it 3.7x slower); the one-wave kernel for
  // groups of 1-3 over token-major rows that the MFMA kernel does not take
  // (fp32 KV or Q, head dim 32 / 64); below kMfmaMinGroup the one-wave
  // kernel first unless the launch asks for an urgent prefetch depth
  // (pf_dist), which only the MFMA kernel's ring serves.
  const bool mfma_ok = !(a->flags & SCHED_PD_FLAG_NO_MFMA) && mfma_applies(a);
  const bool wave_ok = wave_applies(a);
  const bool wave = wave_ok && (!mfma_ok || (G < kMfmaMinGroup && a->pf_dist == 0));
  const bool mfma = mfma_ok && !wave;
  if (!mfma && !linear) {
    // VALU K rows are read with 16-byte vector loads.
    if (!aligned16(a->k_pool) || (a->k_tok_stride * eb) % 16 || (a->k_page_stride * eb) % 16 ||
        (a->k_head_stride * eb) % 16)
      return set_error(hipErrorInvalidValue,
                       "K pool and K page/head/token strides must be 16-byte aligned");
  }

  std::memset(kp, 0, sizeof *kp);
  const bool rt = (a->flags & SCHED_PD_FLAG_RT_TABLES) != 0;
  if (rt) {
    // the kernel reads the tables from the device slots; the host snapshot
    // (what sched_rt_* armed) only decides whether a queue grid is launched
    const RtSnapshot s = rt_snapshot();
    kp->L.order = s.order;
    kp->L.ctrl = static_cast<const uint8_t *>(s.ctrl);
    kp->L.timer = s.timer;
    kp->L.queue = s.queue;
    kp->L.max_tasks = s.rows;
    if (!rt_slot_addresses(kp->L.rt_slot))
      return hipErrorInvalidSymbol;
    kp->L.rt = 1u;
  } else {
    kp->L.order = a->order;
    kp->L.ctrl = static_cast<const uint8_t *>(a->ctrl);
    kp->L.timer = a->timer;
    kp->L.queue = a->queue;
    kp->L.max_tasks = a->max_tasks;
  }
  kp->ntasks = a->num_requests * a->num_kv_heads;
  kp->L.nitems = kp->ntasks;
  if (a->tiles) {
    if (a->tile_format > SCHED_PD_TILES_RANGED)
      return set_error(hipErrorInvalidValue, "tile_format %u is not a tile row format",
                       a->tile_format);
    if (a->num_tiles == 0 || (a->tile_format == SCHED_PD_TILES_PAIRS && a->tile_pages == 0))
      return set_error(hipErrorInvalidValue,
                       "tiles need num_tiles > 0 (and tile_pages > 0 for (task, chunk) rows)");
    const WsLayout W = ws_layout(a);
    if (!a->workspace || a->workspace_bytes < W.total || ((uintptr_t)a->workspace & 255u))
      return set_error(hipErrorInvalidValue,
                       "split tasks need a 256-byte aligned workspace of %llu bytes (got %llu)",
                       (unsigned long long)W.total, (unsigned long long)a->workspace_bytes);
    uint8_t *ws = static_cast<uint8_t *>(a->workspace);
    kp->tiles = a->tiles;
    kp->tile_pages = a->tile_pages;
    kp->tile_ranged = a->tile_format == SCHED_PD_TILES_RANGED ? 1u : 0u;
    kp->L.nitems = a->num_tiles;
    kp->ws_stale = reinterpret_cast<uint32_t *>(ws + W.stale_off);
    kp->ws_count = reinterpret_cast<uint32_t *>(ws + W.count_off);
    kp->ws_ml = reinterpret_cast<float *>(ws + W.ml_off);
    kp->ws_acc = ws + W.acc_off;
  }
  kp->L.wallclock = (a->flags & SCHED_PD_FLAG_WALLCLOCK) ? 1u : 0u;
  kp->L.dT = a->policy_dT;
  kp->L.dR = a->policy_dR;
  kp->L.H = a->policy_H;
  kp->q = a->q;
  kp->out = a->out;
  kp->k_pool = a->k_pool;
  kp->v_pool = a->v_pool;
  kp->kps = a->k_page_stride;
  kp->khs = a->k_head_stride;
  kp->kts = a->k_tok_stride;
  kp->vps = a->v_page_stride;
  kp->vhs = a->v_head_stride;
  kp->vts = a->v_tok_stride;
  kp->vds = a->v_dim_stride;
  kp->k_scale = a->k_scale;
  kp->v_scale = a->v_scale;
  // K and V scales interleaved as (K, V) pairs per (page, head): the two
  // loads of a page's scales then fall in one cache line
  kp->scale_stride = (a->k_scale != nullptr && a->v_scale == a->k_scale + 1) ? 2u : 1u;
  kp->bt = a->block_table;
  kp->indptr = a->page_indptr;
  kp->ctx = a->ctx_lens;
  kp->lin_w = a->lin_w;
  kp->R = a->num_requests;
  kp->Hq = linear ? a->num_kv_heads : a->num_q_heads;
  kp->Hkv = a->num_kv_heads;
  kp->G = G;
  kp->ps = a->page_size;
  kp->bt_stride = a->bt_stride;
  kp->tau_scope = a->tau_scope;
  kp->q_f32 = a->q_dtype == SCHED_PD_F32;
  kp->o_f32 = a->o_dtype == SCHED_PD_F32;
  kp->q_f16 = a->q_dtype == SCHED_PD_F16;
  kp->o_f16 = a->o_dtype == SCHED_PD_F16;
  kp->ctx_in_pages = (a->flags & SCHED_PD_FLAG_CTX_IN_PAGES) ? 1u : 0u;
  kp->shed_loads = (a->flags & SCHED_PD_FLAG_SHED_LOADS) ? 1u : 0u;
  kp->lin_w_period = a->lin_w_period;
  const float scale = a->sm_scale != 0.f ? a->sm_scale : 1.0f / std::sqrt((float)a->head_dim);
  kp->scale_log2 = scale * 1.4426950408889634f;

  sel->per_block = 1;
  if (wave) {
    sel->fn = wave_kernel(a);
    sel->block = SCHED_PD_WAVE_NWT * 64;
    sel->mfma = 2;
    sel->per_block = SCHED_PD_WAVE_NWT;
  } else if (mfma) {
    const bool pg = a->page_size > 16;
    if (a->kv_dtype == SCHED_PD_F16)
      sel->fn = v_token_major(a) ? (pg ? mfma_kernel_f16<true, true>(G) : mfma_kernel_f16<true>(G))
                                 : (pg ? mfma_kernel_f16<false, true>(G)
                                       : mfma_kernel_f16<false>(G));
    else if (a->kv_dtype != SCHED_PD_BF16)
      sel->fn = v_token_major(a) ? (pg ? mfma_kernel<true, true, true>(G, linear)
                                       : mfma_kernel<true, true>(G, linear))
                : pg ? mfma_kernel<true, false, true>(G, linear)
                     : mfma_kernel<true>(G, linear);
    else if (v_token_major(a))
      sel->fn = pg ? mfma_kernel<false, true, true>(G, linear)
                   : mfma_kernel<false, true>(G, linear);
    else
      sel->fn = pg ? mfma_kernel<false, false, true>(G, linear) : mfma_kernel<false>(G, linear);
    sel->block = SCHED_PD_MFMA_NW * 64;
    sel->mfma = 1;
  } else {
    KernelFn fn = nullptr;
    switch (a->kv_dtype) {
    case SCHED_PD_F32:
      fn = a->head_dim == 32   ? valu_kernel<float, 32>(linear, G)
           : a->head_dim == 64 ? valu_kernel<float, 64>(linear, G)
                               : valu_kernel<float, 128>(linear, G);
      break;
    case SCHED_PD_BF16:
      fn = a->head_dim == 64 ? valu_kernel<uint16_t, 64>(linear, G)
                             : valu_kernel<uint16_t, 128>(linear, G);
      break;
    case SCHED_PD_F16:
      fn = a->head_dim == 64 ? valu_kernel<_Float16, 64>(linear, G)
                             : valu_kernel<_Float16, 128>(linear, G);
      break;
    default:
      fn = a->head_dim == 64 ? valu_kernel<uint8_t, 64>(linear, G)
                             : valu_kernel<uint8_t, 128>(linear, G);
      break;
    }
    sel->fn = fn;
    sel->block = SCHED_PD_VALU_NW * 64;
    sel->mfma = 0;
  }
  uint32_t ds = 0, du = 0;
  ring_depths(a, mfma, &ds, &du);
  if (a->pf_dist != 0 && !mfma)
    return set_error(hipErrorInvalidValue,
                     "pf_dist %u: these arguments select a VALU or one-wave kernel, which has "
                     "no prefetch ring (pass 0)", a->pf_dist);
  if (a->pf_dist != 0 && (a->pf_dist < ds || a->pf_dist > du))
    return set_error(hipErrorInvalidValue,
                     "pf_dist %u: the kernel these arguments select keeps %u..%u pages in flight",
                     a->pf_dist, ds, du);
  kp->pf_depth = a->pf_dist;
  return 0;
}

// ---- scratch of the no-allocation entry point ------------------------------
// The split-KV workspace of sched_paged_decode_noalloc: a file-scope device
// array, one copy per GPU, held until the process ends. Host code never
// passes the array's name to a kernel or copy: it uses the device address
// hipGetSymbolAddress returns for the current device (kept per device).
constexpr uint64_t kScratchBytes = 16ull << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];

// The device address of `scratch` on the current device (nullptr on error).
void *scratch_address(int *dev_out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error(e, "hipGetDevice failed: %s", hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_error(hipErrorInvalidDevice, "device %d is beyond the %d the library tracks", dev,
              kMaxDevices);
    return nullptr;
  }
  *dev_out = dev;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      set_error(e != hipSuccess ? e : hipErrorInvalidSymbol,
                "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

// Zero n words at p (stream-ordered; a kernel, so a captured graph records no
// memset node).
__global__ void zero_words(uint32_t *p, uint32_t n) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    p[i] = 0u;
}

} // namespace

extern "C" {

int sched_paged_decode_noalloc(const SchedDecodeArgs *a, void *stream) {
  if (a == nullptr)
    return set_error(hipErrorInvalidValue, "args is NULL");
  if (a->workspace != nullptr || a->workspace_bytes != 0)
    return set_error(hipErrorInvalidValue,
                     "sched_paged_decode_noalloc takes no workspace (it uses the library's "
                     "%llu-byte scratch)", (unsigned long long)kScratchBytes);
  if (a->tiles == nullptr)
    return sched_paged_decode(a, stream);
  KParams kp;
  Selected sel;
  SchedDecodeArgs b = *a;
  // validate first with a stand-in workspace address and an unbounded size
  // (nothing is launched): prepare checks the head counts before anything
  // divides by them, then the scratch's size is checked against the layout
  b.workspace = reinterpret_cast<void *>(uintptr_t(256));
  b.workspace_bytes = ~uint64_t(0);
  int rc = prepare(&b, &kp, &sel);
  if (rc)
    return rc;
  const WsLayout W = ws_layout(a);
  if (W.total > kScratchBytes)
    return set_error(hipErrorInvalidValue,
                     "this launch needs %llu bytes of split workspace; the no-allocation entry "
                     "point holds %llu (use sched_paged_decode with a workspace)",
                     (unsigned long long)W.total, (unsigned long long)kScratchBytes);
  int dev = 0;
  void *ptr = scratch_address(&dev);
  if (ptr == nullptr)
    return hipErrorInvalidSymbol;
  // the stale counter and this launch's arrival counters start at zero
  const uint32_t words = (uint32_t)(W.ml_off / 4u);
  const uint32_t blocks = (words + 255u) / 256u;
  hipLaunchKernelGGL(zero_words, dim3(blocks < 1024u ? blocks : 1024u), dim3(256), 0,
                     (hipStream_t)stream, static_cast<uint32_t *>(ptr), words);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(e, "scratch clear failed: %s", hipGetErrorString(e));
  b.workspace = ptr;
  b.workspace_bytes = kScratchBytes;
  return sched_paged_decode(&b, stream);
}


void sched_pd_default_args(SchedDecodeArgs *a) {
  if (!a)
    return;
  std::memset(a, 0, sizeof *a);
  a->abi_version = SCHED_PD_ABI_VERSION;
  a->kv_dtype = SCHED_PD_F32;
  a->q_dtype = SCHED_PD_F32;
  a->o_dtype = SCHED_PD_F32;
  a->tau_scope = SCHED_PD_TAU_PREFIX;
  a->max_tasks = SCHED_MAX_TASKS;
  a->policy_dT = 1.f;
  a->policy_dR = 1.f;
  a->policy_H = 0.25f;
}

// Workgroups of `fn` resident on the current device at once (occupancy x
// CUs), cached per (device, kernel); 0 if the runtime cannot say.
static uint32_t resident_blocks(const void *fn, int block) {
  static std::mutex mu;
  static std::map<std::pair<int, const void *>, uint32_t> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess)
    return 0;
  std::lock_guard<std::mutex> g(mu);
  auto it = cache.find({dev, fn});
  if (it != cache.end())
    return it->second;
  int blocks = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, block, 0) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  const uint32_t r = (uint32_t)(blocks > 0 ? blocks : 0) * (uint32_t)(cus > 0 ? cus : 0);
  cache[{dev, fn}] = r;
  return r;
}

// The step's new tokens for a fused append (sched_paged_decode_append).
struct AppendRows {
  const void *k, *v;
  int64_t ts, hs;
  bool f32, f16; // source fp32, fp16, else bf16 (16-bit caches: the cache's type)
};

static int launch_decode(const SchedDecodeArgs *a, const AppendRows *app, void *stream) {
  KParams kp;
  Selected sel;
  int rc = prepare(a, &kp, &sel);
  if (rc)
    return rc;
  if (app != nullptr) {
    if (sel.mfma == 0)
      return set_error(hipErrorInvalidValue,
                       "fused append: these arguments select the VALU kernel; the append is "
                       "fused into the MFMA and one-wave kernels only (call sched_kv_append, "
                       "then sched_paged_decode)");
    kp.app_k = app->k;
    kp.app_v = app->v;
    kp.app_ts = app->ts;
    kp.app_hs = app->hs;
    kp.app_f32 = app->f32 ? 1u : 0u;
    kp.app_f16 = app->f16 ? 1u : 0u;
  }
  const uint32_t nitems = kp.L.nitems;
  if (nitems == 0 || kp.ntasks == 0)
    return 0;
  // A work-queue launch needs the queue and ctrl tables; without them the
  // kernel's stock path serves one task per workgroup (or wave), so the grid
  // must then cover every task. For the runtime's tables the pushed num_tasks
  // is known here too (0 = the per-step disarm switch).
  bool wq = a->workers > 0 && kp.L.queue != nullptr && kp.L.ctrl != nullptr;
  if (wq && (a->flags & SCHED_PD_FLAG_RT_TABLES)) {
    const RtSnapshot s = rt_snapshot();
    if (s.num_tasks_known && s.num_tasks == 0)
      wq = false;
  }
  const uint32_t slots = wq ? a->workers : nitems;
  const uint32_t grid = (slots + sel.per_block - 1) / sel.per_block;
  kp.L.wq = wq ? 1u : 0u;
  kp.L.workers = wq ? a->workers : 0u;
  if (sel.per_block > 1 && !wq)
    kp.L.spread = min(grid, resident_blocks(reinterpret_cast<const void *>(sel.fn), sel.block));
  hipLaunchKernelGGL(sel.fn, dim3(grid), dim3(sel.block), 0, (hipStream_t)stream, kp);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(e, "kernel launch failed: %s", hipGetErrorString(e));
  if (a->flags & SCHED_PD_FLAG_RT_TABLES)
    return rt_after_launch(stream);
  return 0;
}

int sched_paged_decode(const SchedDecodeArgs *a, void *stream) {
  return launch_decode(a, nullptr, stream);
}

int sched_paged_decode_append(const SchedDecodeArgs *a, const SchedKvAppendArgs *w,
                              void *stream) {
  if (a == nullptr || w == nullptr)
    return set_error(hipErrorInvalidValue, "args is NULL");
  if (w->abi_version != SCHED_KV_ABI_VERSION)
    return set_error(hipErrorInvalidValue, "append args: abi_version %u, expected %u",
                     w->abi_version, SCHED_KV_ABI_VERSION);
  if (a->mode != SCHED_PD_SOFTMAX || (a->flags & SCHED_PD_FLAG_CTX_IN_PAGES))
    return set_error(hipErrorInvalidValue,
                     "fused append: softmax decode with ctx_lens in tokens only");
  const bool fp8 = a->kv_dtype == SCHED_PD_FP8_E4M3;
  if (a->kv_dtype != SCHED_PD_BF16 && a->kv_dtype != SCHED_PD_F16 && !fp8)
    return set_error(hipErrorInvalidValue, "fused append: bf16, fp16 or fp8 caches only");
  if (w->kv_dtype != a->kv_dtype)
    return set_error(hipErrorInvalidValue, "fused append: the cache dtypes differ");
  if (fp8 ? (w->src_dtype != SCHED_PD_F32 && w->src_dtype != SCHED_PD_BF16 &&
             w->src_dtype != SCHED_PD_F16)
          : (w->src_dtype != a->kv_dtype && w->src_dtype != SCHED_PD_F32))
    return set_error(hipErrorInvalidValue,
                     "fused append: the source must be fp32 or the cache's dtype (fp32, bf16 "
                     "or fp16 for an fp8 cache)");
  if (fp8 && (a->k_scale == nullptr || a->v_scale == nullptr || w->k_scale != a->k_scale ||
              w->v_scale != a->v_scale))
    return set_error(hipErrorInvalidValue,
                     "fused append: an fp8 cache needs its k_scale / v_scale, the same in both "
                     "argument blocks");
  if (a->head_dim != 128 || a->v_dim_stride != 1 || a->v_tok_stride % 2 ||
      a->k_tok_stride % 2 || a->k_page_stride % 2 || a->k_head_stride % 2 ||
      a->v_page_stride % 2 || a->v_head_stride % 2)
    return set_error(hipErrorInvalidValue,
                     "fused append: head dim 128, token-major V (v_dim_stride 1) and even "
                     "strides only");
  if (w->num_requests != a->num_requests || w->num_kv_heads != a->num_kv_heads ||
      w->head_dim != a->head_dim || w->page_size != a->page_size ||
      w->num_tokens != w->num_requests)
    return set_error(hipErrorInvalidValue,
                     "fused append: one token per request (num_tokens == num_requests) of the "
                     "decode's shape");
  if (w->k_pool != a->k_pool || w->v_pool != a->v_pool || w->ctx_lens != a->ctx_lens ||
      w->block_table != a->block_table || w->page_indptr != a->page_indptr ||
      (a->page_indptr == nullptr && w->bt_stride != a->bt_stride) ||
      w->k_page_stride != a->k_page_stride || w->k_head_stride != a->k_head_stride ||
      w->k_tok_stride != a->k_tok_stride || w->v_page_stride != a->v_page_stride ||
      w->v_head_stride != a->v_head_stride || w->v_tok_stride != a->v_tok_stride ||
      w->v_dim_stride != a->v_dim_stride)
    return set_error(hipErrorInvalidValue,
                     "fused append: pools, strides, page table and ctx_lens must be the "
                     "decode's");
  if (w->k_src == nullptr || w->v_src == nullptr || w->src_tok_stride % 2 ||
      w->src_head_stride % 2 || (reinterpret_cast<uintptr_t>(w->k_src) & 3u) ||
      (reinterpret_cast<uintptr_t>(w->v_src) & 3u))
    return set_error(hipErrorInvalidValue,
                     "fused append: source rows must be 4-byte aligned with even strides");
  AppendRows app{w->k_src, w->v_src, w->src_tok_stride, w->src_head_stride,
                 w->src_dtype == SCHED_PD_F32, w->src_dtype == SCHED_PD_F16};
  return launch_decode(a, &app, stream);
}

int64_t sched_paged_decode_workspace_bytes(const SchedDecodeArgs *a) {
  if (a == nullptr || a->num_kv_heads == 0 ||
      (a->mode == SCHED_PD_SOFTMAX && (a->num_q_heads == 0 || a->num_q_heads % a->num_kv_heads)))
    return -1;
  if (a->tiles == nullptr)
    return 0;
  return (int64_t)ws_layout(a).total;
}

int sched_paged_decode_occupancy(const SchedDecodeArgs *a) {
  KParams kp;
  Selected sel;
  if (prepare(a, &kp, &sel))
    return 0;
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, sel.fn, sel.block, 0) != hipSuccess)
    return 0;
  return blocks * sel.per_block;
}

int sched_paged_decode_prefetch_range(const SchedDecodeArgs *a, uint32_t *stock,
                                      uint32_t *deepest) {
  KParams kp;
  Selected sel;
  SchedDecodeArgs b;
  if (a == nullptr)
    return set_error(hipErrorInvalidValue, "args is NULL");
  b = *a;
  b.pf_dist = 0;
  // the depths of the kernel a launch with a nonzero pf_dist selects (the
  // one-wave kernel, which has no ring, gives way to the MFMA kernel then)
  b.flags |= SCHED_PD_FLAG_NO_WAVE;
  int rc = prepare(&b, &kp, &sel);
  if (rc)
    return rc;
  uint32_t ds = 0, du = 0;
  ring_depths(&b, sel.mfma == 1, &ds, &du);
  if (stock)
    *stock = ds;
  if (deepest)
    *deepest = du;
  return 0;
}

int sched_paged_decode_kernel_kind(const SchedDecodeArgs *a) {
  KParams kp;
  Selected sel;
  if (prepare(a, &kp, &sel))
    return -1;
  return sel.mfma;
}

int sched_pd_cu_count(void) {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess)
    return 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  return n;
}

// reference python/kernels/paged_softmax.cu:47-54
static void compat_args(SchedDecodeArgs *a, const void *kv, const void *bt, const void *nbl,
                        const void *q, void *out, int nseq, int bt_stride, int page_tokens) {
  sched_pd_default_args(a);
  a->mode = SCHED_PD_SOFTMAX;
  a->num_requests = nseq > 0 ? (uint32_t)nseq : 0u;
  a->num_q_heads = 1;
  a->num_kv_heads = 1;
  a->head_dim = 32;
  a->page_size = page_tokens > 0 ? (uint32_t)page_tokens : 0u;
  a->bt_stride = bt_stride > 0 ? (uint32_t)bt_stride : 0u;
  a->tau_scope = SCHED_PD_TAU_PER_PAGE;
  a->flags = SCHED_PD_FLAG_RT_TABLES | SCHED_PD_FLAG_CTX_IN_PAGES;
  a->sm_scale = 0.125f;
  a->q = q;
  a->out = out;
  a->k_pool = kv;
  a->v_pool = static_cast<const float *>(kv) + 32;
  a->k_page_stride = (int64_t)a->page_size * 64;
  a->k_tok_stride = 64;
  a->v_page_stride = (int64_t)a->page_size * 64;
  a->v_tok_stride = 64;
  a->v_dim_stride = 1;
  a->block_table = static_cast<const int32_t *>(bt);
  a->ctx_lens = static_cast<const int32_t *>(nbl);
}

void launch_paged_softmax(const void *kv, const void *bt, const void *nbl, const void *q,
                          void *out, int nseq, int bt_stride, int page_tokens, void *stream) {
  SchedDecodeArgs a;
  compat_args(&a, kv, bt, nbl, q, out, nseq, bt_stride, page_tokens);
  sched_paged_decode(&a, stream);
}

// reference python/kernels/paged_softmax.cu:61-67
int paged_softmax_occupancy(void) {
  // Any valid fixture shape selects the same kernel (fp32, d 32, MHA).
  alignas(16) static float dummy[64];
  alignas(16) static int32_t dummy_i[4];
  SchedDecodeArgs a;
  compat_args(&a, dummy, dummy_i, dummy_i, dummy, dummy, 1, 1, 16);
  a.flags &= ~SCHED_PD_FLAG_RT_TABLES;
  return sched_paged_decode_occupancy(&a);
}

} // extern "C"
