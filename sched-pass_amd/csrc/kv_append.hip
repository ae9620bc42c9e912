// kv_append.hip -- the paged KV-cache writer (sched_kv_append): appends
// source token rows into the decode pools, converting to bf16 / fp32 or
// quantising to fp8 e4m3fn with per-(page, kv-head) power-of-two scales.
//
// One workgroup serves one (request, kv-head) pair and a strided subset of
// the pages that request's append touches (grid.y covers the pages of the
// longest append, so a bulk append runs one page per workgroup). Per page it
// handles K, then V:
//   1. fp8: block max of |x| over the appended slots -> the new scale;
//   2. one pass over the page's slots [lo, o1) in storage order, four
//      elements per lane along the contiguous dimension (one 4/8/16-byte
//      store): earlier slots are re-encoded when the scale grew (fp8) or
//      kept, appended slots are converted from the source.
// Every address is bounds-checked against the pool, the page table and the
// source rows; a slot that cannot be written is counted in `errors`.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <type_traits>

#include "common.h"
#include "rt_internal.h"
#include "sched_kv.h"

using namespace schedpd;

namespace {

constexpr int kBlock = 256;

struct AParams {
  const void *k_src, *v_src;
  int64_t s_tok, s_head;
  const int32_t *app, *ctx, *table, *pind;
  uint32_t bt_stride;
  uint32_t R, Hkv, d, ps, num_tokens;
  uint64_t num_pages;
  void *k_pool, *v_pool;
  int64_t kps, khs, kts, vps, vhs, vts, vds;
  float *k_scale, *v_scale;
  uint32_t *errors;
};

template <bool SRC_F32>
__device__ __forceinline__ float load_src(const void *src, int64_t idx) {
  if (SRC_F32)
    return static_cast<const float *>(src)[idx];
  return bf16_bits_to_f32(static_cast<const uint16_t *>(src)[idx]);
}

template <bool SRC_F32>
__device__ __forceinline__ void load_src4(const void *src, int64_t idx, float x[4]) {
  if (SRC_F32) {
    float4 v = *reinterpret_cast<const float4 *>(static_cast<const float *>(src) + idx);
    x[0] = v.x, x[1] = v.y, x[2] = v.z, x[3] = v.w;
  } else {
    uint2 v = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(src) + idx);
    x[0] = __uint_as_float(v.x << 16), x[1] = __uint_as_float(v.x & 0xffff0000u);
    x[2] = __uint_as_float(v.y << 16), x[3] = __uint_as_float(v.y & 0xffff0000u);
  }
}

// Least 2^k (k >= -126) with a <= 448 * 2^k; 0 for a == 0. With
// a = m * 2^e, m in [0.5, 1): k = e - 9 when m <= 0.875 (448 = 0.875 * 2^9),
// else e - 8.
__device__ __forceinline__ float pow2_scale(float a) {
  if (!(a > 0.f))
    return 0.f;
  int e;
  float m = frexpf(a, &e);
  int k = e - 9 + (m > 0.875f ? 1 : 0);
  return ldexpf(1.f, k < -126 ? -126 : k);
}

// x * inv clamped to the e4m3fn range, round-to-nearest-even, four at once
// (byte i of the result is element i).
__device__ __forceinline__ uint32_t encode4_fp8(const float q[4]) {
  float c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    c[i] = fminf(fmaxf(q[i], -448.f), 448.f);
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(c[0], c[1], 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c[2], c[3], w, true);
  return (uint32_t)w;
}

template <int KVD> struct Codec;

template <> struct Codec<SCHED_PD_F32> {
  typedef uint4 Vec;
  __device__ static Vec enc(const float x[4], float) {
    return make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]),
                      __float_as_uint(x[3]));
  }
  __device__ static float dec(const Vec &v, int i) {
    return __uint_as_float(i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w);
  }
  // element i from `old` where bit i of keep is set, else from `v`
  __device__ static Vec keep(Vec v, const Vec &old, uint32_t keep) {
    if (keep & 1u) v.x = old.x;
    if (keep & 2u) v.y = old.y;
    if (keep & 4u) v.z = old.z;
    if (keep & 8u) v.w = old.w;
    return v;
  }
};

template <> struct Codec<SCHED_PD_BF16> {
  typedef uint2 Vec;
  __device__ static Vec enc(const float x[4], float) {
    return make_uint2((uint32_t)f32_to_bf16_rne(x[0]) | ((uint32_t)f32_to_bf16_rne(x[1]) << 16),
                      (uint32_t)f32_to_bf16_rne(x[2]) | ((uint32_t)f32_to_bf16_rne(x[3]) << 16));
  }
  __device__ static float dec(const Vec &v, int i) {
    uint32_t w = i < 2 ? v.x : v.y;
    return bf16_bits_to_f32((i & 1) ? (w >> 16) : (w & 0xffffu));
  }
  __device__ static Vec keep(Vec v, const Vec &old, uint32_t keep) {
    const uint32_t m0 = ((keep & 1u) ? 0xffffu : 0u) | ((keep & 2u) ? 0xffff0000u : 0u);
    const uint32_t m1 = ((keep & 4u) ? 0xffffu : 0u) | ((keep & 8u) ? 0xffff0000u : 0u);
    v.x = (v.x & ~m0) | (old.x & m0);
    v.y = (v.y & ~m1) | (old.y & m1);
    return v;
  }
};

template <> struct Codec<SCHED_PD_FP8_E4M3> {
  typedef uint32_t Vec;
  __device__ static Vec enc(const float x[4], float inv) {
    float q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      q[i] = x[i] * inv;
    return encode4_fp8(q);
  }
  // code value without the scale
  __device__ static float dec(const Vec &v, int i) { return fp8e4m3_to_f32((v >> (8 * i)) & 0xffu); }
  __device__ static Vec keep(Vec v, const Vec &old, uint32_t keep) {
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      m |= (keep >> i & 1u) ? 0xffu << (8 * i) : 0u;
    return (v & ~m) | (old & m);
  }
};

__device__ __forceinline__ float block_max(float v, float *red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1)
    v = fmaxf(v, __shfl_xor(v, off));
  const int w = threadIdx.x >> 6;
  __syncthreads(); // red[] may still be read by a previous call
  if ((threadIdx.x & 63) == 0)
    red[w] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int i = 1; i < kBlock / 64; ++i)
    m = fmaxf(m, red[i]);
  return m;
}

// One tensor (K or V) of one (page, head): slots [o0, o1) are appended from
// source rows row0 + (o - o0).
template <bool SRC_F32, int KVD>
__device__ void write_page(const AParams &P, const void *src, void *pool_v, int64_t base,
                           int64_t tok_stride, int64_t dim_stride, float *scale_slot,
                           uint32_t o0, uint32_t o1, int64_t row0, uint32_t h, float *red) {
  typedef Codec<KVD> C;
  typedef typename C::Vec Vec;
  typedef typename std::conditional<KVD == SCHED_PD_F32, float,
          typename std::conditional<KVD == SCHED_PD_BF16, uint16_t, uint8_t>::type>::type E;
  E *pool = static_cast<E *>(pool_v);
  const uint32_t d = P.d;
  const int64_t shead = (int64_t)h * P.s_head;

  float inv = 0.f, s_prev = 0.f;
  bool requant = false;
  if (KVD == SCHED_PD_FP8_E4M3) {
    const float s_old = *scale_slot;
    float a = 0.f;
    const uint32_t groups = (o1 - o0) * (d / 4);
    for (uint32_t g = threadIdx.x; g < groups; g += kBlock) {
      const uint32_t o = o0 + g / (d / 4), j = (g % (d / 4)) * 4;
      float x[4];
      load_src4<SRC_F32>(src, (row0 + (o - o0)) * P.s_tok + shead + j, x);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a = fmaxf(a, fabsf(x[i]));
    }
    a = block_max(a, red);
    const float p = pow2_scale(a);
    const float s_new = o0 == 0 ? p : fmaxf(s_old, p);
    requant = o0 > 0 && s_new != s_old;
    inv = s_new > 0.f ? 1.f / s_new : 0.f;
    s_prev = s_old; // re-encode: (code * s_old) * inv
    if (threadIdx.x == 0)
      *scale_slot = s_new;
  }

  if (dim_stride == 1) {
    // token rows: groups of four dims, never straddling a slot
    const uint32_t lo = requant ? 0u : o0;
    const uint32_t groups = (o1 - lo) * (d / 4);
    for (uint32_t g = threadIdx.x; g < groups; g += kBlock) {
      const uint32_t o = lo + g / (d / 4), j = (g % (d / 4)) * 4;
      Vec *dst = reinterpret_cast<Vec *>(pool + base + (int64_t)o * tok_stride + j);
      float x[4];
      if (o < o0) {
        const Vec old = *dst;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          x[i] = C::dec(old, i) * s_prev;
      } else {
        load_src4<SRC_F32>(src, (row0 + (o - o0)) * P.s_tok + shead + j, x);
      }
      *dst = C::enc(x, inv);
    }
  } else {
    // d-major: groups of four slots of one dim; slots past o1 in the last
    // group are unused positions and are written as zero
    const uint32_t lo = (requant ? 0u : o0) & ~3u;
    const uint32_t hi = (o1 + 3u) & ~3u;
    const uint32_t per_dim = (hi - lo) / 4;
    const uint32_t groups = per_dim * d;
    for (uint32_t g = threadIdx.x; g < groups; g += kBlock) {
      const uint32_t j = g / per_dim, o = lo + (g % per_dim) * 4;
      Vec *dst = reinterpret_cast<Vec *>(pool + base + (int64_t)j * dim_stride + o);
      Vec old{};
      if (o < o0)
        old = *dst;
      float x[4];
      uint32_t kept = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t t = o + i;
        if (t < o0) {
          // earlier slot: re-encoded at the grown scale, else kept bit for bit
          x[i] = requant ? C::dec(old, i) * s_prev : 0.f;
          kept |= requant ? 0u : 1u << i;
        } else if (t < o1) {
          x[i] = load_src<SRC_F32>(src, (row0 + (t - o0)) * P.s_tok + shead + j);
        } else {
          x[i] = 0.f;
        }
      }
      *dst = C::keep(C::enc(x, inv), old, kept);
    }
  }
}

template <bool SRC_F32, int KVD>
__global__ __launch_bounds__(kBlock) void kv_append_kernel(AParams P) {
  __shared__ float red[kBlock / 64];
  const uint32_t r = blockIdx.x / P.Hkv, h = blockIdx.x % P.Hkv;
  const int32_t a0 = P.app[r], a1 = P.app[r + 1];
  if (a1 <= a0)
    return;
  const int64_t n = (int64_t)a1 - a0, ctx = P.ctx[r], pos0 = ctx - n;
  if (a0 < 0 || (uint32_t)a1 > P.num_tokens || pos0 < 0) {
    if (threadIdx.x == 0 && blockIdx.y == 0 && P.errors)
      atomicAdd(P.errors, (uint32_t)n);
    return;
  }
  const int64_t row = P.pind ? (int64_t)P.pind[r] : (int64_t)r * P.bt_stride;
  const int64_t cap = P.pind ? (int64_t)P.pind[r + 1] - P.pind[r] : (int64_t)P.bt_stride;
  const int64_t b_first = pos0 / P.ps, b_last = (ctx - 1) / P.ps;
  for (int64_t b = b_first + blockIdx.y; b <= b_last; b += gridDim.y) {
    const int64_t pbase = b * P.ps;
    const uint32_t o0 = (uint32_t)(pos0 > pbase ? pos0 - pbase : 0);
    const uint32_t o1 = (uint32_t)(ctx - pbase < P.ps ? ctx - pbase : P.ps);
    const int32_t page = b < cap ? P.table[row + b] : -1;
    if (page < 0 || (uint64_t)page >= P.num_pages) {
      if (threadIdx.x == 0 && P.errors)
        atomicAdd(P.errors, o1 - o0);
      continue;
    }
    const int64_t src_row0 = a0 + (pbase + o0 - pos0);
    const int64_t sidx = (int64_t)page * P.Hkv + h;
    write_page<SRC_F32, KVD>(P, P.k_src, P.k_pool, page * P.kps + h * P.khs, P.kts, 1,
                             P.k_scale ? P.k_scale + sidx : nullptr, o0, o1, src_row0, h, red);
    write_page<SRC_F32, KVD>(P, P.v_src, P.v_pool, page * P.vps + h * P.vhs, P.vts, P.vds,
                             P.v_scale ? P.v_scale + sidx : nullptr, o0, o1, src_row0, h, red);
  }
}

typedef void (*AppendFn)(AParams);

template <bool SRC_F32> AppendFn pick(uint32_t kvd) {
  switch (kvd) {
  case SCHED_PD_F32: return kv_append_kernel<SRC_F32, SCHED_PD_F32>;
  case SCHED_PD_BF16: return kv_append_kernel<SRC_F32, SCHED_PD_BF16>;
  default: return kv_append_kernel<SRC_F32, SCHED_PD_FP8_E4M3>;
  }
}

uint32_t esize(uint32_t dt) { return dt == SCHED_PD_F32 ? 4u : dt == SCHED_PD_BF16 ? 2u : 1u; }

bool aligned(const void *p, uint32_t bytes) { return ((uintptr_t)p % bytes) == 0; }

bool mult4(int64_t s) { return s % 4 == 0; }

} // namespace

extern "C" {

void sched_kv_default_args(SchedKvAppendArgs *a) {
  if (!a)
    return;
  *a = SchedKvAppendArgs{};
  a->abi_version = SCHED_KV_ABI_VERSION;
  a->src_dtype = SCHED_PD_BF16;
  a->kv_dtype = SCHED_PD_BF16;
}

int sched_kv_append(const SchedKvAppendArgs *a, void *stream) {
  if (!a)
    return set_error(-1, "sched_kv_append: args is NULL");
  if (a->abi_version != SCHED_KV_ABI_VERSION)
    return set_error(-1, "sched_kv_append: abi_version %u, library has %u", a->abi_version,
                     SCHED_KV_ABI_VERSION);
  if (a->src_dtype != SCHED_PD_F32 && a->src_dtype != SCHED_PD_BF16)
    return set_error(-1, "sched_kv_append: src dtype %u (F32 or BF16)", a->src_dtype);
  if (a->kv_dtype > SCHED_PD_FP8_E4M3)
    return set_error(-1, "sched_kv_append: kv dtype %u", a->kv_dtype);
  if (a->num_requests == 0)
    return 0;
  if (a->num_kv_heads == 0 || (uint64_t)a->num_requests * a->num_kv_heads > 0x7fffffffu)
    return set_error(-1, "sched_kv_append: num_kv_heads %u", a->num_kv_heads);
  if (a->head_dim == 0 || a->head_dim % 4 || a->head_dim > 256)
    return set_error(-1, "sched_kv_append: head_dim %u (multiple of 4, <= 256)", a->head_dim);
  if (a->page_size == 0 || a->page_size % 4 || a->page_size > 256)
    return set_error(-1, "sched_kv_append: page_size %u (multiple of 4, <= 256)", a->page_size);
  if (!a->k_src || !a->v_src || !a->append_indptr || !a->ctx_lens || !a->block_table ||
      !a->k_pool || !a->v_pool)
    return set_error(-1, "sched_kv_append: a required pointer is NULL");
  if (a->kv_dtype == SCHED_PD_FP8_E4M3 && (!a->k_scale || !a->v_scale))
    return set_error(-1, "sched_kv_append: an fp8 cache needs k_scale and v_scale");
  if (!a->page_indptr && a->bt_stride == 0)
    return set_error(-1, "sched_kv_append: bt_stride is 0 with a 2-D block table");
  if (a->num_pages == 0 || a->num_pages > 0x7fffffffull)
    return set_error(-1, "sched_kv_append: num_pages %llu", (unsigned long long)a->num_pages);
  if (a->v_tok_stride != 1 && a->v_dim_stride != 1)
    return set_error(-1, "sched_kv_append: V needs v_tok_stride == 1 (d-major) or "
                         "v_dim_stride == 1 (token-major)");
  const bool vdm = a->v_tok_stride == 1 && a->v_dim_stride != 1;
  const int64_t v_other = vdm ? a->v_dim_stride : a->v_tok_stride;
  const uint32_t se = esize(a->src_dtype), ke = esize(a->kv_dtype);
  if (!mult4(a->src_tok_stride) || !mult4(a->src_head_stride) || !mult4(a->k_page_stride) ||
      !mult4(a->k_head_stride) || !mult4(a->k_tok_stride) || !mult4(a->v_page_stride) ||
      !mult4(a->v_head_stride) || !mult4(v_other) || !aligned(a->k_src, 4 * se) ||
      !aligned(a->v_src, 4 * se) || !aligned(a->k_pool, 4 * ke) || !aligned(a->v_pool, 4 * ke))
    return set_error(-1, "sched_kv_append: strides must be multiples of 4 elements and "
                         "pointers aligned to 4 elements (4-wide stores)");
  if (a->src_tok_stride <= 0 || a->src_head_stride < 0)
    return set_error(-1, "sched_kv_append: source strides");

  AParams P{};
  P.k_src = a->k_src, P.v_src = a->v_src;
  P.s_tok = a->src_tok_stride, P.s_head = a->src_head_stride;
  P.app = a->append_indptr, P.ctx = a->ctx_lens, P.table = a->block_table, P.pind = a->page_indptr;
  P.bt_stride = a->bt_stride;
  P.R = a->num_requests, P.Hkv = a->num_kv_heads, P.d = a->head_dim, P.ps = a->page_size;
  P.num_tokens = a->num_tokens;
  P.num_pages = a->num_pages;
  P.k_pool = a->k_pool, P.v_pool = a->v_pool;
  P.kps = a->k_page_stride, P.khs = a->k_head_stride, P.kts = a->k_tok_stride;
  P.vps = a->v_page_stride, P.vhs = a->v_head_stride;
  P.vts = vdm ? 1 : a->v_tok_stride;
  P.vds = vdm ? a->v_dim_stride : 1;
  P.k_scale = a->kv_dtype == SCHED_PD_FP8_E4M3 ? a->k_scale : nullptr;
  P.v_scale = a->kv_dtype == SCHED_PD_FP8_E4M3 ? a->v_scale : nullptr;
  P.errors = a->errors;

  const uint32_t max_app = a->max_append ? a->max_append : a->num_tokens;
  uint64_t gy = (uint64_t)(max_app + a->page_size - 1) / a->page_size + 1;
  if (gy > 65535)
    gy = 65535;
  const dim3 grid(a->num_requests * a->num_kv_heads, (uint32_t)gy);
  AppendFn fn = a->src_dtype == SCHED_PD_F32 ? pick<true>(a->kv_dtype) : pick<false>(a->kv_dtype);
  hipLaunchKernelGGL(fn, grid, dim3(kBlock), 0, static_cast<hipStream_t>(stream), P);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(-1, "sched_kv_append: launch failed: %s", hipGetErrorString(e));
  return 0;
}

} // extern "C"
