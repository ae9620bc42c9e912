// kv_append.hip -- the paged KV-cache writer (sched_kv_append): appends
// source token rows (fp32, bf16 or fp16) into the decode pools, converting to
// fp32 / bf16 / fp16 (round to nearest even) or quantising to fp8 e4m3fn
// with per-(page, kv-head) power-of-two scales.
//
// One workgroup serves one request and a group of its kv-heads (all of them
// unless a small append needs more workgroups), over a strided subset of the
// pages the append touches (grid.y covers the pages of the longest append,
// so a bulk append runs one page per workgroup). A page whose appended
// elements fit one round (16 per lane and tensor) is written by
// page_one_round: each lane loads its K and V chunks once (8 or 4 elements
// each), keeps them in registers through the fp8 amax and stores them, a
// d-major V going through an LDS stage (a whole page leaves it as 16-slot
// dim rows, a partial one as 4-slot groups). Larger pages take two passes:
//   1. fp8: max |x| of each head's appended K and V slots (LDS atomics, one
//      per wave when its lanes share a head) -> the new scales;
//   2. K, then V: one pass over the group's slots in storage order, four
//      elements per lane along the contiguous dimension (one 4/8/16-byte
//      store).
// Either way earlier slots are re-encoded when their head's scale grew (fp8)
// or left as they are, and appended slots are converted from the source.
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
  uint32_t scale_stride; // 2 when K and V scales are interleaved (v_scale == k_scale + 1)
  uint32_t *errors;
  uint32_t hpw; // kv-heads per workgroup, divides Hkv
  uint32_t w8;  // one-round path reads and writes 8-element chunks
  uint32_t vrow16; // d-major V rows start 16-element aligned (16-slot row stores)
};

// Source rows are fp32, bf16 or fp16 (SRC is the SCHED_PD_* code).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

template <int SRC> __device__ __forceinline__ float half_to_f32(uint32_t h) {
  if constexpr (SRC == SCHED_PD_BF16)
    return bf16_bits_to_f32(h);
  else
    return f16_bits_to_f32(h);
}

template <int SRC>
__device__ __forceinline__ float load_src(const void *src, int64_t idx) {
  if constexpr (SRC == SCHED_PD_F32)
    return static_cast<const float *>(src)[idx];
  else
    return half_to_f32<SRC>(static_cast<const uint16_t *>(src)[idx]);
}

typedef __attribute__((ext_vector_type(4))) unsigned u32x4_t;
typedef __attribute__((ext_vector_type(2))) unsigned u32x2_t;

// Source rows are read once: non-temporal loads (bulk bf16 append measured
// 280 -> 252 us).
template <int SRC>
__device__ __forceinline__ void load_src4(const void *src, int64_t idx, float x[4]) {
  if constexpr (SRC == SCHED_PD_F32) {
    const u32x4_t v = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4_t *>(static_cast<const float *>(src) + idx));
    x[0] = __uint_as_float(v.x), x[1] = __uint_as_float(v.y);
    x[2] = __uint_as_float(v.z), x[3] = __uint_as_float(v.w);
  } else {
    const u32x2_t v = __builtin_nontemporal_load(
        reinterpret_cast<const u32x2_t *>(static_cast<const uint16_t *>(src) + idx));
    x[0] = half_to_f32<SRC>(v.x & 0xffffu), x[1] = half_to_f32<SRC>(v.x >> 16);
    x[2] = half_to_f32<SRC>(v.y & 0xffffu), x[3] = half_to_f32<SRC>(v.y >> 16);
  }
}

// W consecutive source elements as loaded: fp32 words, or 16-bit codes in
// pairs, which hold a chunk in half the registers while it waits for its
// page's fp8 scale. Elements convert to float where they are used.
template <int SRC, int W> struct Chunk {
  static constexpr int N = SRC == SCHED_PD_F32 ? W : W / 2;
  uint32_t w[N];
  __device__ __forceinline__ float operator[](int i) const {
    if constexpr (SRC == SCHED_PD_F32)
      return __uint_as_float(w[i]);
    else
      return half_to_f32<SRC>((i & 1) ? (w[i >> 1] >> 16) : (w[i >> 1] & 0xffffu));
  }
  __device__ __forceinline__ void to_float(float x[W]) const {
#pragma unroll
    for (int i = 0; i < W; ++i)
      x[i] = (*this)[i];
  }
  // Conversions made before this point are not reused after it (the
  // compiler would otherwise keep the converted floats live instead of the
  // packed codes). No instruction is emitted.
  __device__ __forceinline__ void reload() {
#pragma unroll
    for (int k = 0; k < N; ++k)
      asm volatile("" : "+v"(w[k]));
  }
};

template <int SRC, int W>
__device__ __forceinline__ void load_chunk(const void *src, int64_t idx, Chunk<SRC, W> &c) {
  typedef Chunk<SRC, W> C;
  if constexpr (C::N == 8) {
    const float *p = static_cast<const float *>(src) + idx;
    const u32x4_t a = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
    const u32x4_t b = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p + 4));
    c.w[0] = a.x, c.w[1] = a.y, c.w[2] = a.z, c.w[3] = a.w;
    c.w[4] = b.x, c.w[5] = b.y, c.w[6] = b.z, c.w[7] = b.w;
  } else if constexpr (C::N == 4) {
    const u32x4_t a = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(
        static_cast<const char *>(src) + idx * (SRC == SCHED_PD_F32 ? 4 : 2)));
    c.w[0] = a.x, c.w[1] = a.y, c.w[2] = a.z, c.w[3] = a.w;
  } else {
    static_assert(C::N == 2, "chunk width");
    const u32x2_t a = __builtin_nontemporal_load(
        reinterpret_cast<const u32x2_t *>(static_cast<const uint16_t *>(src) + idx));
    c.w[0] = a.x, c.w[1] = a.y;
  }
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
    return make_uint2(pack_bf16_rne(x[0], x[1]), pack_bf16_rne(x[2], x[3]));
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

// IEEE binary16, round to nearest even (magnitudes from 65520 up become
// infinity, as a cast does).
template <> struct Codec<SCHED_PD_F16> {
  typedef uint2 Vec;
  __device__ static Vec enc(const float x[4], float) {
    return make_uint2(pack_f16_rne(x[0], x[1]), pack_f16_rne(x[2], x[3]));
  }
  __device__ static float dec(const Vec &v, int i) {
    uint32_t w = i < 2 ? v.x : v.y;
    return f16_bits_to_f32((i & 1) ? (w >> 16) : (w & 0xffffu));
  }
  __device__ static Vec keep(Vec v, const Vec &old, uint32_t keep) {
    return Codec<SCHED_PD_BF16>::keep(v, old, keep);
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

constexpr uint32_t kMaxGroup = 64; // kv-heads one workgroup serves at most

// Per-head fp8 state of the page being written, for K (0) and V (1).
struct PageScales {
  uint32_t amax[2][kMaxGroup]; // max |x| as bits (non-negative floats order as integers)
  float inv[2][kMaxGroup];     // 1 / new scale, 0 for a zero scale
  float prev[2][kMaxGroup];    // old scale, to re-encode earlier slots
  uint32_t regrow[2][kMaxGroup];
  uint32_t any_regrow[2];
};

template <int KVD>
using PoolElem = typename std::conditional<
    KVD == SCHED_PD_F32, float,
    typename std::conditional<KVD == SCHED_PD_BF16 || KVD == SCHED_PD_F16, uint16_t,
                              uint8_t>::type>::type;

// max into an LDS slot per head (all lanes active). When a head's chunks
// are at least a wave long, a wave's lanes hold at most two consecutive
// heads: two wave maxima and one or two atomics per wave. Otherwise one
// atomic per lane.
__device__ __forceinline__ void lds_max(uint32_t *slots, uint32_t hh, float v, bool wide) {
  if (!wide) {
    atomicMax(&slots[hh], __float_as_uint(v));
    return;
  }
  const uint32_t h_lo = __builtin_amdgcn_readfirstlane(hh);
  const bool two = __builtin_amdgcn_ballot_w64(hh != h_lo) != 0;
  const float lo = wave_max(hh == h_lo ? v : 0.f);
  const float hi = two ? wave_max(hh == h_lo ? 0.f : v) : 0.f;
  if ((threadIdx.x & 63) == 0) {
    atomicMax(&slots[h_lo], __float_as_uint(lo));
    if (two)
      atomicMax(&slots[h_lo + 1], __float_as_uint(hi));
  }
}

// Chunks in flight per lane: every lane issues the loads of kBatch chunks
// before any store, so a workgroup keeps kBatch x 256 loads outstanding (a
// store to the pool may alias the source as far as the compiler knows, so
// it would not hoist the next load above it by itself).
#ifndef SCHED_KV_BATCH
#define SCHED_KV_BATCH 4
#endif
constexpr uint32_t kBatch = SCHED_KV_BATCH;

// fp8: the new scale of each (page, head) of the group from the appended
// slots [o0, o1), written back; per-head encode state into S.
__device__ void clear_amax(PageScales &S, uint32_t hpw) {
  __syncthreads(); // S may still be read for the previous page
  for (uint32_t i = threadIdx.x; i < 2 * hpw; i += kBlock)
    S.amax[i / hpw][i % hpw] = 0u;
  if (threadIdx.x < 2)
    S.any_regrow[threadIdx.x] = 0u;
  __syncthreads();
}

// One (page, head)'s new scale from its amax (written back), its encode
// state in S; the amax slot is left at zero for the next page.
__device__ __forceinline__ void set_scale(PageScales &S, uint32_t x, uint32_t hh, float *slot,
                                          float s_old, uint32_t o0) {
  const float p = pow2_scale(__uint_as_float(S.amax[x][hh]));
  S.amax[x][hh] = 0u;
  const float s_new = o0 == 0 ? p : fmaxf(s_old, p);
  const uint32_t rq = (o0 > 0 && s_new != s_old) ? 1u : 0u;
  S.inv[x][hh] = s_new > 0.f ? 1.f / s_new : 0.f;
  S.prev[x][hh] = s_old;
  S.regrow[x][hh] = rq;
  if (rq)
    S.any_regrow[x] = 1u;
  *slot = s_new;
}

// After the amax pass: each (page, head)'s new scale (written back) and its
// encode state in S.
__device__ void scales_from_amax(const AParams &P, PageScales &S, int64_t page, uint32_t h0,
                                 uint32_t hpw, uint32_t o0) {
  __syncthreads();
  for (uint32_t i = threadIdx.x; i < 2 * hpw; i += kBlock) {
    const uint32_t x = i / hpw, hh = i % hpw;
    float *slot = (x ? P.v_scale : P.k_scale) + (page * P.Hkv + h0 + hh) * P.scale_stride;
    set_scale(S, x, hh, slot, *slot, o0);
  }
  __syncthreads();
}

template <int SRC>
__device__ void page_scales(const AParams &P, PageScales &S, int64_t page, uint32_t h0,
                            uint32_t hpw, uint32_t o0, uint32_t o1, int64_t row0) {
  const uint32_t q = P.d / 4, per_head = (o1 - o0) * q, total = hpw * per_head;
  clear_amax(S, hpw);
  for (uint32_t c0 = 0; c0 < total; c0 += kBlock * kBatch) {
    float xk[kBatch][4], xv[kBatch][4];
    uint32_t hh[kBatch];
#pragma unroll
    for (uint32_t u = 0; u < kBatch; ++u) {
      const uint32_t c = c0 + u * kBlock + threadIdx.x;
      hh[u] = hpw - 1; // lanes past the end add 0 to the last head
#pragma unroll
      for (int i = 0; i < 4; ++i)
        xk[u][i] = xv[u][i] = 0.f;
      if (c < total) {
        hh[u] = c / per_head;
        const uint32_t rem = c - hh[u] * per_head;
        const uint32_t t = rem / q, j = (rem - t * q) * 4;
        const int64_t s = (row0 + t) * P.s_tok + (int64_t)(h0 + hh[u]) * P.s_head + j;
        load_src4<SRC>(P.k_src, s, xk[u]);
        load_src4<SRC>(P.v_src, s, xv[u]);
      }
    }
#pragma unroll
    for (uint32_t u = 0; u < kBatch; ++u) {
      float mk = 0.f, mv = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        mk = fmaxf(mk, fabsf(xk[u][i]));
        mv = fmaxf(mv, fabsf(xv[u][i]));
      }
      lds_max(S.amax[0], hh[u], mk, per_head >= 64);
      lds_max(S.amax[1], hh[u], mv, per_head >= 64);
    }
  }
  scales_from_amax(P, S, page, h0, hpw, o0);
}

// One tensor (K: x = 0, V: x = 1) of heads [h0, h0 + hpw) of one page:
// slots [o0, o1) appended from source rows row0 + (t - o0); with fp8, the
// earlier slots of heads whose scale grew are re-encoded.
template <int SRC, int KVD>
__device__ void write_tensor(const AParams &P, const PageScales &S, int x, const void *src,
                             void *pool_v, int64_t base, int64_t head_stride, int64_t tok_stride,
                             int64_t dim_stride, uint32_t h0, uint32_t hpw, uint32_t o0,
                             uint32_t o1, int64_t row0) {
  typedef Codec<KVD> C;
  typedef typename C::Vec Vec;
  constexpr bool FP8 = KVD == SCHED_PD_FP8_E4M3;
  PoolElem<KVD> *pool = static_cast<PoolElem<KVD> *>(pool_v) + base;
  const uint32_t d = P.d, lo = (FP8 && S.any_regrow[x]) ? 0u : o0;

  if (dim_stride == 1) {
    // token rows: chunks of four dims, never straddling a slot
    const uint32_t q = d / 4, per_head = (o1 - lo) * q, total = hpw * per_head;
    for (uint32_t c0 = 0; c0 < total; c0 += kBlock * kBatch) {
      Vec *dst[kBatch];
      Vec old[kBatch];
      float v[kBatch][4];
      uint32_t state[kBatch]; // 0 skip, 1 append, 2 re-encode
      uint32_t hh[kBatch];
#pragma unroll
      for (uint32_t u = 0; u < kBatch; ++u) {
        const uint32_t c = c0 + u * kBlock + threadIdx.x;
        state[u] = 0;
        hh[u] = 0;
        dst[u] = nullptr;
        if (c < total) {
          hh[u] = c / per_head;
          const uint32_t rem = c - hh[u] * per_head;
          const uint32_t t = lo + rem / q, j = (rem % q) * 4;
          dst[u] = reinterpret_cast<Vec *>(pool + (int64_t)(h0 + hh[u]) * head_stride +
                                           (int64_t)t * tok_stride + j);
          if (t >= o0) {
            state[u] = 1;
            load_src4<SRC>(
                src, (row0 + (t - o0)) * P.s_tok + (int64_t)(h0 + hh[u]) * P.s_head + j, v[u]);
          } else if (FP8 && S.regrow[x][hh[u]]) {
            state[u] = 2;
            old[u] = *dst[u];
          }
        }
      }
#pragma unroll
      for (uint32_t u = 0; u < kBatch; ++u) {
        if (!state[u])
          continue;
        if (state[u] == 2) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            v[u][i] = C::dec(old[u], i) * S.prev[x][hh[u]];
        }
        *dst[u] = C::enc(v[u], FP8 ? S.inv[x][hh[u]] : 0.f);
      }
    }
  } else {
    // d-major: chunks of four slots of one dim; slots past o1 in the last
    // chunk are unused positions and are written as zero
    const uint32_t lo4 = lo & ~3u, hi4 = (o1 + 3u) & ~3u;
    const uint32_t per_dim = (hi4 - lo4) / 4, per_head = per_dim * d, total = hpw * per_head;
    for (uint32_t c0 = 0; c0 < total; c0 += kBlock * kBatch) {
      Vec *dst[kBatch];
      Vec old[kBatch];
      float v[kBatch][4];
      uint32_t kept[kBatch], hh[kBatch], o[kBatch];
      bool act[kBatch], rq[kBatch];
#pragma unroll
      for (uint32_t u = 0; u < kBatch; ++u) {
        const uint32_t c = c0 + u * kBlock + threadIdx.x;
        act[u] = false;
        rq[u] = false;
        kept[u] = 0;
        hh[u] = 0;
        o[u] = 0;
        dst[u] = nullptr;
        old[u] = Vec{};
        if (c < total) {
          hh[u] = c / per_head;
          const uint32_t rem = c - hh[u] * per_head;
          const uint32_t j = rem / per_dim;
          o[u] = lo4 + (rem % per_dim) * 4;
          rq[u] = FP8 && S.regrow[x][hh[u]];
          act[u] = o[u] + 3u >= o0 || rq[u]; // else four earlier slots, kept as they are
          if (act[u]) {
            dst[u] = reinterpret_cast<Vec *>(pool + (int64_t)(h0 + hh[u]) * head_stride +
                                             (int64_t)j * dim_stride + o[u]);
            if (o[u] < o0)
              old[u] = *dst[u];
            const int64_t s = (int64_t)(h0 + hh[u]) * P.s_head + j;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const uint32_t t = o[u] + i;
              v[u][i] = (t >= o0 && t < o1) ? load_src<SRC>(src, (row0 + (t - o0)) * P.s_tok + s)
                                            : 0.f;
            }
          }
        }
      }
#pragma unroll
      for (uint32_t u = 0; u < kBatch; ++u) {
        if (!act[u])
          continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (o[u] + i < o0) {
            // earlier slot: re-encoded at the grown scale, else kept bit for bit
            if (rq[u])
              v[u][i] = C::dec(old[u], i) * S.prev[x][hh[u]];
            else
              kept[u] |= 1u << i;
          }
        }
        *dst[u] = C::keep(C::enc(v[u], FP8 ? S.inv[x][hh[u]] : 0.f), old[u], kept[u]);
      }
    }
  }
}

// A W-element chunk of token-row dims, encoded and stored (one 4/8/16-byte
// store for W = 4; W = 8 stores 8/16/32 bytes as one or two stores).
template <int KVD, int W>
__device__ __forceinline__ void store_chunk(PoolElem<KVD> *p, const float x[W], float inv) {
  typedef Codec<KVD> C;
  typedef typename C::Vec Vec;
  if constexpr (W == 4) {
    *reinterpret_cast<Vec *>(p) = C::enc(x, inv);
  } else {
    const Vec a = C::enc(x, inv), b = C::enc(x + 4, inv);
    if constexpr (KVD == SCHED_PD_BF16 || KVD == SCHED_PD_F16)
      *reinterpret_cast<uint4 *>(p) = make_uint4(a.x, a.y, b.x, b.y);
    else if constexpr (KVD == SCHED_PD_FP8_E4M3)
      *reinterpret_cast<uint2 *>(p) = make_uint2(a, b);
    else {
      reinterpret_cast<Vec *>(p)[0] = a;
      reinterpret_cast<Vec *>(p)[1] = b;
    }
  }
}

// Slots [o, o + 16) of one d-major V dim row, encoded and stored as 16-byte
// stores (the row start is 16-element aligned).
template <int KVD>
__device__ __forceinline__ void store_row16(PoolElem<KVD> *p, const float v[16], float inv) {
  typedef Codec<KVD> C;
  typename C::Vec e[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    e[q] = C::enc(v + 4 * q, inv);
  uint4 *d = reinterpret_cast<uint4 *>(p);
  if constexpr (KVD == SCHED_PD_FP8_E4M3) {
    d[0] = make_uint4(e[0], e[1], e[2], e[3]);
  } else if constexpr (KVD == SCHED_PD_F32) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      d[q] = e[q];
  } else {
    d[0] = make_uint4(e[0].x, e[0].y, e[1].x, e[1].y);
    d[1] = make_uint4(e[2].x, e[2].y, e[3].x, e[3].y);
  }
}

// Chunks one lane holds in the one-round path, and the LDS stage that
// transposes a d-major V: rows (head, appended slot) of d floats, padded by
// one float so the four slot rows a chunk reads fall in different banks.
constexpr uint32_t kFastChunks = kBlock * kBatch;
constexpr uint32_t kStageFloats = kFastChunks * 4 + kFastChunks;

// Re-encodes slots [0, o0) of token rows for the heads whose scale grew.
template <int KVD>
__device__ void regrow_rows(const AParams &P, const PageScales &S, int x, PoolElem<KVD> *pool,
                            int64_t head_stride, int64_t tok_stride, uint32_t h0, uint32_t hpw,
                            uint32_t o0) {
  typedef Codec<KVD> C;
  typedef typename C::Vec Vec;
  const uint32_t q = P.d / 4, per_head = o0 * q, total = hpw * per_head;
  for (uint32_t c = threadIdx.x; c < total; c += kBlock) {
    const uint32_t hh = c / per_head, rem = c - hh * per_head;
    if (!S.regrow[x][hh])
      continue;
    const uint32_t t = rem / q, j = (rem - t * q) * 4;
    Vec *dst = reinterpret_cast<Vec *>(pool + (int64_t)(h0 + hh) * head_stride +
                                       (int64_t)t * tok_stride + j);
    const Vec old = *dst;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      v[i] = C::dec(old, i) * S.prev[x][hh];
    *dst = C::enc(v, S.inv[x][hh]);
  }
}

// One page of a head group whose appended elements (per tensor) fit one
// round: every lane loads its K and V chunks of W elements once (16 values
// per lane and tensor), keeps them in registers through the fp8 amax, and
// stores them; a d-major V goes through the LDS stage so that the source is
// read in rows and the pool written in slot groups.
template <int SRC, int KVD, int W>
__device__ void page_one_round(const AParams &P, PageScales &S, float *stage, int64_t page,
                               uint32_t h0, uint32_t hpw, uint32_t o0, uint32_t o1,
                               int64_t row0) {
  typedef Codec<KVD> C;
  typedef typename C::Vec Vec;
  constexpr bool FP8 = KVD == SCHED_PD_FP8_E4M3;
  static_assert(W == 4 || (W == 8 && kBatch % 2 == 0), "chunk width");
  constexpr uint32_t NB = kBatch * 4 / W; // chunks per lane and tensor
  const uint32_t d = P.d, q = d / W, nn = o1 - o0, per_head = nn * q, total = hpw * per_head;
  const bool vdm = P.vds != 1;
  const uint32_t row_len = d + 1;
  // fp8: lanes [0, hpw) own the K scales of the group, [hpw, 2 hpw) the V
  // scales; the old values load together with the source
  float *slot = nullptr, s_old = 0.f;
  if (FP8 && threadIdx.x < 2 * hpw) {
    slot = (threadIdx.x < hpw ? P.k_scale : P.v_scale) +
           (page * P.Hkv + h0 + threadIdx.x % hpw) * P.scale_stride;
    s_old = *slot;
  }
  Chunk<SRC, W> xk[NB], xv[NB];
  uint32_t hh[NB], t[NB], j[NB];
#pragma unroll
  for (uint32_t u = 0; u < NB; ++u) {
    const uint32_t c = u * kBlock + threadIdx.x;
    hh[u] = hpw - 1; // lanes past the end add 0 to the last head
    t[u] = j[u] = 0;
#pragma unroll
    for (int k = 0; k < Chunk<SRC, W>::N; ++k)
      xk[u].w[k] = xv[u].w[k] = 0u;
    if (c < total) {
      hh[u] = c / per_head;
      const uint32_t rem = c - hh[u] * per_head;
      t[u] = rem / q;
      j[u] = (rem - t[u] * q) * W;
      const int64_t s = (row0 + t[u]) * P.s_tok + (int64_t)(h0 + hh[u]) * P.s_head + j[u];
      load_chunk<SRC, W>(P.k_src, s, xk[u]);
      load_chunk<SRC, W>(P.v_src, s, xv[u]);
    }
  }
  __syncthreads(); // the stage and S are free: the previous page is written
  if (FP8 && threadIdx.x == 0)
    S.any_regrow[0] = S.any_regrow[1] = 0u;
  if (vdm) {
    // d-major V: stage the appended rows for the slot-group writes below
#pragma unroll
    for (uint32_t u = 0; u < NB; ++u) {
      if (u * kBlock + threadIdx.x < total) {
        float *row = stage + (hh[u] * nn + t[u]) * row_len + j[u];
#pragma unroll
        for (int i = 0; i < W; ++i)
          row[i] = xv[u][i];
      }
    }
  }
  if (FP8) {
    // per lane, a running max over its chunks of one head; flushed to LDS
    // when some lane's next chunk starts a new head, and at the end
    const bool wide = per_head >= 64;
    float mk = 0.f, mv = 0.f;
    uint32_t h_run = hh[0];
#pragma unroll
    for (uint32_t u = 0; u < NB; ++u) {
      if (u > 0 && __builtin_amdgcn_ballot_w64(hh[u] != h_run) != 0) {
        lds_max(S.amax[0], h_run, mk, wide);
        lds_max(S.amax[1], h_run, mv, wide);
        mk = mv = 0.f;
        h_run = hh[u];
      }
#pragma unroll
      for (int i = 0; i < W; ++i) {
        mk = fmaxf(mk, fabsf(xk[u][i]));
        mv = fmaxf(mv, fabsf(xv[u][i]));
      }
    }
    lds_max(S.amax[0], h_run, mk, wide);
    lds_max(S.amax[1], h_run, mv, wide);
  }
  __syncthreads();
  if (FP8) {
    if (slot)
      set_scale(S, threadIdx.x / hpw, threadIdx.x % hpw, slot, s_old, o0);
    __syncthreads();
  }

  // K: token rows
#pragma unroll
  for (uint32_t u = 0; u < NB; ++u) {
    xk[u].reload();
    xv[u].reload();
  }
  PoolElem<KVD> *kpool = static_cast<PoolElem<KVD> *>(P.k_pool) + page * P.kps;
#pragma unroll
  for (uint32_t u = 0; u < NB; ++u) {
    if (u * kBlock + threadIdx.x < total) {
      float x[W];
      xk[u].to_float(x);
      store_chunk<KVD, W>(kpool + (int64_t)(h0 + hh[u]) * P.khs + (int64_t)(o0 + t[u]) * P.kts +
                              j[u],
                          x, FP8 ? S.inv[0][hh[u]] : 0.f);
    }
  }
  if (FP8 && S.any_regrow[0])
    regrow_rows<KVD>(P, S, 0, kpool, P.khs, P.kts, h0, hpw, o0);

  PoolElem<KVD> *vpool = static_cast<PoolElem<KVD> *>(P.v_pool) + page * P.vps;
  if (!vdm) {
    // token-major V: as K
#pragma unroll
    for (uint32_t u = 0; u < NB; ++u) {
      if (u * kBlock + threadIdx.x < total) {
        float x[W];
        xv[u].to_float(x);
        store_chunk<KVD, W>(vpool + (int64_t)(h0 + hh[u]) * P.vhs +
                                (int64_t)(o0 + t[u]) * P.vts + j[u],
                            x, FP8 ? S.inv[1][hh[u]] : 0.f);
      }
    }
    if (FP8 && S.any_regrow[1])
      regrow_rows<KVD>(P, S, 1, vpool, P.vhs, P.vts, h0, hpw, o0);
    return;
  }

  if (o0 == 0 && o1 == P.ps && P.vrow16) {
    // d-major V, the whole page (no earlier slot to keep or re-encode): one
    // item is 16 slots of one dim row, read down a stage column
    const uint32_t rows = P.ps / 16, vper_head = d * rows, vtotal = hpw * vper_head;
    for (uint32_t c = threadIdx.x; c < vtotal; c += kBlock) {
      const uint32_t g = c / vper_head, rem = c - g * vper_head, jj = rem / rows;
      const uint32_t o = (rem - jj * rows) * 16;
      float v[16];
#pragma unroll
      for (int i = 0; i < 16; ++i)
        v[i] = stage[(g * nn + o + i) * row_len + jj];
      store_row16<KVD>(vpool + (int64_t)(h0 + g) * P.vhs + (int64_t)jj * P.vds + o, v,
                       FP8 ? S.inv[1][g] : 0.f);
    }
    return;
  }

  // d-major V: groups of four slots from the stage
  const uint32_t lo4 = ((FP8 && S.any_regrow[1]) ? 0u : o0) & ~3u, hi4 = (o1 + 3u) & ~3u;
  const uint32_t per_dim = (hi4 - lo4) / 4, vper_head = per_dim * d, vtotal = hpw * vper_head;
  for (uint32_t c = threadIdx.x; c < vtotal; c += kBlock) {
    const uint32_t g = c / vper_head, rem = c - g * vper_head;
    const uint32_t jj = rem / per_dim, o = lo4 + (rem - jj * per_dim) * 4;
    const bool rq = FP8 && S.regrow[1][g];
    if (o + 3u < o0 && !rq)
      continue; // four earlier slots, kept as they are
    Vec *dst = reinterpret_cast<Vec *>(vpool + (int64_t)(h0 + g) * P.vhs +
                                       (int64_t)jj * P.vds + o);
    Vec old{};
    if (o < o0)
      old = *dst;
    float v[4];
    uint32_t kept = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t ts = o + i;
      if (ts < o0) {
        v[i] = rq ? C::dec(old, i) * S.prev[1][g] : 0.f;
        kept |= rq ? 0u : 1u << i;
      } else if (ts < o1) {
        v[i] = stage[(g * nn + (ts - o0)) * row_len + jj];
      } else {
        v[i] = 0.f;
      }
    }
    *dst = C::keep(C::enc(v, FP8 ? S.inv[1][g] : 0.f), old, kept);
  }
}

// grid.x = requests x head groups, grid.y strides over the pages of the
// longest append. ONE: the host has checked that a whole page of the group
// fits one round, so the two-pass code is left out (it sets the register
// count of the kernel: 93 -> 74 VGPRs for fp8, 73 -> 57 for bf16).
template <int SRC, int KVD, bool ONE>
__global__ __launch_bounds__(kBlock) void kv_append_kernel(AParams P) {
  __shared__ PageScales S;
  __shared__ float stage[kStageFloats];
  if (KVD == SCHED_PD_FP8_E4M3) {
    // amax slots are zero between pages: set here, reset by each scale update
    for (uint32_t i = threadIdx.x; i < 2 * kMaxGroup; i += kBlock)
      S.amax[i / kMaxGroup][i % kMaxGroup] = 0u;
    __syncthreads();
  }
  const uint32_t groups = P.Hkv / P.hpw;
  const uint32_t r = blockIdx.x / groups, h0 = (blockIdx.x % groups) * P.hpw, hpw = P.hpw;
  const int32_t a0 = P.app[r], a1 = P.app[r + 1];
  if (a1 <= a0)
    return;
  const int64_t n = (int64_t)a1 - a0, ctx = P.ctx[r], pos0 = ctx - n;
  if (a0 < 0 || (uint32_t)a1 > P.num_tokens || pos0 < 0) {
    if (threadIdx.x == 0 && blockIdx.y == 0 && P.errors)
      atomicAdd(P.errors, (uint32_t)(n * hpw));
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
        atomicAdd(P.errors, (o1 - o0) * hpw);
      continue;
    }
    const int64_t row0 = a0 + (pbase + o0 - pos0);
    if (ONE || (uint64_t)hpw * (o1 - o0) * (P.d / 4) <= kFastChunks) {
      if (kBatch % 2 == 0 && P.w8)
        page_one_round<SRC, KVD, (kBatch % 2 == 0 ? 8 : 4)>(P, S, stage, page, h0, hpw, o0,
                                                                o1, row0);
      else
        page_one_round<SRC, KVD, 4>(P, S, stage, page, h0, hpw, o0, o1, row0);
      continue;
    }
    if constexpr (!ONE) {
      if (KVD == SCHED_PD_FP8_E4M3)
        page_scales<SRC>(P, S, page, h0, hpw, o0, o1, row0);
      write_tensor<SRC, KVD>(P, S, 0, P.k_src, P.k_pool, page * P.kps, P.khs, P.kts, 1, h0,
                             hpw, o0, o1, row0);
      write_tensor<SRC, KVD>(P, S, 1, P.v_src, P.v_pool, page * P.vps, P.vhs, P.vts, P.vds, h0,
                             hpw, o0, o1, row0);
    }
  }
}

typedef void (*AppendFn)(AParams);

template <int SRC, bool ONE> AppendFn pick(uint32_t kvd) {
  switch (kvd) {
  case SCHED_PD_F32: return kv_append_kernel<SRC, SCHED_PD_F32, ONE>;
  case SCHED_PD_BF16: return kv_append_kernel<SRC, SCHED_PD_BF16, ONE>;
  case SCHED_PD_F16: return kv_append_kernel<SRC, SCHED_PD_F16, ONE>;
  default: return kv_append_kernel<SRC, SCHED_PD_FP8_E4M3, ONE>;
  }
}

template <bool ONE> AppendFn pick(uint32_t src, uint32_t kvd) {
  return src == SCHED_PD_F32    ? pick<SCHED_PD_F32, ONE>(kvd)
         : src == SCHED_PD_BF16 ? pick<SCHED_PD_BF16, ONE>(kvd)
                                : pick<SCHED_PD_F16, ONE>(kvd);
}

uint32_t esize(uint32_t dt) { return dt == SCHED_PD_F32 ? 4u : dt == SCHED_PD_FP8_E4M3 ? 1u : 2u; }

bool aligned(const void *p, uint32_t bytes) { return ((uintptr_t)p % bytes) == 0; }

bool mult4(int64_t s) { return s % 4 == 0; }

bool mult8(int64_t s) { return s % 8 == 0; }

} // namespace

// Block-table updates: table[row * width + col] = val for each of the n
// (row, col, val) triples packed as rows[n] | cols[n] | vals[n]. One lane per
// update; entries outside the table are ignored.
__global__ void __launch_bounds__(256) table_update_kernel(int32_t *table, int64_t num_rows,
                                                           int64_t width, const int32_t *upd,
                                                           uint32_t n) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= n)
    return;
  const int64_t r = upd[i], c = upd[(size_t)n + i];
  if (r < 0 || c < 0 || r >= num_rows || c >= width)
    return;
  table[r * width + c] = upd[2 * (size_t)n + i];
}

extern "C" {

int sched_kv_table_update(int32_t *table, int64_t num_rows, int64_t width,
                          const int32_t *updates, uint32_t n, void *stream) {
  if (n == 0)
    return 0;
  if (table == nullptr || updates == nullptr || num_rows <= 0 || width <= 0)
    return set_error(-1, "sched_kv_table_update: needs a table of num_rows x width > 0 "
                         "and an update list");
  hipLaunchKernelGGL(table_update_kernel, dim3((n + 255u) / 256u), dim3(256), 0,
                     static_cast<hipStream_t>(stream), table, num_rows, width, updates, n);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(-1, "sched_kv_table_update: launch failed: %s", hipGetErrorString(e));
  return 0;
}

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
  if (a->src_dtype != SCHED_PD_F32 && a->src_dtype != SCHED_PD_BF16 &&
      a->src_dtype != SCHED_PD_F16)
    return set_error(-1, "sched_kv_append: src dtype %u (F32, BF16 or F16)", a->src_dtype);
  if (a->kv_dtype > SCHED_PD_F16)
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
  P.scale_stride = (P.k_scale != nullptr && P.v_scale == P.k_scale + 1) ? 2u : 1u;
  P.errors = a->errors;

  const uint32_t max_app = a->max_append ? a->max_append : a->num_tokens;
  uint32_t hpw = a->heads_per_group;
  if (hpw == 0) {
    // Page-filling appends: the largest group whose appended chunks fit one
    // round, so every lane streams kBatch chunks. Small appends (a few tokens
    // per request, as in a decode step) are latency-bound: groups of at most
    // kBlock / head_dim heads, so a d-major V needs one slot group per lane.
    const uint32_t span = max_app < a->page_size ? max_app : a->page_size;
    const uint64_t per_head = (uint64_t)span * (a->head_dim / 4);
    const bool small = 2 * span < a->page_size;
    hpw = 1;
    while (hpw * 2 <= kMaxGroup && a->num_kv_heads % (hpw * 2) == 0) {
      const uint32_t next = hpw * 2;
      if (next * per_head > kFastChunks || (small && next * a->head_dim > kBlock))
        break;
      hpw = next;
    }
  } else if (hpw > kMaxGroup || a->num_kv_heads % hpw) {
    return set_error(-1, "sched_kv_append: heads_per_group %u must divide num_kv_heads %u "
                         "and be <= %u", hpw, a->num_kv_heads, kMaxGroup);
  }
  P.hpw = hpw;
  // 8-element chunks (16-byte bf16 source loads) when every row the
  // one-round path touches starts on an 8-element boundary
  P.vrow16 = vdm && a->page_size % 16 == 0 && a->v_dim_stride % 16 == 0 &&
             a->v_head_stride % 16 == 0 && a->v_page_stride % 16 == 0 &&
             aligned(a->v_pool, 16 * ke);
  P.w8 = a->head_dim % 8 == 0 && mult8(a->src_tok_stride) && mult8(a->src_head_stride) &&
         mult8(a->k_page_stride) && mult8(a->k_head_stride) && mult8(a->k_tok_stride) &&
         mult8(a->v_page_stride) && mult8(a->v_head_stride) && (vdm || mult8(a->v_tok_stride)) &&
         aligned(a->k_src, 8 * se) && aligned(a->v_src, 8 * se) && aligned(a->k_pool, 8 * ke) &&
         aligned(a->v_pool, 8 * ke);
  // pages an append of max_app tokens can touch: a run of n >= 1 slots
  // starting anywhere in a page spans at most (n + page - 2) / page + 1 pages
  // (one page for a single token); the page loop strides by grid.y, so any
  // grid.y >= 1 writes every page
  uint64_t gy = max_app ? (uint64_t)(max_app + a->page_size - 2) / a->page_size + 1 : 1;
  if (gy > 65535)
    gy = 65535;
  const dim3 grid(a->num_requests * (a->num_kv_heads / hpw), (uint32_t)gy);
  // every page of a group fits one round whatever the append sizes are
  const bool one = (uint64_t)hpw * a->page_size * (a->head_dim / 4) <= kFastChunks;
  AppendFn fn = one ? pick<true>(a->src_dtype, a->kv_dtype) : pick<false>(a->src_dtype, a->kv_dtype);
  hipLaunchKernelGGL(fn, grid, dim3(kBlock), 0, static_cast<hipStream_t>(stream), P);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(-1, "sched_kv_append: launch failed: %s", hipGetErrorString(e));
  return 0;
}

} // extern "C"
