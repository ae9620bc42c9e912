// common.h -- kernel parameter block and small device helpers shared by the
// decode kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "levers.h"

namespace schedpd {

// Everything a decode kernel reads, passed by value as the kernel argument.
struct KParams {
  LeverTables L;
  const void *q;
  void *out;
  const void *k_pool;
  const void *v_pool;
  int64_t kps, khs, kts;      // K strides (elements): page, head, token
  int64_t vps, vhs, vts, vds; // V strides (elements): page, head, token, dim
  const float *k_scale;
  const float *v_scale;
  uint32_t scale_stride; // floats between the scales of consecutive (page, head)s: 2 when
                         // K and V scales are interleaved pairs (v_scale == k_scale + 1)
  const int32_t *bt;
  const int32_t *indptr;
  const int32_t *ctx;
  const float *lin_w;
  uint32_t R, Hq, Hkv, G;
  uint32_t ps, bt_stride, tau_scope;
  uint32_t q_f32, o_f32, ctx_in_pages, shed_loads, lin_w_period;
  uint32_t q_f16, o_f16; // IEEE binary16 Q / output (else bf16 unless *_f32)
  uint32_t pf_depth;     // MFMA kernel: urgent ring depth in pages (0 = the deepest)
  float scale_log2; // softmax scale * log2(e): scores live in the exp2 domain
  // split-KV work items (tiles == nullptr: one work item per task)
  const int32_t *tiles;
  uint32_t ntasks;     // requests x kv-heads
  uint32_t tile_pages;
  uint32_t tile_ranged; // rows (task, chunk | nchunks << 16, p0, p1), else (task, chunk)
  uint32_t *ws_stale;  // tasks found with a stale plan (item_stale)
  uint32_t *ws_count;  // per-task arrival counters
  float *ws_ml;        // per-work-item (m, l) per head
  void *ws_acc;        // per-work-item partial accumulators
  // Fused append (sched_paged_decode_append; nullptr = none): request r's
  // new token is source row r, written into the cache before it is read.
  const void *app_k;
  const void *app_v;
  int64_t app_ts, app_hs; // source strides (elements): row, kv-head
  uint32_t app_f32;       // fp32 source rows (else the cache's 16-bit type, or for an fp8
                          // cache app_f16 ? fp16 : bf16)
  uint32_t app_f16;
};

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kMInit = -1e30f; // running-max start value (test/paged_decode.cu:94)
// Buffer resource word 3 for raw buffer loads (GFX9: data format 32, so that
// a raw load is not treated as an invalid format), and the load's cache
// policy bits: 2 = nt (streamed, as __builtin_nontemporal_load).
constexpr int kBufWord3 = 0x00020000;
constexpr int kBufNT = 2;

__device__ __forceinline__ int32_t page_of(const KParams &P, uint32_t r, uint32_t b) {
  return P.indptr ? P.bt[P.indptr[r] + b] : P.bt[(int64_t)r * P.bt_stride + b];
}

__device__ __forceinline__ uint32_t ctx_tokens(const KParams &P, uint32_t r) {
  // one request's length: the same on every lane, kept in a scalar register
  uint32_t c = __builtin_amdgcn_readfirstlane((uint32_t)P.ctx[r]);
  return P.ctx_in_pages ? c * P.ps : c;
}

// Shed keep test for token position t of a request (budget from task_policy):
// prefix scope counts t, per-page scope counts t's offset in its page.
__device__ __forceinline__ bool keep_pos(const KParams &P, uint32_t budget, uint32_t t) {
  uint32_t ctr = P.tau_scope == SCHED_PD_TAU_PER_PAGE ? t % P.ps : t;
  return ctr < budget;
}

// Tokens that need loading: with a prefix budget the pages past it hold only
// masked tokens, whose contribution is exactly zero, so they are not read
// (unless shed_loads asks for the reference's load-and-mask behaviour).
__device__ __forceinline__ uint32_t load_extent(const KParams &P, uint32_t n, uint32_t budget) {
  if (P.tau_scope == SCHED_PD_TAU_PREFIX && !P.shed_loads && budget < n)
    return budget;
  return n;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// OCP e4m3fn decode by bit construction (1 sign, 4 exponent bits bias 7,
// 3 mantissa bits; S.1111.111 is NaN, there is no infinity).
__device__ __forceinline__ float fp8e4m3_to_f32(uint32_t b) {
  uint32_t s = (b & 0x80u) << 24, e = (b >> 3) & 15u, m = b & 7u;
  float v;
  if (e == 0u)
    v = (float)m * 0.001953125f; // m * 2^-9
  else
    v = __uint_as_float(((e + 120u) << 23) | (m << 20));
  if (e == 15u && m == 7u)
    v = __builtin_nanf("");
  return __uint_as_float(__float_as_uint(v) | s);
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u)
    return (uint16_t)((u >> 16) | 0x40u); // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;
// Round-to-nearest-even pair conversions (v_cvt_pk_bf16_f32 /
// v_cvt_pk_f16_f32; fp32 denormals are preserved, NaN stays NaN).
__device__ __forceinline__ unsigned pack_bf16_rne(float lo, float hi) {
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(unsigned, v);
}
__device__ __forceinline__ unsigned pack_f16_rne(float lo, float hi) {
  const f16x2_t v = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(unsigned, v);
}

// fp8 cache scales (the cache writer's rule, also applied by the decode's
// fused append): the least 2^k (k >= -126) with a <= 448 * 2^k; 0 for a == 0.
// With a = m * 2^e, m in [0.5, 1): k = e - 9 when m <= 0.875 (448 = 0.875 *
// 2^9), else e - 8.
__device__ __forceinline__ float pow2_scale(float a) {
  if (!(a > 0.f))
    return 0.f;
  int e;
  float m = frexpf(a, &e);
  int k = e - 9 + (m > 0.875f ? 1 : 0);
  return ldexpf(1.f, k < -126 ? -126 : k);
}

// q clamped to the e4m3fn range, round-to-nearest-even, four at once (byte i
// of the result is element i). Each element rounds on its own, so encoding
// two at a time (the low half) gives the same bytes.
__device__ __forceinline__ uint32_t encode4_fp8(const float q[4]) {
  float c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    c[i] = fminf(fmaxf(q[i], -448.f), 448.f);
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(c[0], c[1], 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c[2], c[3], w, true);
  return (uint32_t)w;
}
__device__ __forceinline__ uint32_t encode2_fp8(float q0, float q1) {
  const float c0 = fminf(fmaxf(q0, -448.f), 448.f), c1 = fminf(fmaxf(q1, -448.f), 448.f);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c0, c1, 0, false) & 0xffffu;
}

// Max over the 64 lanes of a wave (all lanes active), in VALU cross-lane
// moves: quad permutes and row rotations (DPP) within each row of 16, then
// v_permlane16/32_swap across rows. Every lane gets the result.
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF,
                                                          false))); // quad [1,0,3,2]
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF,
                                                          false))); // quad [2,3,0,1]
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xF, 0xF,
                                                          false))); // row_ror:4
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF,
                                                          false))); // row_ror:8
  const unsigned u = __float_as_uint(x);
  auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const unsigned v = __float_as_uint(x);
  auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Fused append: the K and V rows of request r's new token (source row r,
// kv-head h) into slot `slot` of page `page`, in the cache's 16-bit type (an
// fp32 source rounds to nearest even); lane l writes dims 2l, 2l+1 of both
// rows (head dim 128). Called by the one wave that streams that page (in
// either the MFMA or the one-wave kernel), which waits for its stores
// before it streams, so it reads the token back from the cache like every
// other token (each page of an item is streamed by exactly one wave, and no
// other workgroup reads this (page, kv-head)).
template <bool F16>
__device__ __forceinline__ void append_token(const KParams &P, uint32_t r, uint32_t h,
                                             int64_t page, uint32_t slot, uint32_t lane) {
  const uint32_t j = 2u * lane;
  const int64_t src = (int64_t)r * P.app_ts + (int64_t)h * P.app_hs + j;
  uint32_t kw, vw;
  if (P.app_f32) {
    const float *ks = static_cast<const float *>(P.app_k) + src;
    const float *vs = static_cast<const float *>(P.app_v) + src;
    kw = F16 ? pack_f16_rne(ks[0], ks[1]) : pack_bf16_rne(ks[0], ks[1]);
    vw = F16 ? pack_f16_rne(vs[0], vs[1]) : pack_bf16_rne(vs[0], vs[1]);
  } else {
    kw = *reinterpret_cast<const uint32_t *>(static_cast<const uint16_t *>(P.app_k) + src);
    vw = *reinterpret_cast<const uint32_t *>(static_cast<const uint16_t *>(P.app_v) + src);
  }
  uint16_t *kd = static_cast<uint16_t *>(const_cast<void *>(P.k_pool)) + page * P.kps +
                 (int64_t)h * P.khs + (int64_t)slot * P.kts + j;
  uint16_t *vd = static_cast<uint16_t *>(const_cast<void *>(P.v_pool)) + page * P.vps +
                 (int64_t)h * P.vhs + (int64_t)slot * P.vts + j;
  *reinterpret_cast<uint32_t *>(kd) = kw;
  *reinterpret_cast<uint32_t *>(vd) = vw;
}

__device__ __forceinline__ void store_out(const KParams &P, int64_t idx, float v) {
  if (P.o_f32)
    static_cast<float *>(P.out)[idx] = v;
  else if (P.o_f16)
    static_cast<_Float16 *>(P.out)[idx] = (_Float16)v; // round to nearest even
  else
    static_cast<uint16_t *>(P.out)[idx] = f32_to_bf16_rne(v);
}

__device__ __forceinline__ float load_q(const KParams &P, int64_t idx) {
  return P.q_f32   ? static_cast<const float *>(P.q)[idx]
         : P.q_f16 ? (float)static_cast<const _Float16 *>(P.q)[idx]
                   : bf16_bits_to_f32(static_cast<const uint16_t *>(P.q)[idx]);
}

} // namespace schedpd
