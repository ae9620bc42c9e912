// decode_valu.h -- the general decode kernel on the VALU: any kv dtype
// (fp32 / bf16 / fp16 / fp8 e4m3fn), head dim 32/64/128, any page size that is a
// multiple of 16, general K/V strides, up to 16 q-heads per kv-head, and the
// linear-contraction mode. It serves the fp32 configurations (where the
// score must stay in fp32), the reference's fixture layouts (interleaved
// [token][K|V] pages) and every shape the MFMA kernel does not take.
//
// One workgroup (4 waves) runs one task = (request r, kv-head h). The tokens
// of the request are cut into 16-token chunks; wave w takes chunks w, w+4, ...
// so the split depends only on the context length. Per chunk:
//   score: lane (i = lane%16, slot = lane/16) owns token i of the chunk and
//          q-head 4*pass + slot; dot product against its K row (16-byte loads),
//          running max / sum per head over the 16-lane row (xor shuffles);
//   PV:    lane owns output element d = lane (+64); it loads V for the 16
//          tokens once and accumulates every head, broadcasting p and the
//          rescale factor with v_readlane.
// The 4 wave states (m, l, acc) merge in LDS in fixed wave order, so the
// result bits depend only on the task's inputs, never on which workgroup,
// worker or schedule ran it (pi / work-queue / prefetch invariance).
// Masked and out-of-context tokens get weight exactly 0 (score -inf, value 0),
// the reference's skip semantics (test/paged_decode.cu:136-137).
#pragma once

#include <type_traits>

#include "combine.h"

namespace schedpd {

template <typename KVT> struct Vec16;
template <> struct Vec16<float> { static constexpr int N = 4; };
template <> struct Vec16<uint16_t> { static constexpr int N = 8; };
template <> struct Vec16<uint8_t> { static constexpr int N = 16; };
template <> struct Vec16<_Float16> { static constexpr int N = 8; };

__device__ __forceinline__ void cvt16(const uint4 &raw, float *f, float) {
  f[0] = __uint_as_float(raw.x);
  f[1] = __uint_as_float(raw.y);
  f[2] = __uint_as_float(raw.z);
  f[3] = __uint_as_float(raw.w);
}
__device__ __forceinline__ void cvt16(const uint4 &raw, float *f, uint16_t) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    f[2 * k] = __uint_as_float(w[k] << 16);
    f[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
  }
}
__device__ __forceinline__ void cvt16(const uint4 &raw, float *f, _Float16) {
  typedef __attribute__((ext_vector_type(2))) _Float16 h2;
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const h2 v = __builtin_bit_cast(h2, w[k]);
    f[2 * k] = (float)v.x;
    f[2 * k + 1] = (float)v.y;
  }
}
__device__ __forceinline__ void cvt16(const uint4 &raw, float *f, uint8_t) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int b = 0; b < 4; ++b)
      f[4 * k + b] = fp8e4m3_to_f32((w[k] >> (8 * b)) & 0xffu);
}

__device__ __forceinline__ float ldv(const float *p) { return *p; }
__device__ __forceinline__ float ldv(const uint16_t *p) { return bf16_bits_to_f32(*p); }
__device__ __forceinline__ float ldv(const uint8_t *p) { return fp8e4m3_to_f32(*p); }
__device__ __forceinline__ float ldv(const _Float16 *p) { return (float)*p; }

__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Waves per workgroup (one workgroup per work item). Overridable at build
// time for tuning sweeps.
#ifndef SCHED_PD_VALU_NW
#define SCHED_PD_VALU_NW 4
#endif

template <typename KVT, int D, int GMAX, bool LINEAR>
__global__ void __launch_bounds__(SCHED_PD_VALU_NW * 64) decode_valu(KParams P) {
  constexpr int NW = SCHED_PD_VALU_NW;
  constexpr uint32_t NT = NW * 64;
  constexpr int GH = LINEAR ? 1 : GMAX;  // head rows of state
  constexpr int NP = (GH + 3) / 4;       // score passes (4 heads per pass)
  constexpr int EPL = D >= 64 ? D / 64 : 1;
  constexpr int VN = Vec16<KVT>::N;
  // K loads unrolled in the score: fp8 converts 16 values per load, so 2
  // (not 4) in flight keep it in the register file (4 spilled to AGPRs)
  constexpr int kScoreUnroll = VN == 16 ? 2 : 4;
  __shared__ float s_q[GH][D];
  // Linear mode accumulates in double: an unnormalised sum of thousands of
  // products loses the fp32 tolerance in float; the mode is bandwidth-bound.
  using Acc = typename std::conditional<LINEAR, double, float>::type;
  __shared__ Acc s_acc[NW][GH][D];
  __shared__ float s_m[NW][GH];
  __shared__ float s_l[NW][GH];
  // Page ids of the item's first kPageCache pages, read once per item: a
  // chunk's K/V loads then wait on an LDS read instead of a dependent global
  // load of the page table (which set the pace of single long tasks).
  constexpr uint32_t kPageCache = 256;
  __shared__ int32_t s_page[kPageCache];

  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); // scalar wave index
  const uint32_t i16 = lane & 15u, slot = lane >> 4;
  const bool toff = timer_off_latched(P.L);

  run_tasks(P.L, [&](uint32_t wi, bool) __attribute__((always_inline)) {
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
    const ItemRange R = item_range(P, I, n, (nload + P.ps - 1) / P.ps);
    if (item_skip(P, wi, I, R))
      return;
    const bool stale = item_stale(P, wi, I, R, n);
    const uint32_t G = LINEAR ? 1u : P.G;
    const bool fp8 = sizeof(KVT) == 1;

    if (!LINEAR)
      for (uint32_t idx = threadIdx.x; idx < G * D; idx += NT) {
        uint32_t g = idx / D, j = idx % D;
        s_q[g][j] = load_q(P, ((int64_t)r * P.Hq + h * G + g) * D + j);
      }
    // pages [p0, p_end) hold the chunks below; the first kPageCache of them
    // go to LDS (the previous item's reads ended before its merge barrier)
    const uint32_t tok_end = min(R.p1 * P.ps, nload);
    const uint32_t p_end = (tok_end + P.ps - 1) / P.ps;
    const uint32_t ncache = p_end > R.p0 ? min(p_end - R.p0, kPageCache) : 0u;
    for (uint32_t i = threadIdx.x; i < ncache; i += NT)
      s_page[i] = page_of(P, r, R.p0 + i);
    __syncthreads();

    float m[NP], lsum[NP];
    Acc acc[GH][EPL];
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      m[k] = kMInit;
      lsum[k] = 0.f;
    }
#pragma unroll
    for (int g = 0; g < GH; ++g)
#pragma unroll
      for (int e = 0; e < EPL; ++e)
        acc[g][e] = Acc(0);

    // 16-token chunks of this work item's pages [p0, p1), round-robin over waves
    const uint32_t cpp = P.ps / 16u;
    const uint32_t c_end = (tok_end + 15u) / 16u;
    for (uint32_t c = R.p0 * cpp + w; c < c_end; c += NW) {
      const uint32_t pos0 = c * 16u, b = pos0 / P.ps, o = pos0 % P.ps;
      const int64_t page = b - R.p0 < ncache ? s_page[b - R.p0] : page_of(P, r, b);
      const int64_t si = ((int64_t)page * P.Hkv + h) * P.scale_stride;
      const float ks = (fp8 && P.k_scale) ? P.k_scale[si] : 1.f;
      const float vs = (fp8 && P.v_scale) ? P.v_scale[si] : 1.f;
      float p_hp[NP], c_hp[NP];


      if (!LINEAR) {
        const uint32_t t = pos0 + i16;
        const bool kp = t < n && keep_pos(P, pol.budget, t);
        const KVT *krow = static_cast<const KVT *>(P.k_pool) + page * P.kps +
                          (int64_t)h * P.khs + (int64_t)(o + i16) * P.kts;
#pragma unroll
        for (int hp = 0; hp < NP; ++hp) {
          const uint32_t head = 4u * hp + slot;
          const bool act = kp && head < G;
          float dot = 0.f;
          if (act) {
            const float *qh = s_q[head];
#pragma unroll kScoreUnroll
            for (int j0 = 0; j0 < D; j0 += VN) {
              uint4 raw = *reinterpret_cast<const uint4 *>(krow + j0);
              float f[VN];
              cvt16(raw, f, KVT());
#pragma unroll
              for (int e = 0; e < VN; ++e)
                dot += qh[j0 + e] * f[e];
            }
          }
          const float sc = act ? dot * ks * P.scale_log2 : kNegInf;
          float cmax = sc;
#pragma unroll
          for (int x = 1; x < 16; x <<= 1)
            cmax = fmaxf(cmax, __shfl_xor(cmax, x));
          const float mnew = fmaxf(m[hp], cmax);
          const float cf = exp2f(m[hp] - mnew);
          const float p = exp2f(sc - mnew);
          float ps = p;
#pragma unroll
          for (int x = 1; x < 16; x <<= 1)
            ps += __shfl_xor(ps, x);
          lsum[hp] = lsum[hp] * cf + ps;
          m[hp] = mnew;
          p_hp[hp] = p;
          c_hp[hp] = cf;
        }
      }

      // PV (or the linear contraction): V for the 16 tokens at my elements.
      // Every slot of a page this loop visits is addressable, so the loads
      // are unconditional (issued together, not one branch each) and masked
      // tokens are selected to 0 afterwards; a lane past D reads element D-1
      // and drops it. (Issuing them before the score, or loading K for
      // masked lanes too, measured slower: more VGPRs, fewer waves.)
      float v[16][EPL];
      const KVT *vbase = static_cast<const KVT *>(P.v_pool) + page * P.vps + (int64_t)h * P.vhs;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t ti = pos0 + i;
        const bool ki = ti < n && keep_pos(P, pol.budget, ti);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          const uint32_t d = lane + 64u * e;
          const uint32_t dc = d < (uint32_t)D ? d : (uint32_t)D - 1u;
          const float x = ldv(vbase + (int64_t)(o + i) * P.vts + (int64_t)dc * P.vds);
          v[i][e] = (ki && d < D) ? x * vs : 0.f;
        }
      }
      if (LINEAR) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const uint32_t ti = pos0 + i;
          const bool ki = ti < n && keep_pos(P, pol.budget, ti);
          // weight index clamped into [0, n) (the weights cover the context)
          const uint32_t wix = P.lin_w_period ? ti % P.lin_w_period : min(ti, n - 1u);
          const float wv = P.lin_w[wix];
          const float wi = ki ? wv : 0.f;
#pragma unroll
          for (int e = 0; e < EPL; ++e)
            acc[0][e] += (double)wi * (double)v[i][e];
        }
      } else {
#pragma unroll
        for (int g = 0; g < GH; ++g) {
          if ((uint32_t)g < G) {
            const float cg = readlane_f(c_hp[g / 4], 16 * (g % 4));
#pragma unroll
            for (int e = 0; e < EPL; ++e)
              acc[g][e] *= cg;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const float pgi = readlane_f(p_hp[g / 4], 16 * (g % 4) + i);
#pragma unroll
              for (int e = 0; e < EPL; ++e)
                acc[g][e] += pgi * v[i][e];
            }
          }
        }
      }
    }

    // Merge the 4 wave states in fixed order.
#pragma unroll
    for (int g = 0; g < GH; ++g) {
      if (!LINEAR && lane == 16u * (g % 4)) {
        s_m[w][g] = m[g / 4];
        s_l[w][g] = lsum[g / 4];
      }
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const uint32_t d = lane + 64u * e;
        if (d < D)
          s_acc[w][g][d] = acc[g][e];
      }
    }
    __syncthreads();
    if (stale)
      mark_stale<NW, D, LINEAR>(P, I.chunk, r, h, G);
    else
      finish_item<NW, GH, D, Acc, LINEAR>(P, wi, task, I.chunk, R.nchunks, r, h, G, s_acc, s_m,
                                          s_l);
    timer_commit(P.L, toff, task, t0);
  });
}

} // namespace schedpd
