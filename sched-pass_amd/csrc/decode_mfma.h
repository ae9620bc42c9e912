// decode_mfma.h -- the GQA decode kernel on the CDNA4 matrix cores:
// bf16 or fp8-e4m3fn KV with bf16 Q, or fp16 KV with fp16 Q (F16), head dim
// 128, pages of 16..256 tokens, up to 16 q-heads per kv-head (one MFMA
// column block); and the linear contraction over the same V stream (LINEAR:
// no K, weights as MFMA column 0).
//
// Layout it reads (one (page, kv-head) chunk each for K and V):
//   K: 16 token rows x 128 dims, dims contiguous (row stride k_tok_stride);
//   V: 128 dim rows x 16 tokens, tokens contiguous (v_tok_stride 1, row stride
//      v_dim_stride) -- the per-page d-major V of vLLM's paged cache.
// With these, both MFMA operands load straight from HBM into registers:
//
//   QK  S^T[16 tok x 16 head] = K[16 x 128] . Q^T[128 x 16]
//       4 x v_mfma_f32_16x16x32_bf16; A = K rows (lane: token lane%16,
//       8 dims at slot lane/16 -> one 16-byte load), B = Q (held all task).
//   The accumulator lane layout (head = lane%16, tokens 4*(lane/16)+0..3) is
//   exactly the B-operand layout of v_mfma_f32_16x16x16_bf16, so after the
//   online-softmax update the probabilities feed PV with no data movement:
//   PV  O^T[128 x 16 head] += V^T[128 x 16 tok] . P^T[16 tok x 16 head]
//       8 x v_mfma_f32_16x16x16_bf16; A = V^T rows (lane: dim 16*blk+lane%16,
//       tokens 4*(lane/16)..+3). Lanes load 16-byte V row halves (bf16) or
//       whole rows (fp8) and trade these 4-token slices across lane rows
//       with v_permlane16/32_swap (bf16_v_operands, fp8_v_operands).
//
// Token-major V (FlashInfer's NHD / HND caches): a lane loads dims
// 8*(lane%16)..+7 of tokens 4*(lane/16)..+3 (four 16-byte row pieces, or
// 8-byte ones for fp8), and
// MFMA row lane%16 of dim block blk stands for dim 8*(lane%16) + blk, so each
// block's A operand is two v_perm_b32 of the lane's own registers; the state
// goes to LDS with that dim order undone (bf16_vt_operand, fp8_vt_operands,
// VT).
//
// Pages of 32..256 tokens (PG): the kernel streams 16-token blocks; block b
// is sub-block b % m of table entry b / m (m = page / 16). A d-major V row
// then holds several blocks, which neighbouring waves read at about the same
// time: those loads are temporal, so the line one wave fetched is still in
// L2 for the next. The shed's per-page scope counts the token's offset in its
// whole page.
//
// A workgroup of NW waves runs one task = (request, kv-head); wave w streams
// pages w, w+NW, ... with DEPTH pages of loads in flight (register ring), and
// the wave states merge in LDS in fixed order. Nothing
// in the arithmetic depends on scheduling, so pi, the work queue and the
// prefetch depth leave every output bit unchanged.
//
// Policy lever: urgent tasks stream with a deeper ring than stock (DEPTH_S
// pages in flight per wave): the launch's pf_dist, any depth in
// [DEPTH_S, DEPTH_U], DEPTH_U by default (deeper KV prefetch). Polite tasks
// always stream with non-temporal loads (the reference's "do not keep this
// task's lines"). Stock tasks do too (KV is read once per step), except work
// items longer than kLongItemPages and a queue worker's last item, which take
// the deep ring with ordinary loads; so polite and stock differ only on
// those items.
// fp8: values convert exactly to bf16; the per-(page, head) K scale multiplies
// the score and the V scale multiplies p before PV, so no element is scaled.
#pragma once

#include "combine.h"

namespace schedpd {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) short s16x4_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4_t;
typedef __attribute__((ext_vector_type(2))) unsigned u32x2_t;

template <bool FP8> struct PageRegs;
template <> struct PageRegs<false> {
  u32x4_t k[4]; // 4 x 8 bf16 K
  u32x4_t v[4]; // V row halves, see bf16_v_operands
  float lw[4];  // linear mode: the lane's token weights, loaded with the page
};
template <> struct PageRegs<true> {
  u32x4_t k[2]; // 2 x 16 fp8 K
  u32x4_t v[2]; // V rows lane and lane + 64 (16 fp8 tokens each), see fp8_v_operands
  float lw[4];   // linear mode: the lane's token weights, loaded with the page
  float ks, vs;  // the page's K / V scales, loaded with its KV so that no
                 // load is consumed right after issue (which would drain the
                 // whole prefetch ring with s_waitcnt vmcnt(0))
};

// KV pages are read once per step, so every task streams them with
// non-temporal loads (measured on the 64 x 2048 bf16 step: 93 -> 83 us).
// Polite tasks therefore load as stock ones do, except on long items (below);
// urgent ones keep a deeper ring. Overridable at build time for tuning.
#ifndef SCHED_PD_MFMA_STOCK_NT
#define SCHED_PD_MFMA_STOCK_NT 1
#endif
constexpr bool kStockNT = SCHED_PD_MFMA_STOCK_NT != 0;

// A work item of more pages than this is the step's straggler: it streams
// alone at the end, where a deep pipeline of ordinary (temporal) loads runs
// faster than non-temporal ones (heterogeneous batch, one workgroup per task:
// 828 -> 662 us; 64-page threshold slows the 128-page tasks of the uniform
// batch, 83 -> 94 us). Polite items keep their non-temporal loads.
#ifndef SCHED_PD_MFMA_LONG_ITEM_PAGES
#define SCHED_PD_MFMA_LONG_ITEM_PAGES 256u
#endif
constexpr uint32_t kLongItemPages = SCHED_PD_MFMA_LONG_ITEM_PAGES;
// A queue worker's last item streams in the launch's run-down, with fewer
// and fewer items beside it, where ordinary loads serve it better than
// non-temporal ones (measured with 128-page tiles under urgency order: C3
// queue 377 -> 363 us; the fp8 Qwen2-7B queue over 256-page tiles 355 ->
// 343 us; the graded plans, whose last items are small, -1.5% to 0). The
// loads are what matters: the same items on the deep ring with
// non-temporal loads run as before, on the stock ring with ordinary loads
// as here. They take the long-item path (deep ring, ordinary loads).
#ifndef SCHED_PD_MFMA_LATE_DEEP
#define SCHED_PD_MFMA_LATE_DEEP 1
#endif
constexpr bool kLateDeep = SCHED_PD_MFMA_LATE_DEEP != 0;

template <bool NT, typename T> __device__ __forceinline__ T gload(const T *p) {
  if constexpr (NT)
    return __builtin_nontemporal_load(p);
  else
    return *p;
}

// Dim slot of element e of lane-group g4 in QK step kb. bf16: one 16-byte
// load per step. fp8: one 16-byte load covers steps 2c and 2c+1. Q uses the
// same map, so the dot product runs over the same dims either way.
__device__ __forceinline__ uint32_t qk_dim(bool fp8, uint32_t kb, uint32_t g4) {
  return fp8 ? 64u * (kb >> 1) + 16u * g4 + 8u * (kb & 1u) : 32u * kb + 8u * g4;
}

typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(4))) _Float16 f16x4_t;

// QK and PV MFMAs on 16-bit operands held as raw bits: bf16, or (F16) IEEE
// binary16 for fp16 caches with fp16 Q.
template <bool F16>
__device__ __forceinline__ f32x4_t mfma_qk(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
template <bool F16>
__device__ __forceinline__ f32x4_t mfma_pv(s16x4_t a, s16x4_t b, f32x4_t c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a),
                                                 __builtin_bit_cast(f16x4_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// Reductions across the four 16-lane rows with the gfx950 row swaps (VALU,
// no LDS traffic). v_permlane16_swap(x, x) leaves {x[row], x[row ^ 1]} in its
// two results on every lane, v_permlane32_swap(x, x) {x[half], x[half ^ 1]};
// combining the pair gives the pairwise max / sum, in the same operand order on
// every lane.
__device__ __forceinline__ float max_rows(float x) {
  const unsigned u = __float_as_uint(x);
  auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const unsigned v = __float_as_uint(x);
  auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_rows(float x) {
  const unsigned u = __float_as_uint(x);
  auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const unsigned v = __float_as_uint(x);
  auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// 4 fp8 bytes -> 4 bf16 (exact: every e4m3fn value is a bf16), as two
// dwords: one v_cvt_scalef32_pk_bf16_fp8 (scale 1) per byte pair. The packed
// result is moved as a whole dword (checked on all 256 codes against torch).
__device__ __forceinline__ u32x2_t fp8x4_to_bf16x4(unsigned w) {
  u32x2_t r;
  r.x = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
  r.y = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
  return r;
}

// fp8 V: a lane loads two whole 16-byte V rows (rows lane and lane + 64 of
// the page's 128 dims), a quarter of the load instructions of taking each
// 4-token slice separately. The PV A-operand of lane (g4, c16) for dim block
// blk is dword g4 (tokens 4*g4..+3) of row 16*blk + c16, which the lane in
// row group blk % 4 holds: a 4x4 transpose of (dword, lane row) per load,
// done with two v_permlane32_swap and two v_permlane16_swap (the first swaps
// the upper rows of its first operand with the lower rows of the second, the
// second swaps odd rows of the first with even rows of the second).
__device__ __forceinline__ void rows_transpose4(unsigned d[4]) {
  const auto a = __builtin_amdgcn_permlane32_swap(d[0], d[2], false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(d[1], d[3], false, false);
  const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  const auto e = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  d[0] = c[0];
  d[1] = c[1];
  d[2] = e[0];
  d[3] = e[1];
}

// The eight fp8 PV A-operands (4 tokens of one dim, one per dim block).
__device__ __forceinline__ void fp8_v_operands(const u32x4_t v[2], unsigned out[8]) {
  out[0] = v[0].x, out[1] = v[0].y, out[2] = v[0].z, out[3] = v[0].w;
  out[4] = v[1].x, out[5] = v[1].y, out[6] = v[1].z, out[7] = v[1].w;
  rows_transpose4(out);
  rows_transpose4(out + 4);
}

// bf16 V: load i of a lane in row group g4 is the 16-byte half g4 / 2
// (tokens 8*(g4/2)..+7) of V row 16*(2i + g4 % 2) + c16: even lane rows hold
// dim block 2i, odd ones block 2i + 1, each as the two 4-token slices of the
// half. One v_permlane16_swap per dword pair trades the odd rows' first slice
// for the even rows' second, after which every lane holds its own slice
// (tokens 4*g4..+3) of both blocks: four 16-byte loads and eight swaps per
// page instead of eight 8-byte loads.
__device__ __forceinline__ void bf16_v_operands(u32x4_t v[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const auto a = __builtin_amdgcn_permlane16_swap(v[i].x, v[i].z, false, false);
    const auto b = __builtin_amdgcn_permlane16_swap(v[i].y, v[i].w, false, false);
    v[i] = u32x4_t{a[0], b[0], a[1], b[1]}; // (block 2i slice, block 2i + 1 slice)
  }
}

// Token-major bf16 V: r[v] holds dims 8*c16..+7 of token 4*g4 + v; the A
// operand of block blk is dim 8*c16 + blk of the four tokens (low or high
// halves of dword blk/2, paired by v_perm_b32).
__device__ __forceinline__ s16x4_t bf16_vt_operand(const u32x4_t r[4], int blk) {
  const unsigned sel = (blk & 1) ? 0x07060302u : 0x05040100u;
  const int dw = blk >> 1;
  const unsigned lo = __builtin_amdgcn_perm(r[1][dw], r[0][dw], sel);
  const unsigned hi = __builtin_amdgcn_perm(r[3][dw], r[2][dw], sel);
  return __builtin_bit_cast(s16x4_t, u32x2_t{lo, hi});
}

// Token-major fp8 V: lane (c16, g4) holds dims 8*c16..+7 of tokens 4*g4 + t
// (t = 0..3) as 8 bytes each, v[t >> 1] dwords 2*(t & 1) (dims 0..3) and
// 2*(t & 1) + 1 (dims 4..7). The A operand of block blk is byte blk of those
// tokens, one token per byte: a 4 x 4 byte transpose of the low dwords
// (blocks 0..3) and of the high ones (4..7), two v_perm_b32 per operand.
__device__ __forceinline__ void fp8_vt_transpose(unsigned w0, unsigned w1, unsigned w2,
                                                 unsigned w3, unsigned out[4]) {
  const unsigned t0 = __builtin_amdgcn_perm(w1, w0, 0x05010400u); // w0.0 w1.0 w0.1 w1.1
  const unsigned t1 = __builtin_amdgcn_perm(w3, w2, 0x05010400u); // w2.0 w3.0 w2.1 w3.1
  const unsigned t2 = __builtin_amdgcn_perm(w1, w0, 0x07030602u); // w0.2 w1.2 w0.3 w1.3
  const unsigned t3 = __builtin_amdgcn_perm(w3, w2, 0x07030602u); // w2.2 w3.2 w2.3 w3.3
  out[0] = __builtin_amdgcn_perm(t1, t0, 0x05040100u);
  out[1] = __builtin_amdgcn_perm(t1, t0, 0x07060302u);
  out[2] = __builtin_amdgcn_perm(t3, t2, 0x05040100u);
  out[3] = __builtin_amdgcn_perm(t3, t2, 0x07060302u);
}
__device__ __forceinline__ void fp8_vt_operands(const u32x4_t v[2], unsigned out[8]) {
  fp8_vt_transpose(v[0].x, v[0].z, v[1].x, v[1].z, out);
  fp8_vt_transpose(v[0].y, v[0].w, v[1].y, v[1].w, out + 4);
}

struct MfmaTask {
  uint32_t r, h, n, budget;
  int64_t row; // block-table index of the request's first page
  uint32_t p0, p1; // pages [p0, p1) of the task are read by this work item
  uint32_t w;      // this wave: pages p0 + w, p0 + w + NW, ...
  const uint8_t *kbase; // K pool bytes + per-lane offset
  const uint8_t *vbase;
  int64_t kpage_bytes, khead_bytes, vpage_bytes, vhead_bytes;
  int64_t vrow_bytes; // token-major V: bytes between token rows
  uint32_t vlane;     // token-major V / PG: this lane's V byte offset in a block
  uint32_t bshift, bmask; // PG: 16-token blocks per page = 1 << bshift
  int64_t ksub, vsub;     // PG: bytes from one block of a page to the next
  int64_t vblk;           // PG, d-major V: bytes between the lane's dim blocks
};

// Offset of pidx's first token within its page (PG), else 0.
template <bool PG>
__device__ __forceinline__ uint32_t block_in_page(const MfmaTask &T, uint32_t pidx) {
  if constexpr (PG)
    return (pidx & T.bmask) * 16u;
  else
    return 0u;
}

struct MfmaState {
  float m, lsum;
  f32x4_t acc[8];
  bf16x8_t qop[4];
};

template <bool FP8, bool NT, bool LINEAR, bool VT, bool PG>
__device__ __forceinline__ void issue_page(const KParams &P, const MfmaTask &T, int32_t page,
                                           uint32_t pidx, PageRegs<FP8> &B) {
  if constexpr (LINEAR) {
    // weights of tokens 4*g4..+3 of the page, for the lanes of MFMA column 0;
    // positions past the context are masked later and not read
    const uint32_t lane = threadIdx.x & 63u, g4 = lane >> 4;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const uint32_t t = pidx * 16u + 4u * g4 + v;
      B.lw[v] = ((lane & 15u) == 0u && t < T.n)
                    ? P.lin_w[P.lin_w_period ? t % P.lin_w_period : t] : 0.f;
    }
  }
  const uint32_t sub = PG ? (pidx & T.bmask) : 0u;
  const uint8_t *kp = T.kbase + (int64_t)page * T.kpage_bytes + T.khead_bytes +
                      (PG ? (int64_t)sub * T.ksub : 0);
  const uint8_t *vp = T.vbase + (int64_t)page * T.vpage_bytes + T.vhead_bytes;
  // PG and token-major V: a uniform block base + the lane's 32-bit offset
  const uint8_t *pb = static_cast<const uint8_t *>(P.v_pool) + (int64_t)page * T.vpage_bytes +
                      T.vhead_bytes + (PG ? (int64_t)sub * T.vsub : 0);
  if constexpr (!FP8) {
    if constexpr (!LINEAR)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
        B.k[kb] = gload<NT>(reinterpret_cast<const u32x4_t *>(kp + 64 * kb));
    if constexpr (VT) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        B.v[i] = gload<NT>(reinterpret_cast<const u32x4_t *>(pb + i * T.vrow_bytes + T.vlane));
    } else if constexpr (PG) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        B.v[i] = gload<false>(reinterpret_cast<const u32x4_t *>(pb + i * T.vblk + T.vlane));
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        B.v[i] = gload<NT>(reinterpret_cast<const u32x4_t *>(vp + 1024 * i));
    }
  } else {
    if constexpr (!LINEAR)
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
        B.k[cc] = gload<NT>(reinterpret_cast<const u32x4_t *>(kp + 64 * cc));
    const int64_t si = ((int64_t)page * P.Hkv + T.h) * P.scale_stride;
    B.ks = (!LINEAR && P.k_scale) ? P.k_scale[si] : 1.f;
    B.vs = P.v_scale ? P.v_scale[si] : 1.f;
    if constexpr (VT) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const u32x2_t a =
            gload<NT>(reinterpret_cast<const u32x2_t *>(pb + (2 * t) * T.vrow_bytes + T.vlane));
        const u32x2_t b = gload<NT>(
            reinterpret_cast<const u32x2_t *>(pb + (2 * t + 1) * T.vrow_bytes + T.vlane));
        B.v[t] = u32x4_t{a.x, a.y, b.x, b.y};
      }
    } else if constexpr (PG) {
      B.v[0] = gload<false>(reinterpret_cast<const u32x4_t *>(pb + T.vlane));
      B.v[1] = gload<false>(reinterpret_cast<const u32x4_t *>(pb + T.vblk + T.vlane));
    } else {
      B.v[0] = gload<NT>(reinterpret_cast<const u32x4_t *>(vp));
      B.v[1] = gload<NT>(reinterpret_cast<const u32x4_t *>(vp + 64 * 16));
    }
  }
}

template <bool FP8, bool VT, bool PG, bool F16>
__device__ __forceinline__ void compute_page(const KParams &P, const MfmaTask &T, MfmaState &S,
                                             const PageRegs<FP8> &B, int32_t page, uint32_t pidx,
                                             uint32_t g4) {
  // QK
  f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    bf16x8_t a;
    if constexpr (!FP8) {
      a = __builtin_bit_cast(bf16x8_t, B.k[kb]);
    } else {
      const u32x4_t raw = B.k[kb >> 1];
      const unsigned w0 = (kb & 1) ? raw.z : raw.x, w1 = (kb & 1) ? raw.w : raw.y;
      const u32x2_t lo = fp8x4_to_bf16x4(w0), hi = fp8x4_to_bf16x4(w1);
      const u32x4_t packed = {lo.x, lo.y, hi.x, hi.y};
      a = __builtin_bit_cast(bf16x8_t, packed);
    }
    sc = mfma_qk<F16>(a, S.qop[kb], sc);
  }

  float kscale = P.scale_log2, vs = 1.f;
  if constexpr (FP8) {
    kscale *= B.ks;
    vs = B.vs;
  }

  // Online softmax over this page (exp2 domain).
  const uint32_t pos0 = pidx * 16u, so = block_in_page<PG>(T, pidx);
  const bool prefix = P.tau_scope == SCHED_PD_TAU_PREFIX;
  const bool full = pos0 + 16u <= T.n && (T.budget == 0xFFFFFFFFu ||
                                          (prefix ? pos0 + 16u <= T.budget : so + 16u <= T.budget));
  float s[4];
#pragma unroll
  for (int v = 0; v < 4; ++v)
    s[v] = sc[v] * kscale;
  if (!full) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const uint32_t i = 4u * g4 + v; // token in page (page size 16)
      const uint32_t t = pos0 + i;
      if (!(t < T.n && (prefix ? t : so + i) < T.budget))
        s[v] = kNegInf;
    }
  }
  const float pm = max_rows(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
  const float mnew = fmaxf(S.m, pm);
  if (__builtin_amdgcn_ballot_w64(mnew > S.m)) {
    const float c = __builtin_amdgcn_exp2f(S.m - mnew);
    S.lsum *= c;
#pragma unroll
    for (int blk = 0; blk < 8; ++blk)
      S.acc[blk] *= c;
  }
  S.m = mnew;
  float p[4];
#pragma unroll
  for (int v = 0; v < 4; ++v)
    p[v] = __builtin_amdgcn_exp2f(s[v] - mnew);
  S.lsum += (p[0] + p[1]) + (p[2] + p[3]);
  // P as PV's B operand. bf16 keeps 8 significant bits, which alone would
  // leave ~1.2e-3 relative error in the output (p is close to 1 for nearly
  // flat scores), so bf16 / fp8 carry p as hi + lo bf16 halves through two
  // MFMAs (~16 bits, the linear mode's split). fp16's 11 bits (~3e-4) are
  // kept single.
  u32x2_t pk, pl;
  if constexpr (F16) {
    pk.x = pack_f16_rne(p[0], p[1]);
    pk.y = pack_f16_rne(p[2], p[3]);
  } else {
    float pv[4];
#pragma unroll
    for (int v = 0; v < 4; ++v)
      pv[v] = FP8 ? p[v] * vs : p[v];
    pk.x = pack_bf16_rne(pv[0], pv[1]);
    pk.y = pack_bf16_rne(pv[2], pv[3]);
    pl.x = pack_bf16_rne(pv[0] - __uint_as_float(pk.x << 16),
                         pv[1] - __uint_as_float(pk.x & 0xffff0000u));
    pl.y = pack_bf16_rne(pv[2] - __uint_as_float(pk.y << 16),
                         pv[3] - __uint_as_float(pk.y & 0xffff0000u));
  }
  const s16x4_t pop = __builtin_bit_cast(s16x4_t, pk);

  // PV
  unsigned v8[8];
  u32x4_t vb[4];
  if constexpr (FP8 && VT) {
    fp8_vt_operands(B.v, v8);
  } else if constexpr (FP8) {
    fp8_v_operands(B.v, v8);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      vb[i] = B.v[i];
    if constexpr (!VT)
      bf16_v_operands(vb);
  }
#pragma unroll
  for (int blk = 0; blk < 8; ++blk) {
    s16x4_t a;
    if constexpr (VT && !FP8)
      a = bf16_vt_operand(vb, blk);
    else if constexpr (!FP8)
      a = __builtin_bit_cast(s16x4_t, (blk & 1) ? u32x2_t{vb[blk >> 1].z, vb[blk >> 1].w}
                                                : u32x2_t{vb[blk >> 1].x, vb[blk >> 1].y});
    else
      a = __builtin_bit_cast(s16x4_t, fp8x4_to_bf16x4(v8[blk]));
    S.acc[blk] = mfma_pv<F16>(a, pop, S.acc[blk]);
    if constexpr (!F16)
      S.acc[blk] = mfma_pv<false>(a, __builtin_bit_cast(s16x4_t, pl), S.acc[blk]);
  }
}

// Linear contraction of one page: acc[:, 0] += V^T . w over the page's kept
// tokens. w enters PV as column 0 of the B operand, split into bf16 hi + lo
// halves (two MFMAs) so the weights keep ~16 mantissa bits; V is exact.
template <bool FP8, bool VT, bool PG>
__device__ __forceinline__ void linear_page(const KParams &P, const MfmaTask &T, MfmaState &S,
                                            const PageRegs<FP8> &B, int32_t page, uint32_t pidx,
                                            uint32_t c16, uint32_t g4) {
  float vs = 1.f;
  if constexpr (FP8)
    vs = B.vs;
  const uint32_t pos0 = pidx * 16u, so = block_in_page<PG>(T, pidx);
  const bool prefix = P.tau_scope == SCHED_PD_TAU_PREFIX;
  float wv[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const uint32_t i = 4u * g4 + v, t = pos0 + i;
    const bool keep = c16 == 0u && t < T.n && (prefix ? t : so + i) < T.budget;
    wv[v] = keep ? B.lw[v] * vs : 0.f;
  }
  u32x2_t hi, lo;
  hi.x = pack_bf16_rne(wv[0], wv[1]);
  hi.y = pack_bf16_rne(wv[2], wv[3]);
  const float r0 = wv[0] - __uint_as_float(hi.x << 16), r1 = wv[1] - __uint_as_float(hi.x & 0xffff0000u);
  const float r2 = wv[2] - __uint_as_float(hi.y << 16), r3 = wv[3] - __uint_as_float(hi.y & 0xffff0000u);
  lo.x = pack_bf16_rne(r0, r1);
  lo.y = pack_bf16_rne(r2, r3);
  const s16x4_t bhi = __builtin_bit_cast(s16x4_t, hi), blo = __builtin_bit_cast(s16x4_t, lo);
  unsigned v8[8];
  u32x4_t vb[4];
  if constexpr (FP8 && VT) {
    fp8_vt_operands(B.v, v8);
  } else if constexpr (FP8) {
    fp8_v_operands(B.v, v8);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      vb[i] = B.v[i];
    if constexpr (!VT)
      bf16_v_operands(vb);
  }
#pragma unroll
  for (int blk = 0; blk < 8; ++blk) {
    s16x4_t a;
    if constexpr (VT && !FP8)
      a = bf16_vt_operand(vb, blk);
    else if constexpr (!FP8)
      a = __builtin_bit_cast(s16x4_t, (blk & 1) ? u32x2_t{vb[blk >> 1].z, vb[blk >> 1].w}
                                                : u32x2_t{vb[blk >> 1].x, vb[blk >> 1].y});
    else
      a = __builtin_bit_cast(s16x4_t, fp8x4_to_bf16x4(v8[blk]));
    S.acc[blk] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, bhi, S.acc[blk], 0, 0, 0);
    S.acc[blk] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, blo, S.acc[blk], 0, 0, 0);
  }
}

// Page id of the wave's i-th page (task page p0 + w + NW*i), read through the
// constant address space so it is a scalar load: it is counted by lgkmcnt, not
// by the vmcnt of the KV ring, and the ring's waits stay exact.
template <int NW, bool PG>
__device__ __forceinline__ int32_t page_id(const KParams &P, const MfmaTask &T, int i) {
  typedef const __attribute__((address_space(4))) int32_t cint32;
  const cint32 *bt = (const cint32 *)P.bt;
  if constexpr (PG) // block T.p0 + T.w + NW*i is in table entry block >> bshift
    return bt[T.row + ((T.p0 + T.w + NW * (uint32_t)i) >> T.bshift)];
  else
    return bt[T.row + T.p0 + T.w + (int64_t)NW * i];
}

// Stream the wave's pages with DEPTH pages of loads in flight. The steady
// loop has no branches: each computed page is followed by exactly one page's
// loads, so the compiler's s_waitcnt vmcnt values keep DEPTH-1 pages in flight
// (a conditional load in the loop makes it fall back to vmcnt(0), which
// drains the ring every page). Page ids come one group ahead from scalar
// loads at clamped indices (always inside the wave's table row). Pages go to
// waves round-robin, so the assignment (and with it every summation order)
// depends only on the page index, not on how many pages are read: a task whose
// shed pages are loaded and masked gives the same bits as one that skips them.
template <bool FP8, int NW, int DEPTH, bool NT, bool LINEAR, bool VT, bool PG, bool F16>
__device__ __forceinline__ void stream_pages(const KParams &P, const MfmaTask &T, MfmaState &S,
                                             uint32_t lane, uint32_t g4) {
  const uint32_t span = T.p1 - T.p0;
  const int npg = span > T.w ? (int)((span - T.w + NW - 1) / NW) : 0;
  if (npg <= 0)
    return;
  const int last = npg - 1;
  PageRegs<FP8> buf[DEPTH];
  int32_t pid[DEPTH], idn[DEPTH];
#pragma unroll
  for (int s = 0; s < DEPTH; ++s) {
    pid[s] = page_id<NW, PG>(P, T, min(s, last));
    idn[s] = page_id<NW, PG>(P, T, min(DEPTH + s, last));
  }
  // Unconditional prologue: a wave with fewer than DEPTH pages re-reads its
  // last page into the unused slots (same lines, L2 hits) so that the loop is
  // entered with the same DEPTH pages outstanding as on every back edge.
  auto pidx_of = [&](int j) __attribute__((always_inline)) { return T.p0 + T.w + NW * (uint32_t)j; };
#pragma unroll
  for (int s = 0; s < DEPTH; ++s)
    issue_page<FP8, NT, LINEAR, VT, PG>(P, T, pid[s], pidx_of(min(s, last)), buf[s]);

  auto compute = [&](int s, int j) __attribute__((always_inline)) {
    const uint32_t pidx = pidx_of(j);
    if constexpr (LINEAR)
      linear_page<FP8, VT, PG>(P, T, S, buf[s], pid[s], pidx, lane & 15u, g4);
    else
      compute_page<FP8, VT, PG, F16>(P, T, S, buf[s], pid[s], pidx, g4);
  };
  int j = 0;
  for (; j + 2 * DEPTH <= npg; j += DEPTH) {
#pragma unroll
    for (int s = 0; s < DEPTH; ++s) {
      compute(s, j + s);
      pid[s] = idn[s];
      issue_page<FP8, NT, LINEAR, VT, PG>(P, T, pid[s], pidx_of(j + DEPTH + s), buf[s]);
      idn[s] = page_id<NW, PG>(P, T, min(j + 2 * DEPTH + s, last));
    }
  }
  for (; j < npg; j += DEPTH) {
#pragma unroll
    for (int s = 0; s < DEPTH; ++s) {
      if (j + s < npg) {
        compute(s, j + s);
        if (j + DEPTH + s < npg) {
          pid[s] = idn[s];
          issue_page<FP8, NT, LINEAR, VT, PG>(P, T, pid[s], pidx_of(j + DEPTH + s), buf[s]);
        }
      }
    }
  }
}

// Fused append into an fp8 cache: the writer's rule for a one-token append
// (sched_kv_append) on the token's (page, kv-head h): the new K (and V)
// scale is pow2_scale of the token row's max |x|, or at least the page's
// old scale when the token is not the page's first (slot > 0); the row is
// encoded at it; when the scale grew, the page's earlier rows [0, slot) are
// re-encoded (decoded at the old scale, encoded at the new one); then the
// scales are stored. Lane l encodes dims 2l, 2l+1 of the new row (head dim
// 128, token-major V, one 2-byte store); a re-encode takes 8 bytes of four
// rows per pass (lanes 16i..16i+15 on row i), loading every row of a group
// of 16 before storing any. The source and scale loads go out together.
// The caller waits for the stores (vmcnt 0) before anything reads them.
__device__ __forceinline__ void regrow_rows_fp8(uint8_t *row0, int64_t tstride, uint32_t slot,
                                                float s_old, float inv, uint32_t lane) {
  const uint32_t sub = lane >> 4, off = 8u * (lane & 15u);
  for (uint32_t t0 = 0; t0 < slot; t0 += 16u) {
    u32x2_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t t = min(t0 + 4u * k + sub, slot - 1u); // clamped: re-read, not stored
      w[k] = *reinterpret_cast<const u32x2_t *>(row0 + (int64_t)t * tstride + off);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t t = t0 + 4u * k + sub;
      float q[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        q[i] = fp8e4m3_to_f32((w[k][i >> 2] >> (8 * (i & 3))) & 0xffu) * s_old * inv;
      if (t < slot)
        *reinterpret_cast<u32x2_t *>(row0 + (int64_t)t * tstride + off) =
            u32x2_t{encode4_fp8(q), encode4_fp8(q + 4)};
    }
  }
}

__device__ __forceinline__ void append_token_fp8(const KParams &P, uint32_t r, uint32_t h,
                                                 int64_t page, uint32_t slot, uint32_t lane) {
  const uint32_t j = 2u * lane;
  const int64_t src = (int64_t)r * P.app_ts + (int64_t)h * P.app_hs + j;
  const int64_t si = (page * P.Hkv + h) * P.scale_stride;
  float *scl[2] = {const_cast<float *>(P.k_scale) + si, const_cast<float *>(P.v_scale) + si};
  // the page's old scales matter only past its first slot (a token in slot
  // 0 starts the page afresh): not read otherwise
  float s_old[2] = {0.f, 0.f};
  if (slot > 0u) {
    s_old[0] = *scl[0];
    s_old[1] = *scl[1];
  }
  float x[2][2]; // [K, V][dim]
  for (int t = 0; t < 2; ++t) {
    const void *base = t ? P.app_v : P.app_k;
    if (P.app_f32) {
      const float *f = static_cast<const float *>(base) + src;
      x[t][0] = f[0], x[t][1] = f[1];
    } else {
      const uint32_t w = *reinterpret_cast<const uint32_t *>(static_cast<const uint16_t *>(base) +
                                                            src);
      if (P.app_f16) {
        const f16x2_t hv = __builtin_bit_cast(f16x2_t, w);
        x[t][0] = (float)hv.x, x[t][1] = (float)hv.y;
      } else {
        x[t][0] = bf16_bits_to_f32(w & 0xffffu), x[t][1] = bf16_bits_to_f32(w >> 16);
      }
    }
  }
  uint8_t *row0[2] = {
      static_cast<uint8_t *>(const_cast<void *>(P.k_pool)) + page * P.kps + (int64_t)h * P.khs,
      static_cast<uint8_t *>(const_cast<void *>(P.v_pool)) + page * P.vps + (int64_t)h * P.vhs};
  const int64_t tstride[2] = {P.kts, P.vts};
  float s_new[2];
  for (int t = 0; t < 2; ++t) {
    const float amax = wave_max(fmaxf(fabsf(x[t][0]), fabsf(x[t][1])));
    const float so = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(s_old[t])));
    const float p = pow2_scale(amax);
    const float sn = slot == 0u ? p : fmaxf(so, p);
    const float inv = sn > 0.f ? 1.f / sn : 0.f;
    s_new[t] = sn;
    *reinterpret_cast<uint16_t *>(row0[t] + (int64_t)slot * tstride[t] + j) =
        (uint16_t)encode2_fp8(x[t][0] * inv, x[t][1] * inv);
    if (slot > 0u && sn != so)
      regrow_rows_fp8(row0[t], tstride[t], slot, so, inv, lane);
  }
  if (lane == 0u) {
    *scl[0] = s_new[0];
    *scl[1] = s_new[1];
  }
}

// An urgent task's stream at the launch's ring depth: any depth in
// [DLO, DHI] the host accepted (SchedDecodeArgs.pf_dist); 0 = DHI. Every
// depth computes the same pages in the same order, so the bits do not change.
template <bool FP8, int NW, int DLO, int DHI, bool NT, bool LINEAR, bool VT, bool PG, bool F16>
__device__ __forceinline__ void stream_urgent(const KParams &P, const MfmaTask &T, MfmaState &S,
                                              uint32_t lane, uint32_t g4) {
  if constexpr (DLO < DHI) {
    if (P.pf_depth == (uint32_t)DLO) {
      stream_pages<FP8, NW, DLO, NT, LINEAR, VT, PG, F16>(P, T, S, lane, g4);
      return;
    }
    stream_urgent<FP8, NW, DLO + 1, DHI, NT, LINEAR, VT, PG, F16>(P, T, S, lane, g4);
  } else {
    stream_pages<FP8, NW, DHI, NT, LINEAR, VT, PG, F16>(P, T, S, lane, g4);
  }
}

template <bool FP8, int NW, int GMAX, int DEPTH_S, int DEPTH_U, bool LINEAR = false,
          bool VT = false, bool PG = false, bool F16 = false>
__global__ void __launch_bounds__(NW * 64) decode_mfma(KParams P) {
  static_assert(!(F16 && (FP8 || LINEAR)), "fp16: softmax over an fp16 cache");
  __shared__ float s_acc[NW][GMAX][128];
  __shared__ float s_m[NW][GMAX];
  __shared__ float s_l[NW][GMAX];
  const uint32_t lane = threadIdx.x & 63u;
  // Wave index as a scalar: everything per-wave (page slice, loop bounds,
  // page ids) then stays in SGPRs with uniform branches.
  const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t c16 = lane & 15u, g4 = lane >> 4;
  const bool toff = timer_off_latched(P.L);
  constexpr uint32_t EB = FP8 ? 1u : 2u; // bytes per KV element

  run_tasks(P.L, [&](uint32_t wi, bool last_round) __attribute__((always_inline)) {
    if (wi >= P.L.nitems)
      return;
    const unsigned long long t0 = read_clock(P.L.wallclock);
    const ItemRow I = item_row(P, wi);
    const uint32_t task = I.task;
    if (task >= P.ntasks)
      return;
    MfmaTask T;
    T.r = task / P.Hkv;
    T.h = task % P.Hkv;
    T.row = P.indptr ? (int64_t)__builtin_amdgcn_readfirstlane(P.indptr[T.r])
                     : (int64_t)T.r * P.bt_stride;
    const TaskPolicy pol = task_policy(P.L, task);
    T.n = ctx_tokens(P, T.r);
    T.budget = pol.budget;
    const uint32_t ext = load_extent(P, T.n, pol.budget);
    const ItemRange R = item_range(P, I, T.n, PG ? (ext + P.ps - 1u) / P.ps : (ext + 15u) / 16u);
    if (item_skip(P, wi, I, R))
      return;
    const bool stale = item_stale(P, wi, I, R, T.n);
    if constexpr (PG) {
      // pages [p0, p1) of the item as 16-token blocks, up to the last read.
      // A chunk wholly past a budget that ends inside a page has R.p0 =
      // R.p1 = the page count, whose first block lies past the last block
      // read: p0 is clamped to p1 so that the span is empty, never negative.
      T.bshift = 31u - __builtin_clz(P.ps >> 4);
      T.bmask = (1u << T.bshift) - 1u;
      T.p1 = min(R.p1 << T.bshift, (ext + 15u) / 16u);
      T.p0 = min(R.p0 << T.bshift, T.p1);
    } else {
      T.p0 = R.p0;
      T.p1 = R.p1;
    }
    T.w = w;
    bool wrote = false; // this wave stored the step's token (fused append)
    if constexpr (!LINEAR && VT) {
      // fused append: the item holding the new token writes it (in the
      // wave that streams its page) before streaming. A stale plan may hold
      // no item for that page; then chunk 0's item writes it too, so the
      // cache gets the token whatever the plan (the task's output is NaN
      // then, and a second writer stores the same bytes; an fp8 scale that
      // the first writer grew is not grown again by the second).
      if (P.app_k != nullptr && T.n > 0u) {
        const uint32_t pos = T.n - 1u, pg = pos / P.ps;
        const bool holds =
            P.tiles == nullptr ||
            (P.tile_ranged ? pg >= I.p0 && pg < I.p1 : I.chunk == pg / P.tile_pages);
        if (holds || (stale && I.chunk == 0u)) {
          const uint32_t rel = (PG ? pos / 16u : pg) - T.p0;
          if (rel % (uint32_t)NW == w) {
            const int64_t page = __builtin_amdgcn_readfirstlane(P.bt[T.row + pg]);
            if constexpr (FP8)
              append_token_fp8(P, T.r, T.h, page, pos % P.ps, lane);
            else
              append_token<F16>(P, T.r, T.h, page, pos % P.ps, lane);
            wrote = true;
          }
          // fp8 pages of several 16-token blocks: the re-encoded rows and the
          // new scale belong to blocks other waves stream
          if constexpr (FP8 && PG) {
            if (wrote)
              __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
            wrote = false;
            __syncthreads();
          }
        }
      }
    }
    T.kbase = static_cast<const uint8_t *>(P.k_pool) + (int64_t)c16 * P.kts * EB + 16u * g4;
    // fp8: whole row 16*g4 + c16; bf16: half g4/2 of row 16*(g4%2) + c16;
    // token-major: dims 8*c16.. of token 4*g4 (then rows 4*g4 + 1..3)
    T.vbase = static_cast<const uint8_t *>(P.v_pool) +
              (VT ? (int64_t)(4u * g4) * P.vts * EB + 8u * EB * c16
               : FP8 ? (int64_t)(c16 + 16u * g4) * P.vds
                     : (int64_t)(c16 + 16u * (g4 & 1u)) * P.vds * EB + 16u * (g4 >> 1));
    T.vrow_bytes = P.vts * EB;
    if constexpr (VT)
      T.vlane = (uint32_t)(4u * g4 * (uint32_t)T.vrow_bytes + 8u * EB * c16);
    else
      T.vlane = (uint32_t)(T.vbase - static_cast<const uint8_t *>(P.v_pool));
    T.ksub = 16 * P.kts * EB;
    T.vsub = VT ? 16 * P.vts * EB : 16 * (int64_t)EB;
    T.vblk = FP8 ? 64 * P.vds : 32 * P.vds * EB;
    T.kpage_bytes = P.kps * EB;
    T.khead_bytes = P.khs * EB * T.h;
    T.vpage_bytes = P.vps * EB;
    T.vhead_bytes = P.vhs * EB * T.h;

    MfmaState S;
    S.m = kMInit;
    S.lsum = 0.f;
#pragma unroll
    for (int blk = 0; blk < 8; ++blk)
      S.acc[blk] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const uint32_t G = LINEAR ? 1u : P.G;
    const int64_t qrow = ((int64_t)T.r * P.Hq + T.h * G + c16) * 128;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      u32x4_t qv = {0u, 0u, 0u, 0u};
      if (!LINEAR && c16 < G) {
        const uint32_t d0 = qk_dim(FP8, kb, g4);
        if (P.q_f32) {
          const float *qf = static_cast<const float *>(P.q) + qrow + d0;
          if constexpr (F16)
            qv = u32x4_t{pack_f16_rne(qf[0], qf[1]), pack_f16_rne(qf[2], qf[3]),
                         pack_f16_rne(qf[4], qf[5]), pack_f16_rne(qf[6], qf[7])};
          else
            qv = u32x4_t{pack_bf16_rne(qf[0], qf[1]), pack_bf16_rne(qf[2], qf[3]),
                         pack_bf16_rne(qf[4], qf[5]), pack_bf16_rne(qf[6], qf[7])};
        } else {
          qv = *reinterpret_cast<const u32x4_t *>(static_cast<const uint16_t *>(P.q) + qrow + d0);
        }
      }
      S.qop[kb] = __builtin_bit_cast(bf16x8_t, qv);
    }

    // the appended token is read back from the cache: its stores complete
    // first (issued before the Q loads above, so their latency overlaps)
    if (wrote)
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    if ((T.p1 - T.p0 > kLongItemPages || (kLateDeep && last_round)) && !pol.polite)
      stream_pages<FP8, NW, DEPTH_U, false, LINEAR, VT, PG, F16>(P, T, S, lane, g4);
    else if (pol.urgent)
      stream_urgent<FP8, NW, DEPTH_S, DEPTH_U, kStockNT, LINEAR, VT, PG, F16>(P, T, S, lane, g4);
    else if (pol.polite)
      stream_pages<FP8, NW, DEPTH_S, true, LINEAR, VT, PG, F16>(P, T, S, lane, g4);
    else
      stream_pages<FP8, NW, DEPTH_S, kStockNT, LINEAR, VT, PG, F16>(P, T, S, lane, g4);

    // Wave states to LDS (l summed over the 4 lane rows first), then the
    // work item's result: output, or partial + fixed-order task merge.
    const float lt = sum_rows(S.lsum);
    if (c16 < G) {
      if (g4 == 0) {
        s_m[w][c16] = S.m;
        s_l[w][c16] = lt;
      }
      if constexpr (VT) {
        // row 4*g4 + i of block blk is dim 8*(4*g4 + i) + blk
#pragma unroll
        for (int blk = 0; blk < 8; ++blk)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            s_acc[w][c16][8 * (4 * g4 + i) + blk] = S.acc[blk][i];
      } else {
#pragma unroll
        for (int blk = 0; blk < 8; ++blk)
          *reinterpret_cast<f32x4_t *>(&s_acc[w][c16][16 * blk + 4 * g4]) = S.acc[blk];
      }
    }
    __syncthreads();
    if (stale)
      mark_stale<NW, 128, LINEAR>(P, I.chunk, T.r, T.h, G);
    else
      finish_item<NW, GMAX, 128, float, LINEAR>(P, wi, task, I.chunk, R.nchunks, T.r, T.h, G,
                                                s_acc, s_m, s_l);
    timer_commit(P.L, toff, task, t0);
  });
}

} // namespace schedpd
