/* oracle.c -- CPU restatement of the reference's truncated paged-attention
 * path. TEST INFRASTRUCTURE ONLY: this file gives the expected values the
 * HIP kernels are compared against (tests/), and the CPU baseline that
 * bench.py times beside them. No product code links, loads or calls it.
 *
 * What it restates (reference file:line):
 *   - softmax decode: the online-softmax CPU reference with the -1e30 running
 *     max and skip-not-mask semantics, test/paged_decode.cu:124-153 (one
 *     request, one head, paged K/V, `continue` on dropped tokens so they get
 *     zero weight and leave the max and denominator untouched), extended to
 *     per-request page counts as in test/py/test_dynamic_loop.py:77-100, and
 *     to GQA (q-head group per kv-head) and a partial last page.
 *   - linear contraction: test/paged_decode.cu:155-181 (acc += kv*w) with the
 *     weight indexed by position (paged_decode, :55) or by token-in-page
 *     (test/hetero_batch.cu:72), and the shed value mask v' = keep ? v : 0
 *     (lib/SchedWeave.cpp:672-700).
 *   - shed budget: budget = (ctrl && task < max) ? (tau ? tau : inf) : inf
 *     (lib/SchedWeave.cpp:585-614); keep = counter < budget where the counter
 *     is the token position in the request (prefix scope) or within its page
 *     (per-page scope, the reference fixtures' innermost loop IV).
 *   - dequantisation: bf16 (upper half of an IEEE float), IEEE binary16, and
 *     OCP fp8 e4m3fn (1 sign, 4 exponent bits bias 7, 3 mantissa bits, no
 *     inf, S.1111.111 = NaN) times a per-(page, kv-head) fp32 scale.
 *
 * Two precisions:
 *   ORACLE_F64: every product and sum in double -- the expected values;
 *   ORACLE_F32: the reference CPU loop as written, in float with expf -- the
 *               "port" CPU baseline, parallelised over tasks with OpenMP.
 */
#include "../include/sched_pd.h"

#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_F64 0
#define ORACLE_F32 1

float oracle_bf16_to_float(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* IEEE binary16 decode, from the format definition (1 sign, 5 exponent bits
 * bias 15, 10 mantissa bits; exponent 0 subnormal, 31 inf / NaN). */
float oracle_f16_to_float(uint16_t h) {
  int s = (h >> 15) & 1, e = (h >> 10) & 31, m = h & 1023;
  float v;
  if (e == 31)
    v = m ? NAN : INFINITY;
  else if (e == 0)
    v = ldexpf((float)m, -24); /* m/1024 * 2^-14 */
  else
    v = ldexpf((float)(1024 + m), e - 25); /* (1+m/1024) * 2^(e-15) */
  return s ? -v : v;
}

/* OCP e4m3fn decode, from the format definition. */
float oracle_fp8_e4m3_to_float(uint8_t b) {
  int s = (b >> 7) & 1, e = (b >> 3) & 15, m = b & 7;
  float v;
  if (e == 15 && m == 7)
    v = NAN;
  else if (e == 0)
    v = ldexpf((float)m, -9); /* m/8 * 2^-6 */
  else
    v = ldexpf((float)(8 + m), e - 10); /* (1+m/8) * 2^(e-7) */
  return s ? -v : v;
}

static double load_elem(const void *base, int64_t idx, uint32_t dtype) {
  switch (dtype) {
  case SCHED_PD_F32:
    return ((const float *)base)[idx];
  case SCHED_PD_BF16:
    return oracle_bf16_to_float(((const uint16_t *)base)[idx]);
  case SCHED_PD_F16:
    return oracle_f16_to_float(((const uint16_t *)base)[idx]);
  default:
    return oracle_fp8_e4m3_to_float(((const uint8_t *)base)[idx]);
  }
}

static int64_t page_of(const SchedDecodeArgs *a, uint32_t r, int64_t b) {
  if (a->page_indptr)
    return a->block_table[a->page_indptr[r] + b];
  return a->block_table[(int64_t)r * a->bt_stride + b];
}

/* lib/SchedWeave.cpp:585-614: 0xFFFFFFFF = no cap. */
static uint32_t budget_of(const SchedDecodeArgs *a, const void *ctrl_host,
                          uint32_t task) {
  if (!ctrl_host || task >= a->max_tasks)
    return 0xFFFFFFFFu;
  const uint8_t *row = (const uint8_t *)ctrl_host + SCHED_CTRL_ROWS_OFF +
                       (size_t)task * SCHED_CTRL_ROW_SIZE;
  uint16_t tau;
  memcpy(&tau, row + SCHED_CTRL_ROW_TAU_OFF, 2);
  return tau ? (uint32_t)tau : 0xFFFFFFFFu;
}

static int keep_token(const SchedDecodeArgs *a, uint32_t budget, int64_t pos) {
  if (budget == 0xFFFFFFFFu)
    return 1;
  int64_t ctr = a->tau_scope == SCHED_PD_TAU_PER_PAGE ? pos % a->page_size : pos;
  return ctr < (int64_t)budget;
}

static int64_t ctx_tokens(const SchedDecodeArgs *a, uint32_t r) {
  int64_t c = a->ctx_lens[r];
  return (a->flags & SCHED_PD_FLAG_CTX_IN_PAGES) ? c * a->page_size : c;
}

static double kscale(const SchedDecodeArgs *a, int64_t page, uint32_t h) {
  return (a->kv_dtype == SCHED_PD_FP8_E4M3 && a->k_scale)
             ? a->k_scale[page * a->num_kv_heads + h] : 1.0;
}
static double vscale(const SchedDecodeArgs *a, int64_t page, uint32_t h) {
  return (a->kv_dtype == SCHED_PD_FP8_E4M3 && a->v_scale)
             ? a->v_scale[page * a->num_kv_heads + h] : 1.0;
}

/* One task (request r, kv-head h), fp64. */
static void task_f64(const SchedDecodeArgs *a, const void *ctrl_host,
                     uint32_t r, uint32_t h, double *out) {
  const uint32_t d = a->head_dim, ps = a->page_size;
  const uint32_t task = r * a->num_kv_heads + h;
  const uint32_t budget = budget_of(a, ctrl_host, task);
  const int64_t n = ctx_tokens(a, r);
  const double scale = a->sm_scale != 0.f ? (double)a->sm_scale : 1.0 / sqrt((double)d);

  if (a->mode == SCHED_PD_LINEAR) {
    double *o = out + ((size_t)r * a->num_kv_heads + h) * d;
    for (uint32_t j = 0; j < d; ++j)
      o[j] = 0.0;
    for (int64_t t = 0; t < n; ++t) {
      if (!keep_token(a, budget, t))
        continue; /* value masked to 0: the term vanishes */
      int64_t page = page_of(a, r, t / ps), i = t % ps;
      double w = a->lin_w[a->lin_w_period ? t % a->lin_w_period : t];
      double vs = vscale(a, page, h);
      for (uint32_t j = 0; j < d; ++j) {
        int64_t vi = page * a->v_page_stride + (int64_t)h * a->v_head_stride +
                     i * a->v_tok_stride + (int64_t)j * a->v_dim_stride;
        o[j] += w * (load_elem(a->v_pool, vi, a->kv_dtype) * vs);
      }
    }
    return;
  }

  const uint32_t G = a->num_q_heads / a->num_kv_heads;
  for (uint32_t g = 0; g < G; ++g) {
    const uint32_t hq = h * G + g;
    const int64_t qoff = ((int64_t)r * a->num_q_heads + hq) * d;
    double *o = out + qoff;
    double m = -1e30, l = 0.0;
    for (uint32_t j = 0; j < d; ++j)
      o[j] = 0.0;
    for (int64_t t = 0; t < n; ++t) {
      if (!keep_token(a, budget, t))
        continue; /* -inf score: zero weight, max and denominator untouched */
      int64_t page = page_of(a, r, t / ps), i = t % ps;
      double s = 0.0, ks = kscale(a, page, h), vs = vscale(a, page, h);
      for (uint32_t j = 0; j < d; ++j) {
        int64_t ki = page * a->k_page_stride + (int64_t)h * a->k_head_stride +
                     i * a->k_tok_stride + j;
        s += load_elem(a->q, qoff + j, a->q_dtype) *
             (load_elem(a->k_pool, ki, a->kv_dtype) * ks);
      }
      s *= scale;
      double mn = s > m ? s : m;
      double c = exp(m - mn), w = exp(s - mn);
      l = l * c + w;
      for (uint32_t j = 0; j < d; ++j) {
        int64_t vi = page * a->v_page_stride + (int64_t)h * a->v_head_stride +
                     i * a->v_tok_stride + (int64_t)j * a->v_dim_stride;
        o[j] = o[j] * c + w * (load_elem(a->v_pool, vi, a->kv_dtype) * vs);
      }
      m = mn;
    }
    for (uint32_t j = 0; j < d; ++j)
      o[j] = o[j] / l;
  }
}

/* One task in float, the reference loop (test/paged_decode.cu:128-151). The
 * reference recomputes the score inside its per-lane loop; every lane gets the
 * same float sequence, so it is computed once per token here, which gives the
 * same bits d times faster. */
static void task_f32(const SchedDecodeArgs *a, const void *ctrl_host,
                     uint32_t r, uint32_t h, float *out) {
  const uint32_t d = a->head_dim, ps = a->page_size;
  const uint32_t task = r * a->num_kv_heads + h;
  const uint32_t budget = budget_of(a, ctrl_host, task);
  const int64_t n = ctx_tokens(a, r);
  const float scale = a->sm_scale != 0.f ? a->sm_scale : 1.0f / sqrtf((float)d);

  if (a->mode == SCHED_PD_LINEAR) {
    float *o = out + ((size_t)r * a->num_kv_heads + h) * d;
    for (uint32_t j = 0; j < d; ++j) {
      float acc = 0.f;
      for (int64_t t = 0; t < n; ++t) {
        if (!keep_token(a, budget, t))
          continue;
        int64_t page = page_of(a, r, t / ps), i = t % ps;
        int64_t vi = page * a->v_page_stride + (int64_t)h * a->v_head_stride +
                     i * a->v_tok_stride + (int64_t)j * a->v_dim_stride;
        acc += (float)load_elem(a->v_pool, vi, a->kv_dtype) * (float)vscale(a, page, h) *
               a->lin_w[a->lin_w_period ? t % a->lin_w_period : t];
      }
      o[j] = acc;
    }
    return;
  }

  const uint32_t G = a->num_q_heads / a->num_kv_heads;
  for (uint32_t g = 0; g < G; ++g) {
    const uint32_t hq = h * G + g;
    const int64_t qoff = ((int64_t)r * a->num_q_heads + hq) * d;
    float *o = out + qoff;
    float acc[256], qv[256];
    for (uint32_t j = 0; j < d; ++j) {
      acc[j] = 0.f;
      qv[j] = (float)load_elem(a->q, qoff + j, a->q_dtype);
    }
    float m = -1e30f, l = 0.f;
    for (int64_t t = 0; t < n; ++t) {
      if (!keep_token(a, budget, t))
        continue;
      int64_t page = page_of(a, r, t / ps), i = t % ps;
      float ks = (float)kscale(a, page, h), vs = (float)vscale(a, page, h);
      float s = 0.f;
      for (uint32_t j = 0; j < d; ++j) {
        int64_t ki = page * a->k_page_stride + (int64_t)h * a->k_head_stride +
                     i * a->k_tok_stride + j;
        s += (float)load_elem(a->k_pool, ki, a->kv_dtype) * ks * qv[j];
      }
      s *= scale;
      float mn = s > m ? s : m;
      float c = expf(m - mn), w = expf(s - mn);
      l = l * c + w;
      for (uint32_t lane = 0; lane < d; ++lane) {
        int64_t vi = page * a->v_page_stride + (int64_t)h * a->v_head_stride +
                     i * a->v_tok_stride + (int64_t)lane * a->v_dim_stride;
        acc[lane] = acc[lane] * c +
                    w * ((float)load_elem(a->v_pool, vi, a->kv_dtype) * vs);
      }
      m = mn;
    }
    for (uint32_t lane = 0; lane < d; ++lane)
      o[lane] = acc[lane] / l;
  }
}

/* Decode every task of `a` (host pointers). ctrl_host: SchedCtrl-layout bytes
 * or NULL (reads only the rows' tau). precision ORACLE_F64 writes out_f64,
 * ORACLE_F32 writes out_f32. threads <= 0: OpenMP default. Returns 0, or -1
 * on arguments it does not accept. */
int oracle_decode(const SchedDecodeArgs *a, const void *ctrl_host,
                  double *out_f64, float *out_f32, int precision, int threads) {
  if (!a || a->head_dim == 0 || a->head_dim > 256 || a->page_size == 0 ||
      a->num_kv_heads == 0)
    return -1;
  if (a->mode == SCHED_PD_SOFTMAX &&
      (a->num_q_heads == 0 || a->num_q_heads % a->num_kv_heads))
    return -1;
  if ((precision == ORACLE_F64 && !out_f64) || (precision == ORACLE_F32 && !out_f32))
    return -1;
  const int64_t ntasks = (int64_t)a->num_requests * a->num_kv_heads;
#ifdef _OPENMP
  if (threads > 0)
    omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 1)
#endif
  for (int64_t t = 0; t < ntasks; ++t) {
    uint32_t r = (uint32_t)(t / a->num_kv_heads), h = (uint32_t)(t % a->num_kv_heads);
    if (precision == ORACLE_F64)
      task_f64(a, ctrl_host, r, h, out_f64);
    else
      task_f32(a, ctrl_host, r, h, out_f32);
  }
  return 0;
}

int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* Byte size and field offsets of SchedDecodeArgs as this C compiler lays it
 * out, so the tests can compare them with the ctypes mirror. Order:
 * sizeof, then the offsets of sm_scale, lin_w_period, q, k_page_stride,
 * v_dim_stride, k_scale, block_table, lin_w, order, queue. */
int oracle_args_layout(int64_t *out, int n) {
  const int64_t v[] = {
      (int64_t)sizeof(SchedDecodeArgs),
      (int64_t)offsetof(SchedDecodeArgs, sm_scale),
      (int64_t)offsetof(SchedDecodeArgs, lin_w_period),
      (int64_t)offsetof(SchedDecodeArgs, q),
      (int64_t)offsetof(SchedDecodeArgs, k_page_stride),
      (int64_t)offsetof(SchedDecodeArgs, v_dim_stride),
      (int64_t)offsetof(SchedDecodeArgs, k_scale),
      (int64_t)offsetof(SchedDecodeArgs, block_table),
      (int64_t)offsetof(SchedDecodeArgs, lin_w),
      (int64_t)offsetof(SchedDecodeArgs, order),
      (int64_t)offsetof(SchedDecodeArgs, queue),
      (int64_t)sizeof(SchedCtrl),
      (int64_t)offsetof(SchedDecodeArgs, tile_pages),
      (int64_t)offsetof(SchedDecodeArgs, tiles),
      (int64_t)offsetof(SchedDecodeArgs, num_tiles),
      (int64_t)offsetof(SchedDecodeArgs, workspace),
      (int64_t)offsetof(SchedDecodeArgs, workspace_bytes),
  };
  int m = (int)(sizeof v / sizeof v[0]);
  for (int i = 0; i < m && i < n; ++i)
    out[i] = v[i];
  return m;
}
