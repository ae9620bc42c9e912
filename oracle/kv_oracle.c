/* kv_oracle.c -- CPU restatement of the paged KV-cache writer. TEST
 * INFRASTRUCTURE ONLY: tests/ compare sched_kv_append's output pools and
 * scales with this, byte for byte; no product code links, loads or calls it.
 *
 * What it restates:
 *   - the append position rule of FlashInfer's append_paged_kv_cache
 *     (flashinfer-python==0.6.12, pinned at the reference's
 *     requirements.txt:6; not vendored in the reference): request r's n_r new
 *     rows land at positions seq_len_r - n_r .. seq_len_r - 1, position p in
 *     page-table entry p / page_size, slot p % page_size, over the CSR page
 *     table the reference's tests build (test/py/eval_pi_makespan.py:46-60)
 *     or a 2-D block table;
 *   - fp32 -> bf16 round-to-nearest-even;
 *   - fp32 -> IEEE binary16 round-to-nearest-even, written from the format
 *     definition (5 exponent bits bias 15, 10 mantissa bits, subnormals
 *     m * 2^-24, overflow to infinity from 65520 up); NaN payloads are not
 *     restated (any NaN becomes the quiet NaN 0x7e00 with its sign);
 *   - OCP e4m3fn encoding with round-to-nearest-even and saturation to 448,
 *     written from the format definition (sign, 4 exponent bits bias 7, 3
 *     mantissa bits, subnormals m * 2^-9, no infinity);
 *   - the cache's scale rule for fp8 (per (page, kv-head), powers of two,
 *     grown and re-encoded on later appends), as specified in
 *     include/sched_kv.h.
 * Loops are serial and in the order a reader would write them.
 */
#include "../include/sched_kv.h"

#include <math.h>
#include <stdint.h>
#include <string.h>

float oracle_bf16_to_float(uint16_t h);
float oracle_fp8_e4m3_to_float(uint8_t b);
float oracle_f16_to_float(uint16_t h);

uint16_t oracle_float_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u)
    return (uint16_t)((u >> 16) | 0x40u);
  uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

/* Round-to-nearest-even to binary16. */
uint16_t oracle_float_to_f16(float x) {
  uint16_t sign = signbit(x) ? 0x8000 : 0x0000;
  float a = fabsf(x);
  if (isnan(x))
    return sign | 0x7e00;
  if (a >= 65520.0f) /* the midpoint between 65504 and 2^16 rounds to even: up */
    return sign | 0x7c00;
  if (a < 6.103515625e-05f) { /* below 2^-14: subnormal grid m * 2^-24 */
    float m = nearbyintf(a * 16777216.0f); /* exact scaling, then RNE */
    return sign | (uint16_t)m;             /* m == 1024 is the first normal */
  }
  int e;
  float f = frexpf(a, &e);                         /* a = f * 2^e, f in [0.5, 1) */
  float q = nearbyintf((f * 2.0f - 1.0f) * 1024.0f); /* 10 mantissa bits, RNE */
  int exp = e - 1;
  if (q == 1024.0f) {
    q = 0.0f;
    exp += 1;
  }
  return sign | (uint16_t)(((exp + 15) << 10) | (int)q);
}

/* Round-to-nearest-even to e4m3fn, saturating finite values at +-448. */
uint8_t oracle_fp8_e4m3_from_float(float x) {
  uint8_t sign = signbit(x) ? 0x80 : 0x00;
  float a = fabsf(x);
  if (isnan(x))
    return sign | 0x7f;
  if (a >= 448.0f)
    return sign | 0x7e;
  if (a < 0.015625f) { /* below 2^-6: subnormal grid m * 2^-9, m = 0..8 */
    float m = nearbyintf(a * 512.0f); /* exact scaling, then RNE */
    return sign | (uint8_t)m;         /* m == 8 is the first normal, 0x08 */
  }
  int e;
  float f = frexpf(a, &e);                  /* a = f * 2^e, f in [0.5, 1) */
  float q = nearbyintf((f * 2.0f - 1.0f) * 8.0f); /* 3 mantissa bits, RNE */
  int exp = e - 1;                           /* a = (1 + q/8) * 2^exp */
  if (q == 8.0f) {
    q = 0.0f;
    exp += 1;
  }
  int code = ((exp + 7) << 3) | (int)q;
  if (code > 0x7e)
    code = 0x7e;
  return sign | (uint8_t)code;
}

float oracle_pow2_scale(float a) {
  if (!(a > 0.0f))
    return 0.0f;
  int e;
  float m = frexpf(a, &e);
  int k = e - 9 + (m > 0.875f ? 1 : 0);
  return ldexpf(1.0f, k < -126 ? -126 : k);
}

static uint32_t esize(uint32_t dt) {
  return dt == SCHED_PD_F32 ? 4u : dt == SCHED_PD_FP8_E4M3 ? 1u : 2u;
}

static float src_at(const SchedKvAppendArgs *a, const void *src, int64_t row, uint32_t h,
                    uint32_t j) {
  int64_t i = row * a->src_tok_stride + (int64_t)h * a->src_head_stride + j;
  if (a->src_dtype == SCHED_PD_F32)
    return ((const float *)src)[i];
  if (a->src_dtype == SCHED_PD_F16)
    return oracle_f16_to_float(((const uint16_t *)src)[i]);
  return oracle_bf16_to_float(((const uint16_t *)src)[i]);
}

static float code_value(const void *pool, int64_t i, uint32_t dt) {
  if (dt == SCHED_PD_F32)
    return ((const float *)pool)[i];
  if (dt == SCHED_PD_BF16)
    return oracle_bf16_to_float(((const uint16_t *)pool)[i]);
  if (dt == SCHED_PD_F16)
    return oracle_f16_to_float(((const uint16_t *)pool)[i]);
  return oracle_fp8_e4m3_to_float(((const uint8_t *)pool)[i]);
}

static void put(void *pool, int64_t i, uint32_t dt, float x, float inv) {
  if (dt == SCHED_PD_F32) {
    ((float *)pool)[i] = x;
  } else if (dt == SCHED_PD_BF16) {
    ((uint16_t *)pool)[i] = oracle_float_to_bf16(x);
  } else if (dt == SCHED_PD_F16) {
    ((uint16_t *)pool)[i] = oracle_float_to_f16(x);
  } else {
    float q = fminf(fmaxf(x * inv, -448.0f), 448.0f);
    ((uint8_t *)pool)[i] = oracle_fp8_e4m3_from_float(q);
  }
}

/* One tensor of one (page, head). Element (slot t, dim j) at
 * base + t*tok + j*dim. */
static void write_tensor(const SchedKvAppendArgs *a, const void *src, void *pool, int64_t base,
                         int64_t tok, int64_t dim, float *scale, uint32_t o0, uint32_t o1,
                         int64_t row0, uint32_t h) {
  const uint32_t dt = a->kv_dtype, d = a->head_dim;
  float inv = 0.0f;
  if (dt == SCHED_PD_FP8_E4M3) {
    float amax = 0.0f;
    for (uint32_t t = o0; t < o1; ++t)
      for (uint32_t j = 0; j < d; ++j)
        amax = fmaxf(amax, fabsf(src_at(a, src, row0 + (t - o0), h, j)));
    float s_old = *scale, p = oracle_pow2_scale(amax);
    float s_new = o0 == 0 ? p : fmaxf(s_old, p);
    inv = s_new > 0.0f ? 1.0f / s_new : 0.0f;
    if (o0 > 0 && s_new != s_old) /* re-encode the page's earlier slots */
      for (uint32_t t = 0; t < o0; ++t)
        for (uint32_t j = 0; j < d; ++j) {
          int64_t i = base + t * tok + j * dim;
          put(pool, i, dt, code_value(pool, i, dt) * s_old, inv);
        }
    *scale = s_new;
  }
  for (uint32_t t = o0; t < o1; ++t)
    for (uint32_t j = 0; j < d; ++j)
      put(pool, base + t * tok + j * dim, dt, src_at(a, src, row0 + (t - o0), h, j), inv);
  /* d-major V is written in 4-slot groups: the unused slots after the last
   * appended one, up to the group's end, are zero */
  if (tok == 1 && dim != 1)
    for (uint32_t t = o1; t < ((o1 + 3u) & ~3u); ++t)
      for (uint32_t j = 0; j < d; ++j)
        put(pool, base + t * tok + j * dim, dt, 0.0f, inv);
}

/* Host-memory restatement of sched_kv_append (same argument struct, host
 * pointers). Returns the number of (token, kv-head) pairs it could not write,
 * the kernel's `errors` count. */
long oracle_kv_append(const SchedKvAppendArgs *a) {
  long errors = 0;
  const int vdm = a->v_tok_stride == 1 && a->v_dim_stride != 1;
  const int64_t vts = vdm ? 1 : a->v_tok_stride, vds = vdm ? a->v_dim_stride : 1;
  (void)esize;
  for (uint32_t r = 0; r < a->num_requests; ++r) {
    int64_t a0 = a->append_indptr[r], a1 = a->append_indptr[r + 1];
    if (a1 <= a0)
      continue;
    int64_t n = a1 - a0, ctx = a->ctx_lens[r], pos0 = ctx - n;
    if (a0 < 0 || a1 > (int64_t)a->num_tokens || pos0 < 0) {
      errors += n * a->num_kv_heads;
      continue;
    }
    int64_t row = a->page_indptr ? a->page_indptr[r] : (int64_t)r * a->bt_stride;
    int64_t cap = a->page_indptr ? (int64_t)a->page_indptr[r + 1] - a->page_indptr[r]
                                 : (int64_t)a->bt_stride;
    for (uint32_t h = 0; h < a->num_kv_heads; ++h)
      for (int64_t b = pos0 / a->page_size; b <= (ctx - 1) / a->page_size; ++b) {
        int64_t pbase = b * a->page_size;
        uint32_t o0 = (uint32_t)(pos0 > pbase ? pos0 - pbase : 0);
        uint32_t o1 = (uint32_t)(ctx - pbase < a->page_size ? ctx - pbase : a->page_size);
        int64_t page = b < cap ? a->block_table[row + b] : -1;
        if (page < 0 || (uint64_t)page >= a->num_pages) {
          errors += o1 - o0;
          continue;
        }
        int64_t row0 = a0 + (pbase + o0 - pos0), si = page * a->num_kv_heads + h;
        write_tensor(a, a->k_src, a->k_pool, page * a->k_page_stride + h * a->k_head_stride,
                     a->k_tok_stride, 1, a->k_scale ? a->k_scale + si : NULL, o0, o1, row0, h);
        write_tensor(a, a->v_src, a->v_pool, page * a->v_page_stride + h * a->v_head_stride,
                     vts, vds, a->v_scale ? a->v_scale + si : NULL, o0, o1, row0, h);
      }
  }
  return errors;
}

int oracle_kv_args_layout(int64_t *out, int n) {
  int64_t v[] = {
      (int64_t)sizeof(SchedKvAppendArgs),
      (int64_t)offsetof(SchedKvAppendArgs, num_pages),
      (int64_t)offsetof(SchedKvAppendArgs, k_src),
      (int64_t)offsetof(SchedKvAppendArgs, src_tok_stride),
      (int64_t)offsetof(SchedKvAppendArgs, append_indptr),
      (int64_t)offsetof(SchedKvAppendArgs, k_pool),
      (int64_t)offsetof(SchedKvAppendArgs, k_page_stride),
      (int64_t)offsetof(SchedKvAppendArgs, v_dim_stride),
      (int64_t)offsetof(SchedKvAppendArgs, k_scale),
      (int64_t)offsetof(SchedKvAppendArgs, errors),
  };
  int k = (int)(sizeof v / sizeof v[0]);
  for (int i = 0; i < k && i < n; ++i)
    out[i] = v[i];
  return k;
}
