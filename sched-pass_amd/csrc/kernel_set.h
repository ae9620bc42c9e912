// kernel_set.h -- every decode kernel the launcher can select, and the tuning
// constants of the MFMA ones. paged_decode.hip declares them (extern
// template); the kernels_*.hip files instantiate them, one group per
// translation unit so that the library compiles in parallel.
#pragma once

#include "decode_mfma.h"
#include "decode_valu.h"
#include "decode_wave.h"

// MFMA kernel shape: waves per workgroup, pages in flight per wave (stock,
// urgent). Overridable at build time for tuning sweeps.
#ifndef SCHED_PD_MFMA_NW
#define SCHED_PD_MFMA_NW 4
#endif
#ifndef SCHED_PD_MFMA_DEPTH
#define SCHED_PD_MFMA_DEPTH 2
#endif
#ifndef SCHED_PD_MFMA_DEPTH_URGENT
#define SCHED_PD_MFMA_DEPTH_URGENT 4
#endif
// fp8 pages are half the bytes: twice the pages in flight for the same bytes.
#ifndef SCHED_PD_MFMA_DEPTH_FP8
#define SCHED_PD_MFMA_DEPTH_FP8 4
#endif
#ifndef SCHED_PD_MFMA_DEPTH_FP8_URGENT
#define SCHED_PD_MFMA_DEPTH_FP8_URGENT 6
#endif
// Token-major V keeps its row pieces for the in-lane operand build: an urgent
// ring of 4 pages would need 270 VGPRs (one wave per SIMD); 3 fits in 229.
#ifndef SCHED_PD_MFMA_DEPTH_VT_URGENT
#define SCHED_PD_MFMA_DEPTH_VT_URGENT 3
#endif
// fp8 token-major V: at the fp8 urgent depth of 6 the kernel needs 274
// VGPRs (and spills with page blocks); 4 keeps it in the register file.
#ifndef SCHED_PD_MFMA_DEPTH_FP8_VT_URGENT
#define SCHED_PD_MFMA_DEPTH_FP8_VT_URGENT 4
#endif
// fp8 d-major V on pages of 32..256 tokens: depth 6 needs 258 VGPRs (one wave
// per SIMD instead of two); 5 fits in the register file.
#ifndef SCHED_PD_MFMA_DEPTH_FP8_PG_URGENT
#define SCHED_PD_MFMA_DEPTH_FP8_PG_URGENT 5
#endif
// fp16 d-major V on 16-token pages: depth 4 needs 258 VGPRs; 3 fits.
#ifndef SCHED_PD_MFMA_DEPTH_F16_URGENT
#define SCHED_PD_MFMA_DEPTH_F16_URGENT 3
#endif

namespace schedpd {

constexpr int mfma_ds(bool fp8) { return fp8 ? SCHED_PD_MFMA_DEPTH_FP8 : SCHED_PD_MFMA_DEPTH; }
// Deepest ring (the urgent default). An urgent task's ring depth is any of
// mfma_ds .. mfma_du (SchedDecodeArgs.pf_dist).
constexpr int mfma_du(bool fp8, bool vt, bool pg, bool f16 = false) {
  return fp8 ? (vt ? SCHED_PD_MFMA_DEPTH_FP8_VT_URGENT
                : pg ? SCHED_PD_MFMA_DEPTH_FP8_PG_URGENT
                     : SCHED_PD_MFMA_DEPTH_FP8_URGENT)
         : vt ? SCHED_PD_MFMA_DEPTH_VT_URGENT
         : (f16 && !pg) ? SCHED_PD_MFMA_DEPTH_F16_URGENT
                        : SCHED_PD_MFMA_DEPTH_URGENT;
}

} // namespace schedpd

// One MFMA variant (kv format, V layout, page blocks, fp16): the softmax
// kernels for up to 4 / 8 / 16 q-heads per kv-head, and (LIN) the linear one.
#define SCHED_PD_MFMA_ONE(PRE, FP8, GMAX, LIN, VT, PG, F16)                                      \
  PRE template __global__ void schedpd::decode_mfma<FP8, SCHED_PD_MFMA_NW, GMAX,                 \
                                                    schedpd::mfma_ds(FP8),                       \
                                                    schedpd::mfma_du(FP8, VT, PG, F16), LIN, VT, PG, F16>( \
      schedpd::KParams);
#define SCHED_PD_MFMA_SOFTMAX(PRE, FP8, VT, PG, F16)                                             \
  SCHED_PD_MFMA_ONE(PRE, FP8, 4, false, VT, PG, F16)                                             \
  SCHED_PD_MFMA_ONE(PRE, FP8, 8, false, VT, PG, F16)                                             \
  SCHED_PD_MFMA_ONE(PRE, FP8, 16, false, VT, PG, F16)
#define SCHED_PD_MFMA_WITH_LINEAR(PRE, FP8, VT, PG)                                              \
  SCHED_PD_MFMA_SOFTMAX(PRE, FP8, VT, PG, false)                                                 \
  SCHED_PD_MFMA_ONE(PRE, FP8, 4, true, VT, PG, false)

// The groups, one per translation unit.
#define SCHED_PD_MFMA_BF16_PAGE16(PRE)                                                           \
  SCHED_PD_MFMA_WITH_LINEAR(PRE, false, false, false)                                            \
  SCHED_PD_MFMA_WITH_LINEAR(PRE, false, true, false)
#define SCHED_PD_MFMA_BF16_PAGEBLOCKS(PRE)                                                       \
  SCHED_PD_MFMA_WITH_LINEAR(PRE, false, false, true)                                             \
  SCHED_PD_MFMA_WITH_LINEAR(PRE, false, true, true)
#define SCHED_PD_MFMA_FP8(PRE)                                                                   \
  SCHED_PD_MFMA_WITH_LINEAR(PRE, true, false, false)                                             \
  SCHED_PD_MFMA_WITH_LINEAR(PRE, true, false, true)
#define SCHED_PD_MFMA_FP8_TOKMAJOR(PRE)                                                          \
  SCHED_PD_MFMA_WITH_LINEAR(PRE, true, true, false)                                              \
  SCHED_PD_MFMA_WITH_LINEAR(PRE, true, true, true)
#define SCHED_PD_MFMA_F16(PRE)                                                                   \
  SCHED_PD_MFMA_SOFTMAX(PRE, false, false, false, true)                                          \
  SCHED_PD_MFMA_SOFTMAX(PRE, false, true, false, true)
#define SCHED_PD_MFMA_F16_PAGEBLOCKS(PRE)                                                        \
  SCHED_PD_MFMA_SOFTMAX(PRE, false, false, true, true)                                           \
  SCHED_PD_MFMA_SOFTMAX(PRE, false, true, true, true)

// VALU kernels: kv element type x head dim, each for 1 / 4 / 16 q-heads per
// kv-head and the linear mode.
#define SCHED_PD_VALU_ONE(PRE, KVT, D)                                                           \
  PRE template __global__ void schedpd::decode_valu<KVT, D, 1, true>(schedpd::KParams);          \
  PRE template __global__ void schedpd::decode_valu<KVT, D, 1, false>(schedpd::KParams);         \
  PRE template __global__ void schedpd::decode_valu<KVT, D, 4, false>(schedpd::KParams);         \
  PRE template __global__ void schedpd::decode_valu<KVT, D, 16, false>(schedpd::KParams);
#define SCHED_PD_VALU_ALL(PRE)                                                                   \
  SCHED_PD_VALU_ONE(PRE, float, 32)                                                              \
  SCHED_PD_VALU_ONE(PRE, float, 64)                                                              \
  SCHED_PD_VALU_ONE(PRE, float, 128)                                                             \
  SCHED_PD_VALU_ONE(PRE, uint16_t, 64)                                                           \
  SCHED_PD_VALU_ONE(PRE, uint16_t, 128)                                                          \
  SCHED_PD_VALU_ONE(PRE, _Float16, 64)                                                           \
  SCHED_PD_VALU_ONE(PRE, _Float16, 128)                                                          \
  SCHED_PD_VALU_ONE(PRE, uint8_t, 64)                                                            \
  SCHED_PD_VALU_ONE(PRE, uint8_t, 128)

// One wave per work item (softmax, token-major rows), G = 1..3 q-heads per
// kv-head: one group per translation unit.
#define SCHED_PD_WAVE_ONE(PRE, KVT, D, G)                                                        \
  PRE template __global__ void schedpd::decode_wave<KVT, D, SCHED_PD_WAVE_NWT, G>(               \
      schedpd::KParams);
#define SCHED_PD_WAVE_G(PRE, G)                                                                  \
  SCHED_PD_WAVE_ONE(PRE, float, 32, G)                                                           \
  SCHED_PD_WAVE_ONE(PRE, float, 64, G)                                                           \
  SCHED_PD_WAVE_ONE(PRE, float, 128, G)                                                          \
  SCHED_PD_WAVE_ONE(PRE, uint16_t, 64, G)                                                        \
  SCHED_PD_WAVE_ONE(PRE, uint16_t, 128, G)                                                       \
  SCHED_PD_WAVE_ONE(PRE, _Float16, 64, G)                                                        \
  SCHED_PD_WAVE_ONE(PRE, _Float16, 128, G)
#define SCHED_PD_WAVE_ALL(PRE) SCHED_PD_WAVE_G(PRE, 1)
#define SCHED_PD_WAVE_GROUPS(PRE) SCHED_PD_WAVE_G(PRE, 2) SCHED_PD_WAVE_G(PRE, 3)

// Declarations for the launcher (paged_decode.hip).
#define SCHED_PD_DECLARE_ALL_KERNELS                                                             \
  SCHED_PD_MFMA_BF16_PAGE16(extern)                                                              \
  SCHED_PD_MFMA_BF16_PAGEBLOCKS(extern)                                                          \
  SCHED_PD_MFMA_FP8(extern)                                                                      \
  SCHED_PD_MFMA_FP8_TOKMAJOR(extern)                                                             \
  SCHED_PD_MFMA_F16(extern)                                                                      \
  SCHED_PD_MFMA_F16_PAGEBLOCKS(extern)                                                           \
  SCHED_PD_VALU_ALL(extern)                                                                      \
  SCHED_PD_WAVE_ALL(extern)                                                                      \
  SCHED_PD_WAVE_GROUPS(extern)
