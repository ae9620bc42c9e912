// paged_decode_host.cpp -- a host program of the kind that included the
// reference's runtime/sched_rt.h (test/paged_decode.cu:255-380): it arms the
// levers through the sched_rt_* C ABI, launches the decode through
// sched_paged_decode with the levers read from the __sched_* slots
// (SCHED_PD_FLAG_RT_TABLES), and reads the timer rows back. It links
// libschedpd.so and the HIP runtime only; no kernel is compiled here.
//
// usage: paged_decode_host <dir>
//   <dir>/meta.txt  R Hq Hkv D page bt_stride pages workers
//   <dir>/{q,k,v}.bin  bf16 Q [R][Hq][D], K [pages][Hkv][page][D],
//                      V [pages][Hkv][D][page] (d-major)
//   <dir>/bt.bin, ctx.bin  int32 [R][bt_stride], [R]
//   <dir>/tau.bin  uint16 [R*Hkv] per-task budgets (tokens, 0 = none)
// writes <dir>/out_<mode>.bin (fp32 [R][Hq][D]) for the modes stock,
// neutral, reversed, timed, queue and shed, and timer.bin (u64 [R*Hkv]).
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "sched_pd.h"

namespace {

std::string g_dir;

bool read_file(const char *name, std::vector<char> &buf, size_t want) {
  const std::string path = g_dir + "/" + name;
  FILE *f = std::fopen(path.c_str(), "rb");
  if (!f) {
    std::fprintf(stderr, "cannot open %s\n", path.c_str());
    return false;
  }
  buf.resize(want);
  const size_t got = std::fread(buf.data(), 1, want, f);
  std::fclose(f);
  if (got != want) {
    std::fprintf(stderr, "%s: %zu bytes, expected %zu\n", path.c_str(), got, want);
    return false;
  }
  return true;
}

bool write_file(const std::string &name, const void *p, size_t bytes) {
  const std::string path = g_dir + "/" + name;
  FILE *f = std::fopen(path.c_str(), "wb");
  if (!f)
    return false;
  const size_t put = std::fwrite(p, 1, bytes, f);
  std::fclose(f);
  return put == bytes;
}

bool hip_ok(hipError_t e, const char *what) {
  if (e != hipSuccess) {
    std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
    return false;
  }
  return true;
}

void *to_device(const std::vector<char> &h) {
  void *d = nullptr;
  if (!hip_ok(hipMalloc(&d, h.size()), "hipMalloc") ||
      !hip_ok(hipMemcpy(d, h.data(), h.size(), hipMemcpyHostToDevice), "hipMemcpy"))
    return nullptr;
  return d;
}

} // namespace

int main(int argc, char **argv) {
  if (argc != 2) {
    std::fprintf(stderr, "usage: %s <dir>\n", argv[0]);
    return 2;
  }
  g_dir = argv[1];
  unsigned R, Hq, Hkv, D, ps, bts, pages, W;
  {
    const std::string meta = g_dir + "/meta.txt";
    FILE *f = std::fopen(meta.c_str(), "r");
    if (!f || std::fscanf(f, "%u %u %u %u %u %u %u %u", &R, &Hq, &Hkv, &D, &ps, &bts, &pages,
                          &W) != 8) {
      std::fprintf(stderr, "cannot read %s\n", meta.c_str());
      return 2;
    }
    std::fclose(f);
  }
  const unsigned ntask = R * Hkv;
  const size_t pool = (size_t)pages * Hkv * ps * D * 2;
  std::vector<char> hq, hk, hv, hbt, hctx, htau;
  if (!read_file("q.bin", hq, (size_t)R * Hq * D * 2) || !read_file("k.bin", hk, pool) ||
      !read_file("v.bin", hv, pool) || !read_file("bt.bin", hbt, (size_t)R * bts * 4) ||
      !read_file("ctx.bin", hctx, (size_t)R * 4) || !read_file("tau.bin", htau, ntask * 2))
    return 2;
  void *dq = to_device(hq), *dk = to_device(hk), *dv = to_device(hv);
  void *dbt = to_device(hbt), *dctx = to_device(hctx);
  void *dout = nullptr;
  const size_t out_bytes = (size_t)R * Hq * D * 4;
  if (!dq || !dk || !dv || !dbt || !dctx || !hip_ok(hipMalloc(&dout, out_bytes), "hipMalloc"))
    return 2;

  SchedDecodeArgs a;
  sched_pd_default_args(&a);
  a.mode = SCHED_PD_SOFTMAX;
  a.kv_dtype = SCHED_PD_BF16;
  a.q_dtype = SCHED_PD_BF16;
  a.o_dtype = SCHED_PD_F32;
  a.num_requests = R;
  a.num_q_heads = Hq;
  a.num_kv_heads = Hkv;
  a.head_dim = D;
  a.page_size = ps;
  a.q = dq;
  a.out = dout;
  a.k_pool = dk;
  a.v_pool = dv;
  a.k_page_stride = (int64_t)Hkv * ps * D;
  a.k_head_stride = (int64_t)ps * D;
  a.k_tok_stride = D;
  a.v_page_stride = (int64_t)Hkv * D * ps;
  a.v_head_stride = (int64_t)D * ps;
  a.v_dim_stride = ps;
  a.v_tok_stride = 1;
  a.block_table = static_cast<const int32_t *>(dbt);
  a.bt_stride = bts;
  a.ctx_lens = static_cast<const int32_t *>(dctx);

  std::vector<float> out(out_bytes / 4);
  auto run = [&](const char *mode, uint32_t workers) {
    a.flags = SCHED_PD_FLAG_RT_TABLES;
    a.workers = workers;
    if (!hip_ok(hipMemset(dout, 0xff, out_bytes), "hipMemset"))
      return false;
    const int rc = sched_paged_decode(&a, nullptr);
    if (rc != 0) {
      std::fprintf(stderr, "%s: sched_paged_decode: %s\n", mode, sched_pd_last_error());
      return false;
    }
    if (!hip_ok(hipDeviceSynchronize(), mode) ||
        !hip_ok(hipMemcpy(out.data(), dout, out_bytes, hipMemcpyDeviceToHost), "hipMemcpy"))
      return false;
    std::printf("mode %s done\n", mode);
    std::fflush(stdout);
    return write_file(std::string("out_") + mode + ".bin", out.data(), out_bytes);
  };

  // A: slots empty (nothing armed): the stock decode
  if (!sched_rt_disarm() || !run("stock", 0))
    return 1;
  // B: armed, neutral (identity order, neutral control block)
  if (!sched_rt_init() || !sched_rt_push_ctrl() || !run("neutral", 0))
    return 1;
  // C: pi reversed over every task
  std::vector<int32_t> order(ntask);
  for (unsigned i = 0; i < ntask; ++i)
    order[i] = (int32_t)(ntask - 1 - i);
  sched_rt_set_order_size(ntask);
  if (!sched_rt_set_order(order.data(), ntask) || !sched_rt_push_ctrl() || !run("reversed", 0))
    return 1;
  // D: the timer, rows read back
  sched_rt_timer_clear();
  sched_rt_set_timer_enabled(true);
  if (!sched_rt_push_ctrl() || !run("timed", 0))
    return 1;
  std::vector<unsigned long long> rows(ntask);
  if (!sched_rt_timer_read(rows.data(), ntask) ||
      !write_file("timer.bin", rows.data(), rows.size() * 8))
    return 1;
  // E: the ticket work queue, W workers
  sched_rt_set_num_tasks(ntask);
  if (!sched_rt_push_ctrl() || !sched_rt_queue_reset(W) || !run("queue", W))
    return 1;
  // F: per-task shed budgets, identity order, static grid
  for (unsigned i = 0; i < ntask; ++i)
    order[i] = (int32_t)i;
  sched_rt_set_num_tasks(0);
  const uint16_t *tau = reinterpret_cast<const uint16_t *>(htau.data());
  for (unsigned i = 0; i < ntask; ++i)
    sched_rt_set_tau(i, tau[i]);
  if (!sched_rt_set_order(order.data(), ntask) || !sched_rt_push_ctrl() || !run("shed", 0))
    return 1;
  sched_rt_disarm();
  bool freed = true;
  for (void *p : {dq, dk, dv, dbt, dctx, dout})
    freed = hip_ok(hipFree(p), "hipFree") && freed;
  if (!freed)
    return 1;
  std::printf("ok\n");
  return 0;
}
