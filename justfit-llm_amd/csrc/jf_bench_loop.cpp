// Timing helper for bench.py (not part of libjf_sampler.so): runs prepared
// calls back to back from C++, so the per-step host cost of a native caller
// is measured apart from the Python loop's. jf_bench_sample_loop: each step
// issues args[i % n] on `stream`, then optionally the step's acceptance over
// its tokens (chain: jf_accept_chain; tree: jf_accept_tree, the prepared
// records, or with tree_combined jf_sample_accept_tree for both), then
// optionally one token per row counted into tables[i % n] (the engine's
// commit). jf_bench_draft_loop and jf_bench_gather_loop issue
// jf_draft_select and jf_tree_gather the same way. Each returns the GPU time
// per step (HIP events around the whole loop), the host time per step (wall
// clock of the issuing loop alone) and, with batch_us set, the mean step
// time of each run of `batch` steps between events.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdint>
#include <vector>

#include "jf_sampler.h"

namespace {

// The loop's events and clocks around `issue(i)` for i < steps.
template <class Issue>
int timed_loop(uint32_t steps, void *stream, double *gpu_us_per_step, double *host_us_per_step,
               uint32_t batch, float *batch_us, Issue issue) {
  if (!steps || !gpu_us_per_step || !host_us_per_step) return -1;
  if (batch_us && (!batch || steps % batch)) return -1;
  hipStream_t st = (hipStream_t)stream;
  // Events at the loop's ends, and after every `batch` steps when batch
  // times are asked for (an event per step would add its own packets to
  // every step).
  const uint32_t nb = batch_us ? steps / batch : 1;
  const uint32_t ne = nb + 1;
  std::vector<hipEvent_t> ev(ne, nullptr);
  int rc = 0;
  for (uint32_t i = 0; i < ne && !rc; ++i)
    if (hipEventCreate(&ev[i]) != hipSuccess) rc = -2;
  if (!rc && hipStreamSynchronize(st) != hipSuccess) rc = -2;
  const auto t0 = std::chrono::steady_clock::now();
  if (!rc && hipEventRecord(ev[0], st) != hipSuccess) rc = -2;
  for (uint32_t i = 0; i < steps && !rc; ++i) {
    rc = issue(i);
    const uint32_t per = batch_us ? batch : steps;
    if (!rc && (i + 1) % per == 0 && hipEventRecord(ev[(i + 1) / per], st) != hipSuccess)
      rc = -2;
  }
  const auto t1 = std::chrono::steady_clock::now();
  if (!rc && hipEventSynchronize(ev[ne - 1]) != hipSuccess) rc = -2;
  float ms = 0.0f;
  if (!rc && hipEventElapsedTime(&ms, ev[0], ev[ne - 1]) != hipSuccess) rc = -2;
  for (uint32_t i = 0; batch_us && i < nb && !rc; ++i) {
    float m = 0.0f;
    if (hipEventElapsedTime(&m, ev[i], ev[i + 1]) != hipSuccess) rc = -2;
    batch_us[i] = 1000.0f * m / batch;
  }
  if (!rc) {
    *gpu_us_per_step = 1000.0 * ms / steps;
    *host_us_per_step = std::chrono::duration<double, std::micro>(t1 - t0).count() / steps;
  }
  for (hipEvent_t e : ev)
    if (e) (void)hipEventDestroy(e);
  return rc;
}

}  // namespace

extern "C" int jf_bench_sample_loop(jf_sampler *sampler, const jf_sample_args *args,
                                    uint32_t n, uint32_t steps, jf_penalty_table *const *tables,
                                    const uint32_t *count_rows, const uint32_t *count_tokens,
                                    uint32_t rows, void *stream, double *gpu_us_per_step,
                                    double *host_us_per_step, uint32_t batch, float *batch_us,
                                    const jf_accept_chain_args *chain,
                                    const jf_accept_tree_args *tree, int tree_combined) {
  if (!sampler || !args || !n) return -1;
  return timed_loop(steps, stream, gpu_us_per_step, host_us_per_step, batch, batch_us,
                    [&](uint32_t i) {
                      int rc;
                      if (tree && tree_combined) {
                        rc = jf_sample_accept_tree(sampler, &args[i % n], tree, stream);
                      } else {
                        rc = jf_sample(sampler, &args[i % n], stream);
                        if (!rc && tree) rc = jf_accept_tree(sampler, tree, stream);
                      }
                      if (!rc && chain) rc = jf_accept_chain(sampler, chain, stream);
                      if (!rc && tables)
                        rc = jf_penalty_table_count_rows(tables[i % n], count_rows,
                                                         count_tokens + (uint64_t)i * rows, rows,
                                                         stream);
                      return rc;
                    });
}

extern "C" int jf_bench_draft_loop(jf_draft_selector *selector, const jf_draft_select_args *args,
                                   uint32_t n, uint32_t steps, void *stream,
                                   double *gpu_us_per_step, double *host_us_per_step,
                                   uint32_t batch, float *batch_us) {
  if (!selector || !args || !n) return -1;
  return timed_loop(steps, stream, gpu_us_per_step, host_us_per_step, batch, batch_us,
                    [&](uint32_t i) { return jf_draft_select(selector, &args[i % n], stream); });
}

extern "C" int jf_bench_gather_loop(const jf_tree_gather_args *args, uint32_t n, uint32_t steps,
                                    void *stream, double *gpu_us_per_step,
                                    double *host_us_per_step, uint32_t batch, float *batch_us) {
  if (!args || !n) return -1;
  return timed_loop(steps, stream, gpu_us_per_step, host_us_per_step, batch, batch_us,
                    [&](uint32_t i) { return jf_tree_gather(&args[i % n], stream); });
}
