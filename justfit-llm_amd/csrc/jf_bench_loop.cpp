// Timing helper for bench.py (not part of libjf_sampler.so): runs prepared
// jf_sample calls back to back from C++, so the per-step host cost of a
// native caller is measured apart from the Python loop's. Each step issues
// args[i % n] on `stream`, optionally followed by one token per row counted
// into tables[i % n] (the engine's commit). Returns the GPU time per step
// (HIP events around the whole loop) and the host time per step (wall
// clock of the issuing loop alone).
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdint>

#include "jf_sampler.h"

extern "C" int jf_bench_sample_loop(jf_sampler *sampler, const jf_sample_args *args,
                                    uint32_t n, uint32_t steps, jf_penalty_table *const *tables,
                                    const uint32_t *count_rows, const uint32_t *count_tokens,
                                    uint32_t rows, void *stream, double *gpu_us_per_step,
                                    double *host_us_per_step) {
  if (!sampler || !args || !n || !steps || !gpu_us_per_step || !host_us_per_step) return -1;
  hipStream_t st = (hipStream_t)stream;
  hipEvent_t start, stop;
  if (hipEventCreate(&start) != hipSuccess) return -2;
  if (hipEventCreate(&stop) != hipSuccess) {
    (void)hipEventDestroy(start);
    return -2;
  }
  int rc = hipStreamSynchronize(st) == hipSuccess ? 0 : -2;
  const auto t0 = std::chrono::steady_clock::now();
  if (!rc && hipEventRecord(start, st) != hipSuccess) rc = -2;
  for (uint32_t i = 0; i < steps && !rc; ++i) {
    rc = jf_sample(sampler, &args[i % n], stream);
    if (!rc && tables)
      rc = jf_penalty_table_count_rows(tables[i % n], count_rows,
                                       count_tokens + (uint64_t)i * rows, rows, stream);
  }
  const auto t1 = std::chrono::steady_clock::now();
  if (!rc && hipEventRecord(stop, st) != hipSuccess) rc = -2;
  if (!rc && hipEventSynchronize(stop) != hipSuccess) rc = -2;
  float ms = 0.0f;
  if (!rc && hipEventElapsedTime(&ms, start, stop) != hipSuccess) rc = -2;
  if (!rc) {
    *gpu_us_per_step = 1000.0 * ms / steps;
    *host_us_per_step = std::chrono::duration<double, std::micro>(t1 - t0).count() / steps;
  }
  (void)hipEventDestroy(start);
  (void)hipEventDestroy(stop);
  return rc;
}
