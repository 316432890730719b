// jf_sample_static: jf_sample for callers that cannot allocate device memory
// (code under HIP graph capture, serving loops and harnesses that forbid
// hipMalloc). Its scratch is one file-scope device array that every GPU the
// library runs on holds until the process ends; the call allocates nothing.
//
// The array's name is a host-side stand-in, not a device address: host code
// uses only the address hipGetSymbolAddress returns for the current device,
// taken once per device at the first call.
#include "jf_sampler.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "jf_kernels.h"


namespace {

constexpr uint32_t kStaticRows = 64;
constexpr uint32_t kStaticChunks = 32;  // vocabularies up to 262,144 tokens
constexpr uint32_t kStaticVocabulary = kStaticChunks * jf::kChunkF32;
constexpr uint64_t kBlocks = (uint64_t)kStaticRows * kStaticChunks;

constexpr uint64_t align256(uint64_t x) { return (x + 255u) & ~uint64_t{255}; }
// Byte offsets of the sub-buffers inside the array, each 256-byte aligned.
constexpr uint64_t kParamsOff = 0;
constexpr uint64_t kHeadersOff = align256(kParamsOff + kStaticRows * sizeof(jf::RowParams));
constexpr uint64_t kCandsOff = align256(kHeadersOff + kBlocks * sizeof(jf::BlockHeader));
constexpr uint64_t kCountersOff =
    align256(kCandsOff + kBlocks * jf::kBlockCandidates * sizeof(uint64_t));
constexpr uint64_t kBestsOff = align256(kCountersOff + kStaticRows * sizeof(uint32_t));
constexpr uint64_t kStatesOff = align256(kBestsOff + kBlocks * sizeof(uint64_t));
constexpr uint64_t kPartialsOff = align256(kStatesOff + kStaticRows * sizeof(jf::RowState));
constexpr uint64_t kScratchBytes = align256(kPartialsOff + kBlocks * sizeof(jf::StagePartial));
static_assert(kScratchBytes < (24u << 20), "the static scratch stays under 24 MiB");

// Row parameters travel to the device as kernel arguments, 32 rows a launch.
constexpr uint32_t kParamsPerLaunch = 32;
struct ParamsBatch {
  jf::RowParams p[kParamsPerLaunch];
  uint32_t first;  // first row of this batch
  uint32_t n;      // rows in this batch
};

}  // namespace

// The scratch of every jf_sample_static call on this GPU.
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

// Stores one batch of row parameters, and clears those rows' arrival
// counters and stage fields: what the selection kernels need zero on entry
// (a fill kernel, not a memset, so that a captured graph replays it).
__global__ __launch_bounds__(kParamsPerLaunch * 16) void store_params_kernel(
    uint8_t *base, ParamsBatch b) {
  const uint32_t t = threadIdx.x;
  uint32_t *params = (uint32_t *)(base + kParamsOff) + (uint64_t)b.first * 16u;
  if (t < b.n * 16u) params[t] = ((const uint32_t *)b.p)[t];
  if (t < b.n) {
    ((uint32_t *)(base + kCountersOff))[b.first + t] = 0u;
    ((jf::RowState *)(base + kStatesOff))[b.first + t].stage = jf::kStageDone;
  }
}

int static_upload(void *ctx, const jf::RowParams *params, uint32_t rows,
                  jf::RowParams *, void *stream) {
  uint8_t *base = (uint8_t *)ctx;
  for (uint32_t first = 0; first < rows; first += kParamsPerLaunch) {
    ParamsBatch b;
    b.first = first;
    b.n = rows - first < kParamsPerLaunch ? rows - first : kParamsPerLaunch;
    for (uint32_t i = 0; i < b.n; ++i) b.p[i] = params[first + i];
    hipLaunchKernelGGL(store_params_kernel, dim3(1), dim3(kParamsPerLaunch * 16), 0,
                       (hipStream_t)stream, base, b);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return jf::set_error(JF_ERR_DEVICE, hipGetErrorString(e));
  }
  return JF_OK;
}

constexpr int kMaxDevices = 64;
std::mutex g_lock;
uint8_t *g_scratch[kMaxDevices];  // the array's address on each device

// The array's device address on the current device, looked up once per
// device with that device current.
int scratch_address(uint8_t **out) {
  int device = -1;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return jf::set_error(JF_ERR_DEVICE, hipGetErrorString(e));
  if (device < 0 || device >= kMaxDevices)
    return jf::set_error(JF_ERR_DEVICE, "device ordinal beyond the static scratch table");
  std::lock_guard<std::mutex> guard(g_lock);
  if (!g_scratch[device]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return jf::set_error(JF_ERR_DEVICE, e != hipSuccess ? hipGetErrorString(e)
                                                          : "static scratch has no address");
    g_scratch[device] = (uint8_t *)p;
  }
  *out = g_scratch[device];
  return JF_OK;
}

}  // namespace

extern "C" int jf_sample_static(uint32_t vocabulary, const jf_sample_args *args,
                                void *stream) {
  if (!args) return jf::set_error(JF_ERR_INVALID_ARGUMENT, "null arguments");
  if (!vocabulary) return jf::set_error(JF_ERR_INVALID_ARGUMENT, "invalid sampling geometry");
  if (vocabulary > kStaticVocabulary)
    return jf::set_error(JF_ERR_INVALID_ARGUMENT,
                         "vocabulary exceeds the static sampling scratch (262144 tokens)");
  if (!args->rows || args->rows > kStaticRows)
    return jf::set_error(JF_ERR_INVALID_ARGUMENT,
                         "rows exceed the static sampling scratch (1..64 rows)");
  uint8_t *base = nullptr;
  const int rc = scratch_address(&base);
  if (rc != JF_OK) return rc;
  // Each call's tag of its packed greedy bests (a captured graph replays the
  // one it was captured with; the words are cleared as they are taken).
  static std::atomic<uint32_t> epochs{0};
  const jf::SampleScratch sc{(jf::RowParams *)(base + kParamsOff),
                             (jf::BlockHeader *)(base + kHeadersOff),
                             (uint64_t *)(base + kCandsOff),
                             (uint32_t *)(base + kCountersOff),
                             (uint64_t *)(base + kBestsOff),
                             (jf::RowState *)(base + kStatesOff),
                             (jf::StagePartial *)(base + kPartialsOff),
                             kStaticRows,
                             kStaticChunks,
                             nullptr,
                             epochs.fetch_add(1, std::memory_order_relaxed) % 4095u + 1u,
                             1u << 20,
                             nullptr};
  jf::RowParams params[kStaticRows];
  return jf::sample_core(vocabulary, sc, args, params, static_upload, base, stream);
}
