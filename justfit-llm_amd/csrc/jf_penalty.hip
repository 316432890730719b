// Counted tokens applied to the device penalty table in place: the host copy
// (jf_host.cpp) decides each token's entry index, insertion and slot, and
// one block per table row applies that row's updates in call order. This is
// countPenaltyTokens (Sampling.cpp:75-80) on the table's sparse layout,
// without re-uploading the row.
#include <hip/hip_runtime.h>

#include "jf_host.h"
#include "jf_kernels.h"

namespace jf {

namespace {

constexpr uint32_t kHeld = 16;  // entries per thread moved in one pass
constexpr uint32_t kPass = kHeld * kThreads;

// Inserts `entry` at v[0] after moving v[0, n) up one place (to v[1, n +
// 1)), and, with u set, `slot` at u[0] after moving u[0, m) up one place
// (m <= 2 * kThreads: a chunk's slots). Each pass holds up to kPass entries
// of v in registers (the first pass also all of u): its loads go out
// together, the block waits once, then stores. Passes run top first; a pass
// writes [lo + 1, hi + 1) and the next reads below lo, so passes need no
// barrier between them. The new values go out with the last stores.
__device__ void insert_at(PenaltyEntry *v, uint32_t n, PenaltyEntry entry, uint32_t *u,
                          uint32_t m, uint32_t slot) {
  const uint32_t tid = threadIdx.x;
  uint32_t hi = n;
  bool first = true;
  do {
    const uint32_t lo = hi > kPass ? hi - kPass : 0u;
    PenaltyEntry x[kHeld];
#pragma unroll
    for (uint32_t k = 0; k < kHeld; ++k) {
      const uint32_t p = lo + tid + k * kThreads;
      if (p < hi) x[k] = v[p];
    }
    uint32_t y0 = 0, y1 = 0;
    if (first && u) {
      if (tid < m) y0 = u[tid];
      if (tid + kThreads < m) y1 = u[tid + kThreads];
    }
    __syncthreads();
#pragma unroll
    for (uint32_t k = 0; k < kHeld; ++k) {
      const uint32_t p = lo + tid + k * kThreads;
      if (p < hi) v[p + 1] = x[k];
    }
    if (first && u) {
      if (tid < m) u[tid + 1] = y0;
      if (tid + kThreads < m) u[tid + kThreads + 1] = y1;
      if (tid == 0) u[0] = slot;
    }
    if (lo == 0 && tid == 0) v[0] = entry;
    first = false;
    hi = lo;
  } while (hi > 0);
}

// One row's updates, in call order (block g: ops [start, end) of row `row`).
__device__ __forceinline__ void apply_ops(const PenaltyTableView &t, uint32_t row,
                                          const PackedPenaltyOp *ops, uint32_t k0,
                                          uint32_t k1) {
  const uint32_t tid = threadIdx.x;
  PenaltyEntry *e = t.entries + (uint64_t)row * t.max_entries;
  uint32_t *off = t.offsets + (uint64_t)row * (t.buckets + 1);
  for (uint32_t k = k0; k < k1; ++k) {
    if (k != k0) __syncthreads();  // this update reads the previous one's writes
    const PackedPenaltyOp op = ops[k];
    const uint32_t index = op.index & 0x7fffffffu;
    const bool insert = (op.index >> 31) != 0;
    const uint32_t slot = op.slot & 0xffffu, used = op.slot >> 16;
    uint32_t *sl = nullptr;
    if (slot != 0xffffu)
      sl = t.slots + ((uint64_t)row * t.chunks + op.token / kPenaltyChunk) * t.slot_count +
           slot;
    if (insert) {
      for (uint32_t bk = op.token / kPenaltyBucket + 1 + tid; bk <= t.buckets; bk += kThreads)
        off[bk] += 1u;
      // The chunk's slots [slot, used) move with the entries (used < 512).
      insert_at(e + index, op.entries - index, PenaltyEntry{op.token, op.word}, sl,
                sl ? used - slot : 0u, op.slot_value);
    } else if (tid == 0) {
      e[index].word = op.word;
      if (sl) *sl = op.slot_value;
    }
  }
}

__global__ __launch_bounds__(kThreads) void penalty_count_kernel(PenaltyTableView t,
                                                                 PenaltyOpBatch b) {
  apply_ops(t, b.group_row[blockIdx.x], b.op, b.group_start[blockIdx.x],
            b.group_start[blockIdx.x + 1]);
}

// The batch in host-mapped memory: each block reads its group's bounds, then
// each op at its turn, over the bus.
__global__ __launch_bounds__(kThreads) void penalty_count_mapped_kernel(
    PenaltyTableView t, const PackedPenaltyOp *ops, const uint32_t *group_row,
    const uint32_t *group_start) {
  apply_ops(t, group_row[blockIdx.x], ops, group_start[blockIdx.x],
            group_start[blockIdx.x + 1]);
}

}  // namespace

int launch_penalty_count(const PenaltyTableView &t, const PenaltyOpBatch &b, uint32_t groups,
                         void *stream) {
  hipLaunchKernelGGL(penalty_count_kernel, dim3(groups), dim3(kThreads), 0,
                     (hipStream_t)stream, t, b);
  return (int)hipGetLastError();
}

int launch_penalty_count_mapped(const PenaltyTableView &t, const PackedPenaltyOp *ops,
                                const uint32_t *group_row, const uint32_t *group_start,
                                uint32_t groups, void *stream) {
  hipLaunchKernelGGL(penalty_count_mapped_kernel, dim3(groups), dim3(kThreads), 0,
                     (hipStream_t)stream, t, ops, group_row, group_start);
  return (int)hipGetLastError();
}

}  // namespace jf
