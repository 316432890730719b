// The tree gather on gfx950 (verify_tree_gather, tree.metal:86-107): after
// tree acceptance, each lane's retained path rows move, in place, to rows
// 0 .. retained - 1 of one tensor family (16-bit elements with the layout of
// JustFitTreeGatherParams, TreeVerify.h:54-69). Path rows ascend and
// path[i] >= i, so copying rows in increasing i reads every source before
// it is overwritten; distinct columns touch distinct elements, so columns
// go to threads independently.
//
// A thread moves 8 consecutive columns with 16-byte accesses when the
// columns of a row are contiguous (inner_stride 1, inner a multiple of 8)
// and every stride and the base keep 16-byte alignment; otherwise one
// column. The grid is (column groups, layers, lanes); a block reads its
// lane's retained count and path once.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "jf_device.h"
#include "jf_kernels.h"

#include <type_traits>

namespace jf {

template <bool VEC8>
__global__ __launch_bounds__(256) void tree_gather_kernel(GatherLaunch g) {
  const uint32_t lane = blockIdx.z, layer = blockIdx.y;
  const uint32_t per = VEC8 ? 8u : 1u;
  const uint32_t column = (blockIdx.x * 256u + threadIdx.x) * per;
  if (column >= g.columns) return;
  const uint32_t rows = min(g.retained[lane], kGatherDepth);
  const uint32_t *path = g.path_rows + (uint64_t)lane * kGatherDepth;
  const uint64_t base = (uint64_t)layer * g.layer_stride + (uint64_t)lane * g.lane_stride +
                        (uint64_t)(column / g.inner) * g.outer_stride +
                        (uint64_t)(column % g.inner) * g.inner_stride;
  // Every source first, then every destination: a source row path[i] > i
  // is overwritten (if at all) only at step path[i] of the in-order copy,
  // after step i read it, so reading all sources up front reads the same
  // values, with all loads in flight at once. The path is the block's, so
  // which rows move is decided in scalar registers; a row that stays loads
  // the first moving row's source again (a cache hit, no HBM read) so that
  // every load is unconditional and the values stay in registers.
  uint32_t src[kGatherDepth], move = 0, first = kGatherDepth;
#pragma unroll
  for (uint32_t i = 0; i < kGatherDepth; ++i) {
    src[i] = i < rows ? path[i] : i;
    if (src[i] != i && src[i] < g.rows) {
      move |= 1u << i;
      first = min(first, i);
    }
  }
  if (!move) return;
  typedef uint32_t U32x4 __attribute__((ext_vector_type(4)));
  using Unit = std::conditional_t<VEC8, U32x4, uint16_t>;
  Unit v[kGatherDepth];
#pragma unroll
  for (uint32_t i = 0; i < kGatherDepth; ++i) {
    const uint32_t from = (move >> i) & 1u ? src[i] : src[first];
    v[i] = *(const Unit *)(g.data + base + (uint64_t)from * g.row_stride);
  }
#pragma unroll
  for (uint32_t i = 0; i < kGatherDepth; ++i)
    if ((move >> i) & 1u) *(Unit *)(g.data + base + (uint64_t)i * g.row_stride) = v[i];
}

int launch_tree_gather(const GatherLaunch &g, bool vec8, void *stream, void *start_event,
                       void *stop_event) {
  const uint32_t per = vec8 ? 8u : 1u;
  const uint32_t groups = (g.columns + per - 1) / per;
  const dim3 grid((groups + 255) / 256, g.layers, g.lanes), block(256);
  const hipStream_t st = (hipStream_t)stream;
  if (vec8)
    hipExtLaunchKernelGGL(tree_gather_kernel<true>, grid, block, 0, st, (hipEvent_t)start_event,
                          (hipEvent_t)stop_event, 0, g);
  else
    hipExtLaunchKernelGGL(tree_gather_kernel<false>, grid, block, 0, st, (hipEvent_t)start_event,
                          (hipEvent_t)stop_event, 0, g);
  return (int)hipGetLastError();
}

}  // namespace jf
