// The draft selector on gfx950: the DFlash draft's proposal policy
// (draft_select_top16_sharded, draft_select_edges, draft_select_dflash in
// sampling.metal:995-1359, dispatched by DraftSelector.cpp:38-92).
//
// A lane has 8 query rows of fp32 draft logits; rows 1..7 are its proposal
// positions. Two launches:
//   draft_top16_kernel  one block per (8192-token chunk, proposal row): the
//                       chunk's exact top 16 in (value desc, id asc) order,
//                       written as the chunk's partial list.
//   draft_edges_kernel  one block per (position, lane): merges the partial
//                       lists of its row (and of the previous row) into the
//                       candidates and unary scores, then the 16 x 16 table
//                       of edge scores from the previous position's
//                       candidates (the anchor at position 0) to this
//                       position's, and the walk's step at this position
//                       after each predecessor (greedily or drawing at the
//                       lane's temperature); the lane's last block chains
//                       the 7 positions' steps.
// Edge scores are fp32 sums over the selector rank in ascending dimension
// order (each product of bf16 operands is exact in fp32); the reference sums
// the same terms in another order.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "jf_device.h"
#include "jf_kernels.h"

namespace jf {

namespace {

constexpr uint32_t kDraftChunk = 8192;   // fp32 tokens per block
constexpr int kDraftLoads = 8;           // 16-byte loads per thread
constexpr int kDraftTokens = 32;         // tokens per thread
constexpr uint32_t kDraftK = 16;
constexpr uint32_t kDraftMaxChunks = 64;    // vocabulary <= 524288
constexpr uint32_t kRank = 256;
// LDS row pitch of the edge operands: 16-byte rows for four-float reads,
// and 4 mod 32 words, so the 16 successor rows start on distinct banks in
// pairs (a 2-way conflict at most).
constexpr uint32_t kPad = kRank + 4;

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16f(uint32_t b) { return u2f(b << 16); }
__device__ __forceinline__ float readlane_f32(float v, int l) {
  return u2f(readlane_u32(f2u(v), l));
}

// (key << 32 | ~id): larger means earlier in (value desc, id asc); ids are
// unique within a row, so the order is total. 0 is the empty slot
// (-inf, kNoToken), after every real entry.
__device__ __forceinline__ uint64_t draft_comp(float x, uint32_t id) {
  return ((uint64_t)logit_key(x) << 32) | (uint32_t)~id;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  auto step = [&](uint64_t o) { v = o > v ? o : v; };
  step(xor_u64<1>(v));
  step(xor_u64<2>(v));
  step(xor_u64<4>(v));
  step(xor_u64<8>(v));
  step(xor_u64<16>(v));
  step(xor_u64<32>(v));
  return v;
}
// A reduction of a 32-bit value over the wave (WIDE) or over lanes 0..31
// (when lanes 32..63 hold the operation's identity), in every lane: DPP
// quad permutes and row rotations by 4 and 8 within each 16-lane row, then
// across rows by gfx950's lane swaps, VALU work with no LDS crossbar:
// v_permlane16_swap leaves each lane one value of each row of its row pair
// (rows 0,1 and 2,3), v_permlane32_swap one of each half.
template <bool WIDE, class Op>
__device__ __forceinline__ uint32_t lanes_reduce_u32(uint32_t v, Op op) {
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xF, 0xF, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false));
  const auto rows = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = op((uint32_t)rows[0], (uint32_t)rows[1]);
  if constexpr (WIDE) {
    const auto halves = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    v = op((uint32_t)halves[0], (uint32_t)halves[1]);
  }
  return v;
}
template <bool WIDE>
__device__ __forceinline__ uint32_t lanes_max_u32(uint32_t v) {
  return lanes_reduce_u32<WIDE>(v, [](uint32_t a, uint32_t b) { return max(a, b); });
}
// The largest value of each 16-lane row, in every lane of the row (DPP
// only): the wave's largest when every row holds the same 16 values.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return u2f((uint32_t)__builtin_amdgcn_update_dpp(0, (int)f2u(x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_max_f32(float v) {
  v = __builtin_fmaxf(v, dpp_f32<0xB1>(v));   // quad xor 1
  v = __builtin_fmaxf(v, dpp_f32<0x4E>(v));   // quad xor 2
  v = __builtin_fmaxf(v, dpp_f32<0x124>(v));  // row rotate by 4
  v = __builtin_fmaxf(v, dpp_f32<0x128>(v));  // row rotate by 8
  return v;
}

// Lane k of each 16-lane row, in every lane of the row.
__device__ __forceinline__ float row_lane_f32(float v, int k) {
  const float r0 = readlane_f32(v, k), r1 = readlane_f32(v, 16 + k),
              r2 = readlane_f32(v, 32 + k), r3 = readlane_f32(v, 48 + k);
  const uint32_t r = lane_id() >> 4;
  return r == 0 ? r0 : r == 1 ? r1 : r == 2 ? r2 : r3;
}
// Lane j of each 16-lane row ends holding ((0 + w_0) + w_1) + ... + w_j: a
// sum in lane order with that order's rounding, each step taking the sum
// so far from the lane before by a DPP row shift.
__device__ __forceinline__ float row_ordered_sums(float w, uint32_t j) {
  float c = 0.0f + w;
#pragma unroll
  for (uint32_t k = 1; k < kDraftK; ++k) {
    const float before = dpp_f32<0x111>(c);  // row_shr:1
    c = j == k ? before + w : c;
  }
  return c;
}

struct __align__(16) DraftTopLds {
  uint32_t wtop[kWaves];             // each wave's 4th largest lane maximum
  uint64_t comp[kThreads];           // the chunk's entries at or above the bound
  uint32_t vbits[kThreads];
  uint64_t top[kDraftK];
  uint32_t topv[kDraftK];
  uint64_t wbest[kWaves];
  uint32_t wcount[kWaves];
  uint32_t taken;                    // slots taken by the waves' entries
};

}  // namespace

// One chunk of one proposal row: its top 16 in rank order (empty slots 0,
// value -inf) into the row's partials. Each thread holds 32 tokens. The 16th
// largest lane maximum of the block bounds the chunk's top 16 (16 lanes hold
// a token at least that large); each wave sorts its lane maxima, and every
// wave sorts the 64 wave leaders to find it. The tokens at or above the bound
// are compacted by a prefix sum and ranked by counting. A chunk with more
// than 256 of them (ties) takes its top 16 by 16 rounds of block maxima.
template <bool ALIGNED>
__global__ __launch_bounds__(kThreads) void draft_top16_kernel(DraftLaunch d) {
  __shared__ DraftTopLds s;
  const uint32_t chunk = blockIdx.x, row = blockIdx.y;
  const uint32_t lane_index = row / kDraftPositions, p = row % kDraftPositions;
  const uint32_t V = d.vocabulary, S = d.chunks;
  const float *rowp = d.logits + ((uint64_t)lane_index * kDraftQueryRows + p + 1) * d.stride;
  const uint32_t tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const uint32_t base = chunk * kDraftChunk, lane_base = base + tid * 4;
  auto token_of = [&](int i) -> uint32_t { return lane_base + (i >> 2) * 1024 + (i & 3); };

  float x[kDraftTokens];
  if (ALIGNED && base + kDraftChunk <= V) {
#pragma unroll
    for (int j = 0; j < kDraftLoads; ++j) {
      const f32x4 v = *(const f32x4 *)(rowp + lane_base + j * 1024);
      x[j * 4 + 0] = v.x;
      x[j * 4 + 1] = v.y;
      x[j * 4 + 2] = v.z;
      x[j * 4 + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kDraftTokens; ++i) {
      const uint32_t t = token_of(i);
      x[i] = t < V ? rowp[t] : __builtin_nanf("");
    }
  }
  if (tid < kDraftK) {
    s.top[tid] = 0;
    s.topv[tid] = f2u(-__builtin_inff());
  }
  // The first 64 slots read 0 (below every entry) until an entry lands.
  if (tid < 64) s.comp[tid] = 0ull;
  if (tid == 0) s.taken = 0;
  // The lane's largest key among its non-NaN tokens (0: none): fmax skips
  // NaN operands, so the float maximum is NaN only when every token is, and
  // the key order is the float order (the two zeros share a key).
  float mx = x[0];
#pragma unroll
  for (int i = 1; i < kDraftTokens; ++i) mx = __builtin_fmaxf(mx, x[i]);
  const uint32_t mkey = mx == mx ? logit_key(mx) : 0u;
  // The bound: the smallest of the waves' 4th largest lane maxima. Each
  // wave has four lanes, each with a token at or above its own, so the
  // chunk has 16 tokens at or above the bound and its top 16 lie there.
  uint32_t rest = mkey, t4 = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    t4 = __builtin_amdgcn_readfirstlane(lanes_max_u32<true>(rest));
    const uint64_t at = ballot(rest == t4);
    if (lane == (uint32_t)__builtin_ctzll(at)) rest = 0;
  }
  if (lane == 0) s.wtop[w] = t4;
  __syncthreads();
  uint32_t bound = s.wtop[0];
#pragma unroll
  for (int k = 1; k < kWaves; ++k) bound = min(bound, s.wtop[k]);
  bound = __builtin_amdgcn_readfirstlane(bound);

  // The tokens at or above the bound: at most 64 (the usual case) are
  // gathered per wave and ranked by wave 0; more are compacted by a block
  // prefix sum and ranked by counting.
  // key(x) >= bound as a float compare: the bound is 0 (every non-NaN token)
  // or the key of a real value (-inf or above), and NaN fails every compare.
  const float bv = bound ? key_logit(bound) : -__builtin_inff();
  uint32_t hits = 0;
#pragma unroll
  for (int i = 0; i < kDraftTokens; ++i) hits |= (x[i] >= bv ? 1u : 0u) << i;
  const uint32_t cnt = (uint32_t)__popc(hits);
  // The tokens at or above the bound into the first 64 slots, each wave's
  // at the slots it takes from a block counter (more than 64 in the block
  // leave the slots to the block's compaction below). A lane with one
  // holds it as its maximum (the one token at or above the bound is the
  // largest) at index ctz(hits); the rare lanes with more are read out one
  // at a time.
  const uint32_t wcount = lanes_reduce_u32<true>(cnt, [](uint32_t a, uint32_t b) { return a + b; });
  uint32_t first = 0;
  if (lane == 0) {
    s.wcount[w] = wcount;
    first = wcount ? atomicAdd(&s.taken, wcount) : 0u;
  }
  first = __builtin_amdgcn_readfirstlane(first);
  const uint64_t single = ballot(cnt == 1u);
  if (cnt == 1u) {
    const uint32_t slot = first + mbcnt(single);
    if (slot < 64u) {
      s.comp[slot] = draft_comp(mx, token_of(__builtin_ctz(hits)));
      s.vbits[slot] = f2u(mx);
    }
  }
  uint64_t multi = ballot(cnt > 1u);
  uint32_t slot = first + (uint32_t)__popcll(single);
  while (multi) {
    const uint32_t l = (uint32_t)__builtin_ctzll(multi);
    multi &= multi - 1u;
    uint32_t h = readlane_u32(hits, (int)l);
    while (h) {
      const uint32_t i = (uint32_t)__builtin_ctz(h);
      h &= h - 1u;
      const float v = readlane_f32(x[i], (int)l);
      if (lane == 0 && slot < 64u) {
        s.comp[slot] = draft_comp(v, base + (w * 64 + l) * 4 + (i >> 2) * 1024 + (i & 3));
        s.vbits[slot] = f2u(v);
      }
      ++slot;
    }
  }
  __syncthreads();
  const uint32_t n = __builtin_amdgcn_readfirstlane(s.taken);
  if (n <= 64) {
    // Wave 0 ranks them: lane j takes slot j and counts the entries above
    // it (sixteen slots a step, read by all lanes at once; slots past n
    // read 0), then writes its entry at its rank. Slots past n stay empty.
    if (w != 0) return;
    const uint64_t pi = ((uint64_t)row * S + chunk) * kDraftK;
    const uint64_t me = s.comp[lane];
    const uint32_t bits = s.vbits[lane];
    uint32_t rank = 0;
    for (uint32_t e = 0; e < n; e += 16) {
      ulonglong2 two[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        two[u] = *reinterpret_cast<const ulonglong2 *>(&s.comp[min(e + 2 * u, 62u)]);
#pragma unroll
      for (int u = 0; u < 8; ++u)
        rank += (two[u].x > me ? 1u : 0u) + (two[u].y > me ? 1u : 0u);
    }
    if (lane < n && rank < kDraftK) {
      d.part_comp[pi + rank] = me;
      d.part_vbits[pi + rank] = bits;
    }
    if (lane >= n && lane < kDraftK) {
      d.part_comp[pi + lane] = 0ull;
      d.part_vbits[pi + lane] = f2u(-__builtin_inff());
    }
    return;
  }
  uint32_t before = 0;
#pragma unroll
  for (int k = 0; k < kWaves; ++k) before += (uint32_t)k < w ? s.wcount[k] : 0u;
  // More than 64: the block's compaction (which rewrites the slots) and
  // ranking.
  if (n <= kThreads) {
    uint32_t pos = before + wave_incl_scan_u32(cnt) - cnt;
#pragma unroll
    for (int i = 0; i < kDraftTokens; ++i)
      if ((hits >> i) & 1u) {
        s.comp[pos] = draft_comp(x[i], token_of(i));
        s.vbits[pos] = f2u(x[i]);
        ++pos;
      }
    __syncthreads();
    // Rank by counting, eight reads in flight per step.
    if (tid < n) {
      const uint64_t me = s.comp[tid];
      uint32_t rank = 0;
      for (uint32_t e = 0; e < n; e += 8) {
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u)
          rank += e + u < n && s.comp[min(e + u, (uint32_t)kThreads - 1u)] > me ? 1u : 0u;
      }
      if (rank < kDraftK) {
        s.top[rank] = me;
        s.topv[rank] = s.vbits[tid];
      }
    }
  } else {
    // Ties: 16 rounds of the block's largest remaining entry.
    uint32_t removed = 0;
    for (uint32_t r = 0; r < kDraftK; ++r) {
      uint64_t best = 0;
#pragma unroll
      for (int i = 0; i < kDraftTokens; ++i) {
        const uint64_t c = x[i] == x[i] && !((removed >> i) & 1u) ? draft_comp(x[i], token_of(i)) : 0ull;
        best = c > best ? c : best;
      }
      const uint64_t wbest = wave_max_u64(best);
      __syncthreads();  // the previous round's readers are done
      if (lane == 0) s.wbest[w] = wbest;
      __syncthreads();
      uint64_t top = s.wbest[0];
#pragma unroll
      for (int k = 1; k < kWaves; ++k) top = s.wbest[k] > top ? s.wbest[k] : top;
      if (top == 0) break;  // uniform: nothing left
      if (best == top) {
#pragma unroll
        for (int i = 0; i < kDraftTokens; ++i)
          if (x[i] == x[i] && !((removed >> i) & 1u) && draft_comp(x[i], token_of(i)) == top) {
            removed |= 1u << i;
            s.top[r] = top;
            s.topv[r] = f2u(x[i]);
          }
      }
    }
  }
  __syncthreads();
  const uint64_t pi = ((uint64_t)row * S + chunk) * kDraftK;
  if (tid < kDraftK) {
    d.part_comp[pi + tid] = s.top[tid];
    d.part_vbits[pi + tid] = s.topv[tid];
  }
}

// The top 16 of one proposal row from its chunks' lists (each in rank
// order), by one wave: lane c holds chunk c's head (S <= 64, S <= 32 unless
// WIDE) and 16 rounds pop the largest head, comparing the value keys first
// and, where several heads share the largest, the ids. A head past its
// list's entries is 0 and never wins (a real entry's value key is nonzero);
// once every head is 0 the remaining slots stay empty. `comp`/`vbits` are
// the row's partials in LDS.
template <bool WIDE>
__device__ __forceinline__ void draft_merge_row(const uint64_t *comp, const uint32_t *vbits,
                                                uint32_t S, uint32_t *ids, float *values) {
  const uint32_t lane = lane_id();
  uint32_t head = 0;
  // Each list's head and the entry after it. Every round reads the entry
  // after that, which lands while the round compares heads (past the
  // list's end it reads the last entry; the win that would take it there
  // takes 0 instead). Lanes past S hold 0 and never win.
  const bool live = lane < S;
  uint64_t hc = live ? comp[lane * kDraftK] : 0ull;
  uint64_t hn = live ? comp[lane * kDraftK + 1] : 0ull;
  // Lane r < 16 collects slot r: its id and where its value bits lie.
  uint32_t my_id = kNoToken, my_at = ~0u;
  for (uint32_t r = 0; r < kDraftK; ++r) {
    const uint64_t after = comp[lane * kDraftK + min(head + 2, kDraftK - 1)];
    const uint32_t hi = (uint32_t)(hc >> 32);
    // top == 0: every list is spent; every lane then ties on (0, 0), lane
    // 0 takes the round and the slot stays empty.
    const uint32_t top = __builtin_amdgcn_readfirstlane(lanes_max_u32<WIDE>(hi));
    uint64_t at = ballot(hi == top);
    if (__builtin_popcountll(at) > 1) {
      const uint32_t lo = hi == top ? (uint32_t)hc : 0u;
      const uint32_t lo_top = __builtin_amdgcn_readfirstlane(lanes_max_u32<WIDE>(lo));
      at = ballot(hi == top && (uint32_t)hc == lo_top);
    }
    const uint32_t winner = (uint32_t)__builtin_ctzll(at);
    const uint32_t id = ~readlane_u32((uint32_t)hc, (int)winner);
    const uint32_t entry = winner * kDraftK + readlane_u32(head, (int)winner);
    if (lane == r && top != 0) {
      my_id = id;
      my_at = entry;
    }
    if (lane == winner) {
      ++head;
      hc = head < kDraftK ? hn : 0ull;
      hn = after;
    }
  }
  if (lane < kDraftK) {
    ids[lane] = my_id;
    values[lane] = my_at != ~0u ? u2f(vbits[my_at]) : -__builtin_inff();
  }
}

// The top 16 of one proposal row from its chunks' lists, by one wave,
// through a bound: the first m = min(64 / S, 16) entries of every list, one
// a lane, are at least 16 entries, so the 16th largest of their value keys,
// taken to its upper 16 bits (a 16-step bitwise descent), bounds the row's
// 16th entry from below. Each list's entries at or above it (a prefix: the
// lists are in rank order) are gathered into `keys`/`at` (64 slots that read
// 0 past the entries) and ranked by counting. Returns false, having written
// no output, when the bound is 0 (fewer than 16 non-empty entries among
// those probed) or more than 64 entries reach it: the caller then merges
// round by round.
__device__ __forceinline__ bool draft_merge_bounded(const uint64_t *comp, const uint32_t *vbits,
                                                    uint32_t S, uint64_t *keys, uint32_t *at,
                                                    uint32_t *ids, float *values) {
  const uint32_t lane = lane_id();
  const uint32_t m = min(64u / S, kDraftK);
  const uint32_t pc = lane / m, pt = lane - pc * m;
  const uint32_t probe = pc < S ? (uint32_t)(comp[pc * kDraftK + pt] >> 32) : 0u;
  uint32_t bound = 0;
#pragma unroll
  for (int b = 31; b >= 16; --b) {
    const uint32_t trial = bound | (1u << b);
    if ((uint32_t)__popcll(ballot(probe >= trial)) >= kDraftK) bound = trial;
  }
  if (bound == 0) return false;
  uint32_t count = 0;
  if (lane < S) {
    const ulonglong2 *list = reinterpret_cast<const ulonglong2 *>(comp + lane * kDraftK);
#pragma unroll
    for (int k = 0; k < (int)kDraftK / 2; ++k) {
      const ulonglong2 two = list[k];
      count += ((uint32_t)(two.x >> 32) >= bound ? 1u : 0u) +
               ((uint32_t)(two.y >> 32) >= bound ? 1u : 0u);
    }
  }
  const uint32_t incl = wave_incl_scan_u32(count);
  const uint32_t n = readlane_u32(incl, 63);
  if (n > 64) return false;
  for (uint32_t t = 0, o = incl - count; t < count; ++t, ++o) {
    keys[o] = comp[lane * kDraftK + t];
    at[o] = lane * kDraftK + t;
  }
  // (The wave's LDS writes land before its reads below: one wave's LDS
  // operations complete in order.)
  const uint64_t me = keys[lane];
  uint32_t rank = 0;
  for (uint32_t e = 0; e < n; e += 16) {
    ulonglong2 two[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) two[u] = *reinterpret_cast<const ulonglong2 *>(&keys[e + 2 * u]);
#pragma unroll
    for (int u = 0; u < 8; ++u) rank += (two[u].x > me ? 1u : 0u) + (two[u].y > me ? 1u : 0u);
  }
  if (lane < n && rank < kDraftK) {
    ids[rank] = ~(uint32_t)me;
    values[rank] = u2f(vbits[at[lane]]);
  }
  return true;
}

struct __align__(16) DraftEdgeLds {
  float ctx[kDraftK][kPad];   // predecessor codebook row x hidden
  float succ[kDraftK][kPad];  // successor codebook rows
  float hid[kRank];
  uint64_t pcomp[2][kDraftMaxChunks * kDraftK];  // partials of this row, previous row
  uint32_t pvbits[2][kDraftMaxChunks * kDraftK];
  uint32_t ids[2][kDraftK];                 // the merged candidates of both rows
  float vals[2][kDraftK];
  uint32_t pred[kDraftK];
  uint32_t cand[kDraftK];
  uint64_t mkeys[2][64];  // the bounded merge's entries (0 past them)
  uint32_t mat[2][64];
  uint32_t last;
};

// One proposal position of one lane: this row's top 16 from its chunk
// partials (the row's candidates and unary scores), the previous row's for
// its predecessors (the anchor at position 0), then the edge scores from
// each predecessor to each candidate, summed over the rank in ascending
// order; ids are clamped into the codebooks (sampling.metal:1259-1262),
// and the walk's step after each predecessor. The lane's last block walks.
__global__ __launch_bounds__(kThreads) void draft_edges_kernel(DraftLaunch d) {
  __shared__ DraftEdgeLds s;
  __shared__ float tbl[kDraftPositions][kDraftK * kDraftK];  // the walk's probabilities
  const uint32_t p = blockIdx.x, lane_index = blockIdx.y;
  const uint32_t row = lane_index * kDraftPositions + p, tid = threadIdx.x;
  const uint32_t V = d.vocabulary, S = d.chunks;
  const DraftLaneParams lp = d.lane_params[lane_index];
  const bool sampled = lp.sampled != 0;
  // This position's proposal uniform, requested now for the walk's step.
  const float uniform =
      sampled ? d.uniforms[(uint64_t)lane_index * kSamplingUniforms + kUniformProposals + p] : 0.0f;
  const uint32_t total = S * kDraftK, rows_here = p ? 2u : 1u;
  // Every partial load issued before any lands in LDS (a load-then-store
  // loop would wait for each round trip in turn).
  constexpr uint32_t kPartLoads = 2 * kDraftMaxChunks * kDraftK / kThreads;
  uint64_t pc[kPartLoads];
  uint32_t pv[kPartLoads];
#pragma unroll
  for (uint32_t r = 0; r < kPartLoads; ++r) {
    const uint32_t e = tid + r * kThreads;
    const uint32_t which = e >= total, k = e - which * total;
    const uint64_t at = (uint64_t)(row - which) * total + k;
    const bool in = e < rows_here * total;
    pc[r] = in ? d.part_comp[at] : 0ull;
    pv[r] = in ? d.part_vbits[at] : 0u;
  }
#pragma unroll
  for (uint32_t r = 0; r < kPartLoads; ++r) {
    const uint32_t e = tid + r * kThreads;
    const uint32_t which = e >= total, k = e - which * total;
    if (e < rows_here * total) {
      s.pcomp[which][k] = pc[r];
      s.pvbits[which][k] = pv[r];
    }
  }
  const uint16_t *h = d.hidden + ((uint64_t)lane_index * kDraftQueryRows + p + 1) * kRank;
  s.hid[tid] = bf16f(h[tid]);
  if (tid < 128) s.mkeys[tid >> 6][tid & 63] = 0ull;
  __syncthreads();
  const uint32_t wave = tid >> 6;
  if (wave < rows_here &&
      !draft_merge_bounded(s.pcomp[wave], s.pvbits[wave], S, s.mkeys[wave], s.mat[wave],
                           s.ids[wave], s.vals[wave])) {
    if (S > 32)
      draft_merge_row<true>(s.pcomp[wave], s.pvbits[wave], S, s.ids[wave], s.vals[wave]);
    else
      draft_merge_row<false>(s.pcomp[wave], s.pvbits[wave], S, s.ids[wave], s.vals[wave]);
  }
  __syncthreads();
  if (tid < kDraftK) {
    s.cand[tid] = min(s.ids[0][tid], V - 1u);
    s.pred[tid] = min(p ? s.ids[1][tid] : lp.anchor, V - 1u);
  }
  __syncthreads();
  // 16 rows x 32 sixteen-byte pieces of each codebook, two pieces a thread.
  const uint32_t preds = p ? kDraftK : 1u;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const uint32_t k = tid + r * kThreads, i = k >> 5, piece = k & 31;
    const uint4 sv = *(const uint4 *)(d.succ_codebook + (uint64_t)s.cand[i] * kRank + piece * 8);
    const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s.succ[i][piece * 8 + 2 * e] = bf16f(sw[e] & 0xffffu);
      s.succ[i][piece * 8 + 2 * e + 1] = bf16f(sw[e] >> 16);
    }
    if (i < preds) {
      const uint4 pv = *(const uint4 *)(d.pred_codebook + (uint64_t)s.pred[i] * kRank + piece * 8);
      const uint32_t pw[4] = {pv.x, pv.y, pv.z, pv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t dm = piece * 8 + 2 * e;
        s.ctx[i][dm] = bf16f(pw[e] & 0xffffu) * s.hid[dm];
        s.ctx[i][dm + 1] = bf16f(pw[e] >> 16) * s.hid[dm + 1];
      }
    }
  }
  // This row's outputs (the walk reads them back device-coherently), stored
  // after the codebook reads have landed: a wait for a read also waits for
  // every store issued before it.
  if (tid < kDraftK) {
    st_dev(d.candidates + (uint64_t)row * kDraftK + tid, s.ids[0][tid]);
    st_dev(d.unary + (uint64_t)row * kDraftK + tid, s.vals[0][tid]);
  }
  __syncthreads();
  const uint32_t i = tid >> 4, j = tid & 15;
  float *table = d.tables + (uint64_t)lane_index * kDraftPositions * kDraftK * kDraftK;
  if (i < preds) {
    // Four dimensions a read, summed one at a time in ascending order.
    const f32x4 *cr = reinterpret_cast<const f32x4 *>(s.ctx[i]);
    const f32x4 *sr = reinterpret_cast<const f32x4 *>(s.succ[j]);
    float acc = 0.0f;
#pragma unroll 8
    for (uint32_t q4 = 0; q4 < kRank / 4; ++q4) {
      const f32x4 a = cr[q4], b = sr[q4];
      acc = acc + a.x * b.x;
      acc = acc + a.y * b.y;
      acc = acc + a.z * b.z;
      acc = acc + a.w * b.w;
    }
    st_dev(table + (p * kDraftK + i) * kDraftK + j, acc);
    // The walk's step at this position after each predecessor i
    // (sampling.metal:1316-1359), row i with lane j holding candidate j:
    // the score is the candidate's unary plus the edge. The row maximum is
    // a DPP reduction (fmax is order-free, so it equals the running
    // maximum); the sum and the cumulative sums, whose rounding depends on
    // the order, go in candidate order.
    const float score = s.vals[0][j] + acc;
    const uint32_t shift = tid & 48;
    uint32_t pick = 0;
    if (sampled) {
      const float maximum = row_max_f32(score);
      const float prob = exp_weight((score - maximum) / lp.temperature);
      const float sum = row_lane_f32(row_ordered_sums(prob, j), kDraftK - 1);
      const float q = prob / sum;
      st_dev(d.choice_q + ((uint64_t)row * kDraftK + i) * kDraftK + j, q);
      // The first candidate whose cumulative sum passes the uniform, else
      // the last.
      const uint32_t passed =
          (uint32_t)(ballot(row_ordered_sums(q, j) > uniform) >> shift) & 0xffffu;
      pick = passed ? (uint32_t)__builtin_ctz(passed) : kDraftK - 1;
    } else {
      // The first strict maximum in candidate order: candidate 0 when its
      // score is NaN (nothing compares above it), else the first candidate
      // holding the largest non-NaN score.
      const float s0 = row_lane_f32(score, 0);
      if (s0 == s0) {
        const float best = row_max_f32(score);
        pick = (uint32_t)__builtin_ctz((uint32_t)(ballot(score == best) >> shift) & 0xffffu);
      }
    }
    if (j == 0) st_dev(d.choices + (uint64_t)row * kDraftK + i, pick);
  }
  wait_memory();
  __syncthreads();
  if (tid == 0) {
    uint32_t *counter = d.counters + d.lanes * kDraftPositions + lane_index;
    const uint32_t prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    s.last = prev == kDraftPositions - 1 ? 1u : 0u;
    if (prev == kDraftPositions - 1) st_dev(counter, 0u);
  }
  __syncthreads();
  if (!s.last) return;

  // The walk: the last block of the lane chains the positions' steps. Lane
  // c holds position pp's candidate c and pick after predecessor c; the
  // picked row's probabilities come through LDS. Every load issued before
  // any lands.
  const uint64_t r0 = (uint64_t)lane_index * kDraftPositions * kDraftK;
  static_assert(kDraftK * kDraftK == kThreads, "one probability per thread and position");
  float qv[kDraftPositions];
  if (sampled) {
#pragma unroll
    for (uint32_t pp = 0; pp < kDraftPositions; ++pp)
      qv[pp] = pp || tid < kDraftK ? ld_dev(d.choice_q + (r0 + pp * kDraftK) * kDraftK + tid) : 0.0f;
  }
  uint32_t cv[kDraftPositions] = {}, picks[kDraftPositions] = {};
  if (tid < kDraftK) {
#pragma unroll
    for (uint32_t pp = 0; pp < kDraftPositions; ++pp) {
      cv[pp] = ld_dev(d.candidates + r0 + pp * kDraftK + tid);
      picks[pp] = pp || tid == 0 ? ld_dev(d.choices + r0 + pp * kDraftK + tid) : 0u;
    }
  }
  if (sampled) {
#pragma unroll
    for (uint32_t pp = 0; pp < kDraftPositions; ++pp) tbl[pp][tid] = qv[pp];
    __syncthreads();
  }
  if (tid >= 64) return;
  const uint32_t lane = tid;
  // The chain of picks first (scalar work), then every store.
  uint32_t from[kDraftPositions], pick[kDraftPositions];
  uint32_t pred_index = 0;
#pragma unroll
  for (uint32_t pp = 0; pp < kDraftPositions; ++pp) {
    from[pp] = pred_index;
    pick[pp] = readlane_u32(picks[pp], (int)pred_index);
    pred_index = pick[pp];
  }
  if (lane < kDraftPositions) {
    uint32_t token = 0;
#pragma unroll
    for (uint32_t pp = 0; pp < kDraftPositions; ++pp)
      if (lane == pp) token = readlane_u32(cv[pp], (int)pick[pp]);
    d.tokens[(uint64_t)lane_index * kDraftPositions + lane] = token;
  }
  if (sampled && lane < kDraftK) {
#pragma unroll
    for (uint32_t pp = 0; pp < kDraftPositions; ++pp)
      d.q_probs[(r0 + pp * kDraftK) + lane] = tbl[pp][from[pp] * kDraftK + lane];
  }
}

int launch_draft_select(const DraftLaunch &d, bool aligned, void *stream,
                        void *start_event, void *stop_event) {
  const hipStream_t st = (hipStream_t)stream;
  const dim3 g1(d.chunks, d.lanes * kDraftPositions), block(kThreads);
  if (aligned)
    hipExtLaunchKernelGGL(draft_top16_kernel<true>, g1, block, 0, st, (hipEvent_t)start_event,
                          (hipEvent_t)stop_event, 0, d);
  else
    hipExtLaunchKernelGGL(draft_top16_kernel<false>, g1, block, 0, st, (hipEvent_t)start_event,
                          (hipEvent_t)stop_event, 0, d);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL(draft_edges_kernel, dim3(kDraftPositions, d.lanes), block, 0, st, d);
  return (int)hipGetLastError();
}

}  // namespace jf
