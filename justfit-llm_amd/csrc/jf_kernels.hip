// gfx950 kernels of JustFit's logits->token path.
//
// One selection is one launch of select_kernel over rows x chunks blocks
// (plus, for rows whose candidates do not fit, the multi-pass stage_kernel
// launches). Each block holds its chunk of a row in registers: one pass over
// HBM with 16-byte loads, the penalties, the constraint mask and the stop
// exclusion applied on the fly (the reference's decode_sample_penalize,
// TargetRow::admits; sampling.metal:33-37, 928-993). A greedy row reduces its
// argmax (sampling.metal:1427-1512); a sampled row writes its chunk's
// maximum and the tokens that can still belong to its min-p/top-k/top-p
// distribution. The last block of a row to finish (the reference's
// split_arrive_last, split_reduce.h:14-28) merges: the global maximum, the
// min-p floor, the exact top-k in (logit desc, id asc) order, the top-p
// nucleus, and the inverse-CDF draw in id order with the residual of a
// drafted row (sampling.metal:585-829). Every sum that decides a token is an
// exact 64-bit sum of floor(w * 2^44), so the parallel order never changes
// a result.
#include <hip/hip_ext.h>

#include <mutex>

#include "jf_device.h"
#include "jf_kernels.h"

// The kernels compile in four parts (JF_PART 1..4, one object each) so the
// build runs in parallel; JF_PART 0 (the default) compiles all of them.
#ifndef JF_PART
#define JF_PART 0
#endif
#define JF_IN(p) (JF_PART == 0 || JF_PART == (p))

namespace jf {

template <int DT>
struct Geo;
template <>
struct Geo<0> {  // fp32: 4 tokens per 16-byte load
  static constexpr int VEC = 4, LOADS = 8, TPL = 32, SLAB = kThreads * VEC;
  static constexpr uint32_t CHUNK = kChunkF32;
};
template <>
struct Geo<1> {  // bf16: 8 tokens per 16-byte load
  static constexpr int VEC = 8, LOADS = 4, TPL = 32, SLAB = kThreads * VEC;
  static constexpr uint32_t CHUNK = kChunkBF16;
};

constexpr uint32_t kMaxChunkWords = kChunkF32 / 32;
constexpr uint32_t kLowestKey = 0x007fffffu;  // the key of -infinity
constexpr uint32_t kMaxChunks = 64;

// A chunk's penalized values, compact: the table's entries of the chunk
// (sorted by token) are processed in rounds of kPenaltySlots; an entry's
// value sits at its rank within the round, and the lane holding a token
// finds that rank from the bitmap: the rank of its word's first entry plus
// the entries before it in the word. Extra (draft) tokens the table does
// not hold have their own bitmap and values by extra index.
constexpr uint32_t kPenaltySlots = 512;
struct PrepLds {
  float pvals[kPenaltySlots + 8];  // + the reads past a vector's last entry
  uint32_t pbits[kMaxChunkWords];  // this round's entries
  uint32_t wrank[kMaxChunkWords];  // rank of each word's first entry
  uint32_t tbits[kMaxChunkWords];  // every entry of the chunk (verify rows)
  uint32_t xbits[kMaxChunkWords];  // extra tokens outside the table
  float xvals[kMaxExtra];
  uint32_t extras[kMaxExtra];
};
struct MergeLds {
  uint32_t key[kMergeCapacity];
  uint32_t id[kMergeCapacity];
  uint8_t fl[kMergeCapacity];
  uint32_t bins[1024];
};

struct __align__(16) Lds {
  union {
    PrepLds prep;
    MergeLds merge;
  };
  uint64_t hist[256];
  uint64_t wj[kWaves][8];
  uint64_t wl[kWaves];
  float wf[kWaves];
  uint32_t wu[kWaves];
  uint32_t wu2[kWaves];
  float hmax[kMaxChunks];
  uint32_t hcnt[kMaxChunks];
  uint32_t hoff[kMaxChunks + 1];
  uint32_t cids[16];
  float cprobs[16];
  uint32_t last;
  uint32_t sel_bin;
  uint64_t sel_excl;
  uint32_t hit;
  uint32_t found_id;
  float found_w;
  uint32_t u32a;
  uint32_t nbound;
  float row_max;
  uint32_t row_admitted;
  uint32_t row_overflow;
  uint32_t row_floor;
  uint32_t row_maxcount;
  uint32_t row_long;  // merge_small_kernel: a list is longer than its fetched slots
  uint64_t u64a;
};

// The select kernel's LDS: the chunk's penalty lookup and the reductions.
constexpr uint32_t kWaveCandidates = kBlockCandidates / kWaves;
struct __align__(16) SelectLds {
  PrepLds prep;
  uint64_t stage[kWaves][kWaveCandidates];  // each wave's candidates
  uint32_t wcount[kWaves];
  uint64_t wj[kWaves][8];
  uint64_t wl[kWaves];
  uint64_t slices[kWaves * 8];  // an uncut row's slice masses
  float wf[kWaves];
  uint32_t wu[kWaves];
  uint32_t wu2[kWaves];
};

// The mass-and-draw kernel's LDS: the chunk's penalty lookup, the
// reductions and the walk's offsets (no merge buffers, so more blocks stay
// resident during the mass pass).
struct __align__(16) DrawLds {
  PrepLds prep;
  uint64_t wj[kWaves][8];
  uint64_t wl[kWaves];
  uint32_t cids[16];
  float cprobs[16];
  uint32_t last;
  uint32_t hit;
  uint32_t sel_bin;
  uint64_t sel_excl;
  uint64_t u64a;
  uint32_t slice;          // the last block's slice and its remainder
  uint64_t slice_within;
};

// ---- block helpers (every thread of the block calls them) ---------------

template <class L>
__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, L &s) {
  v = wave_sum_u32(v);
  __syncthreads();
  if (lane_id() == 0) s.wu[threadIdx.x >> 6] = v;
  __syncthreads();
  return s.wu[0] + s.wu[1] + s.wu[2] + s.wu[3];
}
template <class L>
__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, L &s) {
  v = wave_sum_u64(v);
  __syncthreads();
  if (lane_id() == 0) s.wl[threadIdx.x >> 6] = v;
  __syncthreads();
  return s.wl[0] + s.wl[1] + s.wl[2] + s.wl[3];
}
template <class L>
__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, L &s) {
  v = wave_max_u32(v);
  __syncthreads();
  if (lane_id() == 0) s.wu[threadIdx.x >> 6] = v;
  __syncthreads();
  return max(max(s.wu[0], s.wu[1]), max(s.wu[2], s.wu[3]));
}
template <class L>
__device__ __forceinline__ uint32_t block_min_u32(uint32_t v, L &s) {
  v = wave_min_u32(v);
  __syncthreads();
  if (lane_id() == 0) s.wu[threadIdx.x >> 6] = v;
  __syncthreads();
  return min(min(s.wu[0], s.wu[1]), min(s.wu[2], s.wu[3]));
}
template <class L>
__device__ __forceinline__ float block_max_f32(float v, L &s) {
  v = wave_max_f32(v);
  __syncthreads();
  if (lane_id() == 0) s.wf[threadIdx.x >> 6] = v;
  __syncthreads();
  return __builtin_fmaxf(__builtin_fmaxf(s.wf[0], s.wf[1]),
                         __builtin_fmaxf(s.wf[2], s.wf[3]));
}
// Exclusive prefix over threads in thread order; *total gets the block sum.
template <class L>
__device__ __forceinline__ uint64_t block_excl_scan_u64(uint64_t v, L &s,
                                                        uint64_t *total) {
  const uint64_t incl = wave_incl_scan_u64(v);
  const uint32_t w = threadIdx.x >> 6;
  __syncthreads();
  if (lane_id() == 63) s.wl[w] = incl;
  __syncthreads();
  uint64_t off = 0, tot = 0;
#pragma unroll
  for (int k = 0; k < kWaves; ++k) {
    off += (k < (int)w) ? s.wl[k] : 0;
    tot += s.wl[k];
  }
  if (total) *total = tot;
  return off + incl - v;
}

// Wave 0 finds the highest bin b of s.hist whose suffix sum (bins >= b)
// reaches T; s.sel_bin = b, s.sel_excl = sum of the bins above b. The
// caller guarantees the total reaches T.
__device__ __forceinline__ void crossing_bin(Lds &s, uint64_t T) {
  if (threadIdx.x < 64) {
    const uint32_t l = threadIdx.x;
    const uint64_t h0 = s.hist[4 * l], h1 = s.hist[4 * l + 1],
                   h2 = s.hist[4 * l + 2], h3 = s.hist[4 * l + 3];
    const uint64_t own = h0 + h1 + h2 + h3;
    // Suffix sum over lanes: the total less the prefix before this lane.
    const uint64_t incl = wave_incl_scan_u64(own);
    const uint64_t suf = readlane_u64(incl, 63) - (incl - own);
    const uint64_t m = ballot(suf >= T);
    const int L = m ? (int)__popcll(m) - 1 : 0;
    const uint64_t above = readlane_u64(suf - own, L);
    if ((int)l == L) {
      // Walk this lane's four bins from the top.
      uint64_t acc = above;
      uint32_t bin = 4 * l;
      uint64_t excl = acc;
      if (acc + h3 >= T) {
        bin = 4 * l + 3;
        excl = acc;
      } else if (acc + h3 + h2 >= T) {
        bin = 4 * l + 2;
        excl = acc + h3;
      } else if (acc + h3 + h2 + h1 >= T) {
        bin = 4 * l + 1;
        excl = acc + h3 + h2;
      } else {
        bin = 4 * l;
        excl = acc + h3 + h2 + h1;
      }
      s.sel_bin = bin;
      s.sel_excl = excl;
    }
  }
  __syncthreads();
}

__device__ __forceinline__ bool at_or_before(uint32_t key, uint32_t token,
                                             uint32_t bkey, uint32_t bid) {
  return key > bkey || (key == bkey && token <= bid);
}

// ---- one chunk of one row into registers ---------------------------------

constexpr float kNotAdmitted = __builtin_nanf("");

// Makes the compiler treat the chunk's registers as rewritten here, so it
// does not hoist per-token work out of the loop that follows (which would
// hold a second copy of the chunk in registers).
template <int N>
__device__ __forceinline__ void opaque(float (&xs)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(xs[i]));
}
// A load through the scalar cache (uniform address). Its wait counts only
// scalar loads, so it does not wait behind the vector loads in flight.
__device__ __forceinline__ uint32_t scalar_load_u32(const uint32_t *p) {
  const uint64_t addr = (uint64_t)p;
  const uint64_t u =
      ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(addr >> 32)) << 32) |
      (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)addr);
  uint32_t v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)"
               : "=s"(v)
               : "s"(u)
               : "memory");
  return v;
}
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// The select kernel's first round of a chunk's penalized tokens, held by
// the threads of their table entries: token id and penalized value (NaN when
// the row does not admit the token). The lanes that hold these tokens drop
// them, so each token counts once.
constexpr int kSideEntries = kPenaltySlots / kThreads;
struct SideEntries {
  uint32_t tok[kSideEntries];
  float val[kSideEntries];
};

// Loads chunk `chunk` of `row`: xs[j*VEC+e] is token
// chunk*CHUNK + j*SLAB + tid*VEC + e (SLAB = kThreads*VEC: the block's j-th
// 16-byte loads cover one contiguous slab, so a partial last chunk leaves
// every thread some of its tokens)
// after its penalties, or NaN when the row does not admit it (outside the
// vocabulary, outside a constrained row's mask, an excluded stop token). A
// NaN logit is never selected either (greedy comparisons skip it, sampled
// rows keep no NaN), so one NaN test covers both. Block-uniform control
// flow: every thread calls it.
template <int DT, bool kSide = false, class L>
__device__ __forceinline__ void load_chunk(const SampleLaunch &a,
                                           const RowParams &rp, uint32_t row,
                                           uint32_t chunk, L &s,
                                           float (&xs)[Geo<DT>::TPL],
                                           SideEntries *side = nullptr) {
  constexpr int VEC = Geo<DT>::VEC, LOADS = Geo<DT>::LOADS,
                SLAB = Geo<DT>::SLAB;
  constexpr uint32_t CHUNK = Geo<DT>::CHUNK;
  constexpr uint32_t VMASK = (1u << VEC) - 1u;
  const uint32_t tid = threadIdx.x;
  const uint32_t V = a.vocabulary;
  const uint32_t base = chunk * CHUNK;
  const uint32_t lane_base = base + tid * VEC;

  if constexpr (DT == 0) {
    const float *rowp = (const float *)a.logits + (uint64_t)row * a.stride;
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const uint32_t t0 = lane_base + j * SLAB;
      if (t0 + VEC <= V && a.aligned) {
        const f32x4 v = *(const f32x4 *)(rowp + t0);
        xs[j * 4 + 0] = v.x;
        xs[j * 4 + 1] = v.y;
        xs[j * 4 + 2] = v.z;
        xs[j * 4 + 3] = v.w;
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          xs[j * VEC + e] = (t0 + e < V) ? rowp[t0 + e] : kNotAdmitted;
      }
    }
  } else {
    const uint16_t *rowp =
        (const uint16_t *)a.logits + (uint64_t)row * a.stride;
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const uint32_t t0 = lane_base + j * SLAB;
      if (t0 + VEC <= V && a.aligned) {
        const u32x4 v = *(const u32x4 *)(rowp + t0);
        xs[j * 8 + 0] = u2f(v.x << 16);
        xs[j * 8 + 1] = u2f(v.x & 0xffff0000u);
        xs[j * 8 + 2] = u2f(v.y << 16);
        xs[j * 8 + 3] = u2f(v.y & 0xffff0000u);
        xs[j * 8 + 4] = u2f(v.z << 16);
        xs[j * 8 + 5] = u2f(v.z & 0xffff0000u);
        xs[j * 8 + 6] = u2f(v.w << 16);
        xs[j * 8 + 7] = u2f(v.w & 0xffff0000u);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          xs[j * VEC + e] =
              (t0 + e < V) ? bf16_to_float(rowp[t0 + e]) : kNotAdmitted;
      }
    }
  }

  // The constraint mask words of those tokens (constrained rows), also
  // requested before anything waits.
  const bool constrained = (rp.flags & kRowConstrained) != 0;
  uint32_t mwords[LOADS];
  if (constrained) {
    const uint32_t *mrow = a.masks + (uint64_t)rp.mask_row * a.mask_stride;
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const uint32_t t0 = lane_base + j * SLAB;
      mwords[j] = t0 < V ? mrow[t0 >> 5] : 0u;
    }
  }

  // Penalty entries of this chunk: its range in the table by scalar loads
  // (which do not wait behind the vector loads above), then the entries,
  // which arrive after the logits (vector loads complete in issue order).
  const bool penalized = (rp.flags & kRowPenalized) != 0;
  constexpr uint32_t NWORDS = CHUNK / 32;
  constexpr int EPT = kPenaltySlots / kThreads;  // entries per thread held in registers
  const uint32_t nx = penalized ? rp.extra_count : 0u;
  if constexpr (kSide) {
#pragma unroll
    for (int k = 0; k < kSideEntries; ++k) {
      side->tok[k] = kNoToken;
      side->val[k] = kNotAdmitted;
    }
  }
  uint32_t lo = 0, hi = 0;
  const uint2 *ent = nullptr;
  uint2 pe[EPT];
  if (penalized) {
    PrepLds &p = s.prep;
    for (uint32_t i = tid; i < NWORDS; i += kThreads) {
      p.pbits[i] = 0;
      p.wrank[i] = kNoToken;
      if (nx) {
        p.tbits[i] = 0;
        p.xbits[i] = 0;
      }
    }
    if (tid < nx) p.extras[tid] = a.extra[(uint64_t)rp.extra_offset + tid];
    const uint32_t prow = rp.penalty_row;
    const uint32_t *offs = a.pen_offsets + (uint64_t)prow * (a.pen_buckets + 1);
    const uint32_t b0 = base / kPenaltyBucket;
    const uint32_t b1 = min((base + CHUNK) / kPenaltyBucket, a.pen_buckets);
    lo = scalar_load_u32(offs + b0);
    hi = scalar_load_u32(offs + b1);
    ent = a.pen_entries + (uint64_t)prow * a.pen_max_entries;
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const uint32_t i = lo + tid + k * kThreads;
      pe[k] = i < hi ? ent[i] : make_uint2(kNoToken, 0u);
    }
  }

  if (penalized) {
    // Each entry's thread reads its token's logit again (an L2 hit: the
    // block has just loaded it) and writes the penalized value
    // (sampling.metal:928-963) at its rank; the lanes holding the tokens
    // take the values. Verify rows also count the extra (draft) tokens of
    // their context. An entry with nothing to apply keeps its logit.
    PrepLds &p = s.prep;
    auto value_of = [&](uint32_t t, uint32_t word) -> float {
      uint32_t count = word & kCountMask;
      for (uint32_t k = 0; k < nx; ++k) count += p.extras[k] == t;
      const float x = DT == 0 ? ((const float *)a.logits)[(uint64_t)row * a.stride + t]
                              : bf16_to_float(((const uint16_t *)a.logits)[(uint64_t)row * a.stride + t]);
      if (!count && !(word & kPromptBit)) return x;
      return penalize(x, count, rp.repetition, rp.repetition_inverse, rp.presence,
                      rp.frequency);
    };
    auto place = [&](uint32_t t, uint32_t word, uint32_t rank) {
      const uint32_t o = t - base;
      p.pvals[rank] = value_of(t, word);
      atomicOr(&p.pbits[o >> 5], 1u << (o & 31));
      atomicMin(&p.wrank[o >> 5], rank);
      if (nx) atomicOr(&p.tbits[o >> 5], 1u << (o & 31));
    };
    // The lanes take this round's values: the vector's first rank is its
    // word's first rank plus the entries before it in the word; its k-th
    // penalized token takes the value k places further.
    auto take = [&]() {
#pragma unroll
      for (int j = 0; j < LOADS; ++j) {
        const uint32_t o0 = j * SLAB + tid * VEC;
        const uint32_t pw = p.pbits[o0 >> 5];
        const uint32_t sh = o0 & 31;
        const uint32_t nib = (pw >> sh) & VMASK;
        if (nib) {
          const uint32_t r = p.wrank[o0 >> 5] + __popc(pw & ((1u << sh) - 1u));
          if constexpr (VEC == 4) {
            const float v0 = p.pvals[r], v1 = p.pvals[r + 1], v2 = p.pvals[r + 2],
                        v3 = p.pvals[r + 3];
            const uint32_t c1 = nib & 1u, c2 = c1 + ((nib >> 1) & 1u),
                           c3 = c2 + ((nib >> 2) & 1u);
            float *x = &xs[j * 4];
            x[0] = (nib & 1u) ? v0 : x[0];
            x[1] = (nib & 2u) ? (c1 ? v1 : v0) : x[1];
            x[2] = (nib & 4u) ? (c2 == 0 ? v0 : (c2 == 1 ? v1 : v2)) : x[2];
            x[3] = (nib & 8u) ? (c3 == 0 ? v0 : (c3 == 1 ? v1 : (c3 == 2 ? v2 : v3))) : x[3];
          } else {
            uint32_t rr = r;
#pragma unroll
            for (int e = 0; e < VEC; ++e)
              if ((nib >> e) & 1u) xs[j * VEC + e] = p.pvals[rr++];
          }
        }
      }
    };
    const uint32_t total = hi - lo;
    __syncthreads();  // bitmaps cleared, extras staged
    if constexpr (kSide) {
      // The first round's tokens stay with their entries' threads (value
      // and admission computed there); the lanes holding them drop them.
      static_assert(EPT == kSideEntries, "one side entry per prefetched entry");
      const uint32_t *mrow = a.masks + (uint64_t)rp.mask_row * a.mask_stride;
#pragma unroll
      for (int k = 0; k < EPT; ++k) {
        const uint32_t e = tid + k * kThreads;
        if (e < total) {
          const uint32_t t = pe[k].x, o = t - base;
          atomicOr(&p.pbits[o >> 5], 1u << (o & 31));
          if (nx) atomicOr(&p.tbits[o >> 5], 1u << (o & 31));
          float v = value_of(t, pe[k].y);
          if (constrained && !((mrow[t >> 5] >> (t & 31)) & 1u)) v = kNotAdmitted;
          if ((rp.flags & kRowExcludeStop) && (t == a.stop0 || t == a.stop1)) v = kNotAdmitted;
          side->tok[k] = t;
          side->val[k] = v;
        }
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < LOADS; ++j) {
        const uint32_t o0 = j * SLAB + tid * VEC;
        const uint32_t nib = (p.pbits[o0 >> 5] >> (o0 & 31)) & VMASK;
        if (nib) {
#pragma unroll
          for (int e = 0; e < VEC; ++e)
            xs[j * VEC + e] = ((nib >> e) & 1u) ? kNotAdmitted : xs[j * VEC + e];
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < EPT; ++k) {
        const uint32_t e = tid + k * kThreads;
        if (e < total) place(pe[k].x, pe[k].y, e);
      }
      __syncthreads();
      take();
    }
    // More entries than one round holds (a history crowded into this
    // chunk): further rounds, entries read as they go.
    for (uint32_t r0 = kPenaltySlots; r0 < total; r0 += kPenaltySlots) {
      __syncthreads();
      for (uint32_t i = tid; i < NWORDS; i += kThreads) {
        p.pbits[i] = 0;
        p.wrank[i] = kNoToken;
      }
      __syncthreads();
      for (uint32_t e = r0 + tid; e < min(total, r0 + kPenaltySlots); e += kThreads) {
        const uint2 en = ent[lo + e];
        place(en.x, en.y, e - r0);
      }
      __syncthreads();
      take();
    }
    if (nx) {
      // Extra tokens the table does not hold: the first of equal ones
      // applies, with the count of all of them.
      __syncthreads();
      if (tid < nx) {
        const uint32_t t = p.extras[tid];
        bool first = t >= base && t < base + CHUNK && t < V;
        for (uint32_t k = 0; k < tid; ++k) first = first && p.extras[k] != t;
        if (first && !((p.tbits[(t - base) >> 5] >> ((t - base) & 31)) & 1u)) {
          p.xvals[tid] = value_of(t, 0u);
          atomicOr(&p.xbits[(t - base) >> 5], 1u << ((t - base) & 31));
        }
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < LOADS; ++j) {
        const uint32_t o0 = j * SLAB + tid * VEC;
        const uint32_t nib = (p.xbits[o0 >> 5] >> (o0 & 31)) & VMASK;
        if (nib) {
#pragma unroll
          for (int e = 0; e < VEC; ++e)
            if ((nib >> e) & 1u) {
              const uint32_t t = base + o0 + e;
              uint32_t k = 0;
              while (p.extras[k] != t) ++k;  // the first equal extra
              xs[j * VEC + e] = p.xvals[k];
            }
        }
      }
    }
    __syncthreads();  // the prep area is reused by the caller
  }

  // Admission: the constraint mask and the stop tokens.
  uint32_t stop_j[2] = {0xffu, 0xffu}, stop_e[2] = {0, 0};
  if (rp.flags & kRowExcludeStop) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const uint32_t st = k ? a.stop1 : a.stop0;
      if (st >= base && st < base + CHUNK) {
        const uint32_t o = st - base;
        if ((o % SLAB) / VEC == tid) {
          stop_j[k] = o / SLAB;
          stop_e[k] = o % VEC;
        }
      }
    }
  }
  if (constrained || (rp.flags & kRowExcludeStop)) {
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const uint32_t t0 = lane_base + j * SLAB;
      uint32_t vm = VMASK;
      if (constrained && t0 < V) vm = (mwords[j] >> (t0 & 31)) & VMASK;
      if (stop_j[0] == (uint32_t)j) vm &= ~(1u << stop_e[0]);
      if (stop_j[1] == (uint32_t)j) vm &= ~(1u << stop_e[1]);
      if (vm != VMASK) {
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          xs[j * VEC + e] = ((vm >> e) & 1u) ? xs[j * VEC + e] : kNotAdmitted;
      }
    }
  }
}

// Offsets in block id order. A chunk's tokens run in (j, tid, e) order:
// load j of every thread, threads ascending, VEC tokens each. Given each
// thread's per-load values v[j] (counts or weights), off[j] is the sum of
// the values of every load that comes before this thread's load j; returns
// the block total. Every thread calls it.
template <int LOADS, class T, class L>
__device__ __forceinline__ T order_offsets(const T (&v)[LOADS], T (&off)[LOADS],
                                           L &s) {
  const uint32_t w = threadIdx.x >> 6;
  T incl[LOADS];
#pragma unroll
  for (int j = 0; j < LOADS; ++j) {
    if constexpr (sizeof(T) == 8)
      incl[j] = wave_incl_scan_u64(v[j]);
    else
      incl[j] = wave_incl_scan_u32(v[j]);
  }
  __syncthreads();
  if (lane_id() == 63)
#pragma unroll
    for (int j = 0; j < LOADS; ++j) s.wj[w][j] = (uint64_t)incl[j];
  __syncthreads();
  T run = 0;
#pragma unroll
  for (int j = 0; j < LOADS; ++j) {
    T before = 0, tot = 0;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) {
      const T t = (T)s.wj[k][j];
      before += k < (int)w ? t : T(0);
      tot += t;
    }
    off[j] = run + before + incl[j] - v[j];
    run += tot;
  }
  return run;
}

// ---- outputs --------------------------------------------------------------

__device__ __forceinline__ void write_result(const SampleLaunch &a,
                                             uint32_t row, uint32_t token,
                                             float draft_p, uint32_t kept) {
  a.out_tokens[row] = token;
  if (a.out_draft) a.out_draft[row] = draft_p;
  if (a.out_kept_counts) a.out_kept_counts[row] = kept;
}

__device__ __forceinline__ float row_uniform(const SampleLaunch &a,
                                             uint32_t row) {
  return a.uniforms[a.uniform_index ? (uint64_t)a.uniform_index[row]
                                     : a.uniform_offset + row * a.uniform_stride];
}

// The draft token a row's draw corrects, or kNoToken.
__device__ __forceinline__ uint32_t row_draft(const SampleLaunch &a, const RowParams &rp) {
  return (a.draft_tokens && rp.draft_index != kNoToken) ? a.draft_tokens[rp.draft_index]
                                                        : kNoToken;
}

// The draft's probability of `token` for a drafted row: its dense q, or
// the first sparse candidate that lists it (sampling.metal:703-708); the
// merge stages the row's 16 candidates in s.cids/s.cprobs.
// A sampled row with no min-p, top-k or top-p cut: it keeps every admitted
// token. The merges and stages skip such rows; uncut_kernel draws them.
__device__ __forceinline__ bool uncut_row(const RowParams &rp) {
  return (rp.flags & kRowSampled) && !(rp.flags & (kRowMinP | kRowTopK | kRowTopP));
}

template <class L>
__device__ __forceinline__ float draft_q(const SampleLaunch &a, const RowParams &rp,
                                         uint32_t token, const L &s) {
  if (a.dense_q) return a.dense_q[(uint64_t)rp.cand_index * a.q_stride + token];
  for (int j = 0; j < 16; ++j)
    if (s.cids[j] == token) return s.cprobs[j];
  return 0.0f;
}
template <class L>
__device__ __forceinline__ void stage_candidates(const SampleLaunch &a,
                                                 const RowParams &rp, L &s) {
  if (threadIdx.x < 16) {
    const bool sparse = !a.dense_q && row_draft(a, rp) != kNoToken;
    const uint64_t c = (uint64_t)rp.cand_index * 16 + threadIdx.x;
    s.cids[threadIdx.x] = sparse ? a.cand_ids[c] : kNoToken;
    s.cprobs[threadIdx.x] = sparse ? a.cand_probs[c] : 0.0f;
  }
  __syncthreads();
}

// A drafted row's residual weight max(wq - Q, 0) (sampling.metal:700-708,
// 760-765): Q = floor(q * m) for m the mass rounded to a float and the
// product rounded to a float (both to nearest even); q NaN or <= 0 takes
// nothing off. Every weight is at most 2^44, so a product at or above 2^44
// leaves nothing; below it the product's integer part is two exact 32-bit
// conversions (its floor over 2^32, and the remainder, which the fused
// multiply-add leaves exact).
__device__ __forceinline__ uint64_t residual_of(uint64_t wq, uint64_t mass,
                                                float q) {
  const float x = q > 0.0f ? q * (float)mass : 0.0f;
  if (!(x < 0x1p44f)) return 0;
  const float hf = __builtin_floorf(x * 0x1p-32f);
  const uint64_t qm =
      ((uint64_t)(uint32_t)hf << 32) | (uint32_t)__builtin_fmaf(hf, -0x1p32f, x);
  return wq > qm ? wq - qm : 0;
}

// ---- the merge of a sampled row ------------------------------------------

// Items of the merge live in s.merge (key, id, flag) in id order. Per-thread
// contiguous ranges give ordered scans.
struct ItemRange {
  uint32_t begin, end;
};
__device__ __forceinline__ ItemRange my_items(uint32_t n) {
  const uint32_t per = (n + kThreads - 1) / kThreads;
  const uint32_t b = min(threadIdx.x * per, n);
  return {b, min(b + per, n)};
}

// Keeps, among flagged items, the first `keep` in (key desc, id asc) order:
// radix descent over the key bytes, then the lowest ids among the ties.
__device__ __forceinline__ void lds_topk(Lds &s, uint32_t n, uint32_t keep) {
  MergeLds &m = s.merge;
  uint32_t prefix = 0, pmask = 0;
  uint64_t need = keep;
  for (int d = 3; d >= 0; --d) {
    s.hist[threadIdx.x] = 0;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < n; i += kThreads) {
      const uint32_t k = m.key[i];
      if (m.fl[i] && (k & pmask) == prefix)
        atomicAdd((unsigned long long *)&s.hist[(k >> (8 * d)) & 255u], 1ull);
    }
    __syncthreads();
    crossing_bin(s, need);
    need -= s.sel_excl;
    prefix |= s.sel_bin << (8 * d);
    pmask |= 255u << (8 * d);
    __syncthreads();
  }
  // need = how many tokens tied at `prefix` stay, lowest ids first.
  const ItemRange r = my_items(n);
  uint32_t ties = 0;
  for (uint32_t i = r.begin; i < r.end; ++i) ties += m.fl[i] && m.key[i] == prefix;
  uint32_t rank = (uint32_t)block_excl_scan_u64(ties, s, nullptr);
  for (uint32_t i = r.begin; i < r.end; ++i) {
    if (!m.fl[i]) continue;
    const uint32_t k = m.key[i];
    if (k > prefix) continue;
    if (k < prefix) {
      m.fl[i] = 0;
    } else {
      m.fl[i] = rank < need ? 1 : 0;
      ++rank;
    }
  }
  __syncthreads();
}

// Top-p over the flagged items (sampling.metal:615-641): keep them in order
// until the running mass exceeds floor(top_p * mass); that token stays.
__device__ __forceinline__ void lds_topp(Lds &s, uint32_t n, float maximum, float inv_t,
                         float top_p) {
  MergeLds &m = s.merge;
  uint64_t local = 0;
  for (uint32_t i = threadIdx.x; i < n; i += kThreads)
    if (m.fl[i]) local += quantize(weight_of(key_logit(m.key[i]), maximum, inv_t));
  const uint64_t mass = block_sum_u64(local, s);
  if (mass == 0) return;  // nothing weighs: the nucleus never closes
  const uint64_t nucleus = floor_mul(mass, top_p);
  uint64_t need = nucleus + 1;  // the kept prefix's mass must reach this
  uint32_t prefix = 0, pmask = 0;
  for (int d = 3; d >= 0; --d) {
    s.hist[threadIdx.x] = 0;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < n; i += kThreads) {
      const uint32_t k = m.key[i];
      if (m.fl[i] && (k & pmask) == prefix) {
        const uint64_t wq = quantize(weight_of(key_logit(k), maximum, inv_t));
        if (wq) atomicAdd((unsigned long long *)&s.hist[(k >> (8 * d)) & 255u],
                          (unsigned long long)wq);
      }
    }
    __syncthreads();
    crossing_bin(s, need);
    need -= s.sel_excl;
    prefix |= s.sel_bin << (8 * d);
    pmask |= 255u << (8 * d);
    __syncthreads();
  }
  const uint64_t wk = quantize(weight_of(key_logit(prefix), maximum, inv_t));
  const uint64_t ties_kept = (need + wk - 1) / wk;
  const ItemRange r = my_items(n);
  uint32_t ties = 0;
  for (uint32_t i = r.begin; i < r.end; ++i) ties += m.fl[i] && m.key[i] == prefix;
  uint32_t rank = (uint32_t)block_excl_scan_u64(ties, s, nullptr);
  for (uint32_t i = r.begin; i < r.end; ++i) {
    if (!m.fl[i]) continue;
    const uint32_t k = m.key[i];
    if (k > prefix) continue;
    if (k < prefix) {
      m.fl[i] = 0;
    } else {
      m.fl[i] = rank < ties_kept ? 1 : 0;
      ++rank;
    }
  }
  __syncthreads();
}

// The draw over the flagged items in id order (sampling.metal:694-829) and
// the row's outputs.
__device__ __forceinline__ void lds_draw(const SampleLaunch &a, const RowParams &rp,
                                         uint32_t row, Lds &s, uint32_t n, float maximum,
                                         float inv_t) {
  MergeLds &m = s.merge;
  const ItemRange r = my_items(n);
  uint64_t mloc = 0;
  uint32_t kloc = 0;
  for (uint32_t i = r.begin; i < r.end; ++i)
    if (m.fl[i]) {
      mloc += quantize(weight_of(key_logit(m.key[i]), maximum, inv_t));
      ++kloc;
    }
  uint64_t mass3;
  (void)block_excl_scan_u64(mloc, s, &mass3);
  uint64_t kept_total;
  const uint32_t kept_rank = (uint32_t)block_excl_scan_u64(kloc, s, &kept_total);
  const double scale = (double)mass3 * 0x1p-44;
  if (a.out_kept_ids) {
    uint32_t k = kept_rank;
    for (uint32_t i = r.begin; i < r.end; ++i) {
      if (!m.fl[i]) continue;
      if (k < a.kept_cap) {
        const float w = weight_of(key_logit(m.key[i]), maximum, inv_t);
        a.out_kept_ids[(uint64_t)row * a.kept_cap + k] = m.id[i];
        a.out_kept_probs[(uint64_t)row * a.kept_cap + k] =
            mass3 ? (float)((double)w / scale) : 0.0f;
      }
      ++k;
    }
  }
  if (mass3 == 0) {
    if (threadIdx.x == 0) write_result(a, row, kNoToken, 0.0f, (uint32_t)kept_total);
    return;
  }
  const uint32_t draft = row_draft(a, rp);
  const bool drafted = draft != kNoToken;
  uint64_t dloc = 0;
  uint32_t any = 0;
  if (drafted) {
    for (uint32_t i = r.begin; i < r.end; ++i)
      if (m.fl[i]) {
        const uint64_t wq =
            quantize(weight_of(key_logit(m.key[i]), maximum, inv_t));
        const uint64_t d = residual_of(wq, mass3, draft_q(a, rp, m.id[i], s));
        dloc += d;
        any |= d > 0;
      }
  }
  const bool residual = drafted && block_max_u32(any, s) != 0;
  if (!residual) dloc = mloc;
  uint64_t total;
  const uint64_t excl = block_excl_scan_u64(dloc, s, &total);
  uint64_t target = floor_mul(total, row_uniform(a, row));
  if (target >= total) target = total - 1;
  if (threadIdx.x == 0) {
    s.hit = kNoToken;
    s.found_w = 0.0f;
  }
  __syncthreads();
  if (excl <= target && excl + dloc > target) {
    uint64_t run = excl;
    for (uint32_t i = r.begin; i < r.end; ++i) {
      if (!m.fl[i]) continue;
      const uint64_t wq =
          quantize(weight_of(key_logit(m.key[i]), maximum, inv_t));
      run += residual ? residual_of(wq, mass3, draft_q(a, rp, m.id[i], s)) : wq;
      if (run > target) {
        s.hit = m.id[i];
        break;
      }
    }
  }
  if (drafted)
    for (uint32_t i = r.begin; i < r.end; ++i)
      if (m.fl[i] && m.id[i] == draft)
        s.found_w = weight_of(key_logit(m.key[i]), maximum, inv_t);
  __syncthreads();
  if (threadIdx.x == 0)
    write_result(a, row, s.hit,
                 drafted ? (float)((double)s.found_w / scale) : 0.0f,
                 (uint32_t)kept_total);
}

// The merge of at most kThreads items in s.merge (any order): thread t
// holds item t and counts its rank in (key desc, id asc) order, which gives
// the top-k cut and the rank-order walk of top-p; the kept items' ranks by id
// give the id-order draw.
__device__ __forceinline__ void small_merge(const SampleLaunch &a,
                                            const RowParams &rp, uint32_t row,
                                            Lds &s, uint32_t n, float maximum) {
  MergeLds &m = s.merge;
  const uint32_t t = threadIdx.x;
  const bool have = t < n;
  const uint32_t key = have ? m.key[t] : 0u;
  const uint32_t id = have ? m.id[t] : kNoToken;
  uint32_t rank = 0;
  if (have)
    for (uint32_t j = 0; j < n; ++j) {
      const uint32_t kj = m.key[j];
      rank += (kj > key) || (kj == key && m.id[j] < id);
    }
  const uint32_t n2 = min(rp.top_k, n);
  const float w = have ? weight_of(key_logit(key), maximum, rp.inv_t) : 0.0f;
  const uint64_t wq = quantize(w);
  if (have) m.bins[t] = rank;
  uint32_t n3 = n2;
  if (rp.flags & kRowTopP) {
    // Weights in rank order, their running sum, the first rank past the
    // nucleus.
    __syncthreads();
    if (have && rank < n2) s.hist[rank] = wq;
    __syncthreads();
    const uint64_t mine = t < n2 ? s.hist[t] : 0;
    uint64_t mass2;
    const uint64_t excl = block_excl_scan_u64(mine, s, &mass2);
    if (t == 0) s.hit = n2;
    __syncthreads();
    if (mass2) {
      const uint64_t nucleus = floor_mul(mass2, rp.top_p);
      if (t < n2 && excl <= nucleus && excl + mine > nucleus) s.hit = t + 1;
    }
    __syncthreads();
    n3 = s.hit;
  }
  __syncthreads();
  const bool kept = have && rank < n3;
  uint32_t irank = 0;  // rank by id among the kept items
  if (kept)
    for (uint32_t j = 0; j < n; ++j) irank += m.bins[j] < n3 && m.id[j] < id;
  uint64_t mass3;
  (void)block_excl_scan_u64(kept ? wq : 0, s, &mass3);
  const double scale = (double)mass3 * 0x1p-44;
  if (a.out_kept_ids && kept && irank < a.kept_cap) {
    a.out_kept_ids[(uint64_t)row * a.kept_cap + irank] = id;
    a.out_kept_probs[(uint64_t)row * a.kept_cap + irank] =
        mass3 ? (float)((double)w / scale) : 0.0f;
  }
  if (mass3 == 0) {
    if (t == 0) write_result(a, row, kNoToken, 0.0f, n3);
    return;
  }
  const uint32_t draft = row_draft(a, rp);
  const bool drafted = draft != kNoToken;
  uint64_t d = kept ? wq : 0;
  if (drafted) {
    const uint64_t r = kept ? residual_of(wq, mass3, draft_q(a, rp, id, s)) : 0;
    if (block_max_u32(r > 0 ? 1u : 0u, s)) d = r;
  }
  // The draw weights in id order, their running sum, the first past u.
  __syncthreads();
  if (kept) {
    s.hist[irank] = d;
    m.bins[256 + irank] = id;
  }
  if (t == 0) {
    s.found_w = 0.0f;
    s.hit = kNoToken;
  }
  __syncthreads();
  const uint64_t dp = t < n3 ? s.hist[t] : 0;
  uint64_t total;
  const uint64_t excl = block_excl_scan_u64(dp, s, &total);
  uint64_t target = floor_mul(total, row_uniform(a, row));
  if (target >= total) target = total - 1;
  if (t < n3 && excl <= target && excl + dp > target) s.hit = m.bins[256 + t];
  if (drafted && kept && id == draft) s.found_w = w;
  __syncthreads();
  if (t == 0)
    write_result(a, row, s.hit, drafted ? (float)((double)s.found_w / scale) : 0.0f,
                 n3);
}

// Makes one wave's LDS writes visible to its own later LDS reads of other
// lanes' entries: LDS runs one wave's instructions in order, so waiting for
// them to finish and keeping the compiler from moving memory operations
// across is enough.
__device__ __forceinline__ void wave_lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// The last steps of a row with at most 64 items left (s.merge.key/id[0, n),
// any order), run by one wave. Each item counts the items ahead of it in
// (key desc, id asc) order, which gives the top-k cut and the walk of top-p
// (sampling.metal:585-650); each kept item counts the kept items of lower
// id, which gives the draw's order and the kept outputs
// (sampling.metal:700-829).
__device__ __forceinline__ void wave_merge(const SampleLaunch &a,
                                           const RowParams &rp, uint32_t row,
                                           Lds &s, uint32_t n, float maximum,
                                           float u, uint32_t draft) {
  MergeLds &m = s.merge;
  uint64_t *A = s.hist;        // items as key:~id, arrival order
  uint64_t *B = s.hist + 64;   // the same in rank order
  uint64_t *D = s.hist + 128;  // draw weights in id order
  uint32_t *E = m.bins;        // kept ids in rank order
  uint32_t *F = m.bins + 128;  // kept ids in id order
  const uint32_t lane = lane_id();
  const bool have = lane < n;
  // (key desc, id asc) is the descending order of key:~id.
  const uint64_t c = have ? ((uint64_t)m.key[lane] << 32) | (uint32_t)~m.id[lane] : 0ull;
  A[lane] = c;
  wave_lds_sync();
  // Lanes at or past n hold 0, which ranks after every item.
  uint32_t rank = 0;
#pragma unroll
  for (int j = 0; j < 64; j += 2) {
    const uint64_t c0 = A[j], c1 = A[j + 1];
    rank += (c0 > c ? 1u : 0u) + (c1 > c ? 1u : 0u);
  }
  if (have) B[rank] = c;
  wave_lds_sync();
  const uint64_t cr = have ? B[lane] : 0ull;
  const uint32_t key = (uint32_t)(cr >> 32), id = ~(uint32_t)cr;
  const uint32_t n2 = min(rp.top_k, n);
  const bool in2 = lane < n2;
  const float w = in2 ? weight_of(key_logit(key), maximum, rp.inv_t) : 0.0f;
  const uint64_t wq = quantize(w);
  uint32_t n3 = n2;
  if (rp.flags & kRowTopP) {
    const uint64_t incl = wave_incl_scan_u64(wq);
    const uint64_t mass2 = readlane_u64(incl, 63);
    if (mass2) {
      const uint64_t nucleus = floor_mul(mass2, rp.top_p);
      const uint64_t hm = ballot(in2 && incl - wq <= nucleus && incl > nucleus);
      if (hm) n3 = (uint32_t)__builtin_ctzll(hm) + 1;
    }
  }
  const bool kept = lane < n3;
  const uint64_t mass3 = wave_sum_u64(kept ? wq : 0);
  // Id order of the kept items: rank among the kept ids.
  E[lane] = kept ? id : kNoToken;
  wave_lds_sync();
  uint32_t irank = 0;
#pragma unroll
  for (int q = 0; q < 64; q += 4) {
    const uint4 e4 = *(const uint4 *)&E[q];
    irank += (e4.x < id ? 1u : 0u) + (e4.y < id ? 1u : 0u) + (e4.z < id ? 1u : 0u) +
             (e4.w < id ? 1u : 0u);
  }
  const double scale = (double)mass3 * 0x1p-44;
  if (a.out_kept_ids && kept && irank < a.kept_cap) {
    a.out_kept_ids[(uint64_t)row * a.kept_cap + irank] = id;
    a.out_kept_probs[(uint64_t)row * a.kept_cap + irank] =
        mass3 ? (float)((double)w / scale) : 0.0f;
  }
  if (mass3 == 0) {
    if (lane == 0) write_result(a, row, kNoToken, 0.0f, n3);
    return;
  }
  const bool drafted = draft != kNoToken;
  uint64_t d = kept ? wq : 0;
  if (drafted) {
    const uint64_t r = kept ? residual_of(wq, mass3, draft_q(a, rp, id, s)) : 0;
    if (ballot(r > 0)) d = r;
  }
  const uint64_t fm = ballot(drafted && kept && id == draft);
  const float fw = u2f(readlane_u32(f2u(w), fm ? (int)__builtin_ctzll(fm) : 0));
  if (kept) {
    D[irank] = d;
    F[irank] = id;
  }
  wave_lds_sync();
  const uint64_t dd = kept ? D[lane] : 0ull;
  const uint64_t incl = wave_incl_scan_u64(dd);
  const uint64_t total = readlane_u64(incl, 63);
  uint64_t target = floor_mul(total, u);
  if (target >= total) target = total - 1;
  const uint64_t hm = ballot(kept && incl - dd <= target && incl > target);
  const uint32_t token = hm ? F[__builtin_ctzll(hm)] : kNoToken;
  if (lane == 0)
    write_result(a, row, token, drafted && fm ? (float)((double)fw / scale) : 0.0f, n3);
}

// The exact top-K (K <= 64) of the candidates at or above `thr` that the
// block holds in registers (v[k] = item first + k, key in the low word, id
// in the high word): a 1024-bin value histogram over [value(thr), maximum]
// finds the bin where the count from the top reaches K, and that bin's
// items are ranked exactly. The kept items (all of them when there are at
// most K) are appended to s.merge.key/id; returns their number, or -1 when
// the boundary bin holds more than kThreads items or the values do not
// spread over the bins. The caller zeroed s.merge.bins before a barrier.
template <int PER>
__device__ __forceinline__ int fast_select(const uint64_t (&v)[PER],
                                           uint32_t first, uint32_t n_all,
                                           uint32_t thr, uint32_t K,
                                           float maximum, Lds &s) {
  MergeLds &m = s.merge;
  const uint32_t tid = threadIdx.x;
  const float lo = key_logit(thr);
  const float scale = 1023.0f / (maximum - lo);
  if (!(scale > 0.0f && scale < 3.0e38f)) return -1;
  auto bin_of = [&](uint32_t key) -> uint32_t {
    return min(1023u, (uint32_t)((key_logit(key) - lo) * scale));
  };
  if (tid == 0) {
    s.u32a = 0;
    s.nbound = 0;
  }
#pragma unroll
  for (int k = 0; k < PER; ++k)
    if (first + k < n_all && (uint32_t)v[k] >= thr)
      atomicAdd(&m.bins[bin_of((uint32_t)v[k])], 1u);
  __syncthreads();
  uint32_t own = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) own += m.bins[4 * tid + k];
  uint64_t total;
  const uint32_t before = (uint32_t)block_excl_scan_u64(own, s, &total);
  const uint32_t suffix = (uint32_t)total - before;  // bins >= 4 tid
  const bool all = total <= K;
  if (!all && suffix >= K && suffix - own < K) {
    uint32_t acc = suffix - own;
    uint32_t b = 4 * tid + 3;
    for (int k = 3; k >= 0; --k) {
      b = 4 * tid + k;
      if (acc + m.bins[b] >= K) break;
      acc += m.bins[b];
    }
    s.sel_bin = b;
    s.sel_excl = acc;
  }
  __syncthreads();
  const uint32_t bstar = all ? 0u : s.sel_bin;
  const uint32_t need = all ? 0u : K - (uint32_t)s.sel_excl;
  if (!all && m.bins[bstar] > (uint32_t)kThreads) return -1;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const uint32_t key = (uint32_t)v[k];
    if (first + k >= n_all || key < thr) continue;
    const uint32_t b = bin_of(key);
    if (all || b > bstar) {
      const uint32_t slot = atomicAdd(&s.u32a, 1u);
      m.key[slot] = key;
      m.id[slot] = (uint32_t)(v[k] >> 32);
    } else if (b == bstar) {
      s.hist[atomicAdd(&s.nbound, 1u)] = v[k];
    }
  }
  __syncthreads();
  const uint32_t nb = s.nbound;
  if (tid < nb) {
    const uint64_t me = s.hist[tid];
    const uint32_t key = (uint32_t)me, id = (uint32_t)(me >> 32);
    uint32_t rank = 0;
    for (uint32_t j = 0; j < nb; ++j) {
      const uint64_t o = s.hist[j];
      const uint32_t ok = (uint32_t)o, oi = (uint32_t)(o >> 32);
      rank += ok > key || (ok == key && oi < id);
    }
    if (rank < need) {
      const uint32_t slot = atomicAdd(&s.u32a, 1u);
      m.key[slot] = key;
      m.id[slot] = id;
    }
  }
  __syncthreads();
  return (int)s.u32a;
}

// The exact top-K (K <= 64) candidates of a row held in registers (v[k] =
// key | id << 32; bit k of `valid` set for a real item at or above the
// floor): a 1024-bin
// value histogram over [value(thr), maximum] locates the bin where the
// count from the top reaches K (wave 0 finds it), and every item of that
// bin and above goes to s.merge.key/id. Returns their number (then K plus
// the boundary bin's other items, or all items when there are at most K),
// or -1 when the values do not spread over the bins. The caller zeroed
// s.merge.bins before a barrier.
template <int PER>
__device__ __forceinline__ int spec_select(const uint64_t (&v)[PER], uint32_t valid,
                                           uint32_t thr, uint32_t K, float maximum,
                                           Lds &s) {
  MergeLds &m = s.merge;
  const uint32_t tid = threadIdx.x;
  const float lo = key_logit(thr);
  const float scale = 1023.0f / (maximum - lo);
  if (!(scale > 0.0f && scale < 3.0e38f)) return -1;
  auto bin_of = [&](uint32_t key) -> uint32_t {
    return min(1023u, (uint32_t)((key_logit(key) - lo) * scale));
  };
  if (tid == 0) s.u32a = 0;
#pragma unroll
  for (int k = 0; k < PER; ++k)
    if ((valid >> k) & 1) atomicAdd(&m.bins[bin_of((uint32_t)v[k])], 1u);
  __syncthreads();
  if (tid < 64) {
    // Lane l owns bins 16 l .. 16 l + 15; the suffix count from the top.
    uint32_t own = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) own += m.bins[16 * tid + k];
    const uint32_t incl = wave_incl_scan_u32(own);
    const uint32_t total = readlane_u32(incl, 63);
    const uint32_t suffix = total - (incl - own);  // bins >= 16 l
    if (total <= K) {
      if (tid == 0) s.sel_bin = 0;
    } else if (suffix >= K && suffix - own < K) {
      uint32_t acc = suffix - own, b = 16 * tid + 15;
      for (int k = 15; k >= 0; --k) {
        b = 16 * tid + k;
        if (acc + m.bins[b] >= K) break;
        acc += m.bins[b];
      }
      s.sel_bin = b;
    }
  }
  __syncthreads();
  const uint32_t bstar = s.sel_bin;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    if (!((valid >> k) & 1)) continue;
    const uint32_t key = (uint32_t)v[k];
    if (bin_of(key) >= bstar) {
      const uint32_t slot = atomicAdd(&s.u32a, 1u);
      m.key[slot] = key;
      m.id[slot] = (uint32_t)(v[k] >> 32);
    }
  }
  __syncthreads();
  return (int)s.u32a;
}

// Sorts the n items of s.merge by id (bitonic, padded to a power of two
// with id kNoToken), so that the radix path sees them in id order.
__device__ __forceinline__ void lds_sort_by_id(Lds &s, uint32_t n) {
  MergeLds &m = s.merge;
  uint32_t P = 1;
  while (P < n) P <<= 1;
  for (uint32_t i = n + threadIdx.x; i < P; i += kThreads) {
    m.key[i] = 0;
    m.id[i] = kNoToken;
  }
  __syncthreads();
  for (uint32_t size = 2; size <= P; size <<= 1)
    for (uint32_t stride = size >> 1; stride; stride >>= 1) {
      for (uint32_t i = threadIdx.x; i < P / 2; i += kThreads) {
        const uint32_t lo = 2 * stride * (i / stride) + (i % stride);
        const uint32_t hi = lo + stride;
        const bool ascending = (lo & size) == 0;
        const uint32_t a = m.id[lo], b = m.id[hi];
        if ((a > b) == ascending) {
          m.id[lo] = b;
          m.id[hi] = a;
          const uint32_t k = m.key[lo];
          m.key[lo] = m.key[hi];
          m.key[hi] = k;
        }
      }
      __syncthreads();
    }
  for (uint32_t i = threadIdx.x; i < n; i += kThreads) m.fl[i] = 1;
  __syncthreads();
}

// Keeps the first K of the n compacted items (id order in s.merge) in
// (key desc, id asc) order, compacted in id order, when K <= kThreads: a
// 1024-bin histogram of the values between the items' least value and the
// row maximum finds the bin of the K-th item, whose few items are ranked
// exactly. Returns false, changing nothing, when the values do not spread
// over the bins (the caller then takes the radix path).
__device__ __forceinline__ bool hist_select(Lds &s, uint32_t &n, uint32_t K,
                                            float maximum) {
  MergeLds &m = s.merge;
  constexpr int PER = kMergeCapacity / kThreads;
  const uint32_t tid = threadIdx.x;
  uint32_t kmin = 0xffffffffu;
  for (uint32_t i = tid; i < n; i += kThreads) kmin = min(kmin, m.key[i]);
  kmin = block_min_u32(kmin, s);
  const float lo = key_logit(kmin);
  const float scale = 1023.0f / (maximum - lo);
  if (!(scale > 0.0f && scale < 3.0e38f) || kmin <= kLowestKey) return false;
  for (uint32_t b = tid; b < 1024; b += kThreads) m.bins[b] = 0;
  if (tid == 0) s.u32a = 0;
  __syncthreads();
  auto bin_of = [&](uint32_t key) -> uint32_t {
    const float v = (key_logit(key) - lo) * scale;
    return min(1023u, (uint32_t)v);
  };
  for (uint32_t i = tid; i < n; i += kThreads) atomicAdd(&m.bins[bin_of(m.key[i])], 1u);
  __syncthreads();
  // The highest bin whose suffix count reaches K.
  uint32_t own = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) own += m.bins[4 * tid + k];
  uint64_t total;
  const uint32_t before = (uint32_t)block_excl_scan_u64(own, s, &total);
  const uint32_t suffix = (uint32_t)total - before;  // bins >= 4 tid
  if (suffix >= K && suffix - own < K) {
    uint32_t acc = suffix - own;
    uint32_t b = 4 * tid + 3;
    for (int k = 3; k >= 0; --k) {
      b = 4 * tid + k;
      if (acc + m.bins[b] >= K) break;
      acc += m.bins[b];
    }
    s.sel_bin = b;
    s.sel_excl = acc;
  }
  __syncthreads();
  const uint32_t bstar = s.sel_bin;
  const uint32_t need = K - (uint32_t)s.sel_excl;
  if (m.bins[bstar] > (uint32_t)kThreads) return false;
  // The items of the boundary bin, ranked exactly.
  for (uint32_t i = tid; i < n; i += kThreads) {
    const uint32_t b = bin_of(m.key[i]);
    m.fl[i] = b > bstar ? 1 : 0;
    if (b == bstar) {
      const uint32_t slot = atomicAdd(&s.u32a, 1u);
      s.hist[slot] = ((uint64_t)m.key[i] << 32) | i;
    }
  }
  __syncthreads();
  const uint32_t nb = s.u32a;
  if (tid < nb) {
    const uint64_t me = s.hist[tid];
    const uint32_t key = (uint32_t)(me >> 32), pos = (uint32_t)me;
    uint32_t rank = 0;
    for (uint32_t j = 0; j < nb; ++j) {
      const uint64_t o = s.hist[j];
      const uint32_t ok = (uint32_t)(o >> 32), op = (uint32_t)o;
      rank += ok > key || (ok == key && m.id[op] < m.id[pos]);
    }
    if (rank < need) m.fl[pos] = 1;
  }
  __syncthreads();
  // Ordered compaction of the kept items.
  uint32_t kk[PER], ki[PER];
  uint32_t cnt = 0;
  const uint32_t first = tid * PER;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const uint32_t i = first + k;
    const bool keep = i < n && m.fl[i];
    kk[k] = keep ? m.key[i] : 0u;
    ki[k] = keep ? m.id[i] : kNoToken;
    cnt += keep;
  }
  uint64_t kept;
  uint32_t out = (uint32_t)block_excl_scan_u64(cnt, s, &kept);
#pragma unroll
  for (int k = 0; k < PER; ++k)
    if (ki[k] != kNoToken) {
      m.key[out] = kk[k];
      m.id[out] = ki[k];
      m.fl[out] = 1;
      ++out;
    }
  n = (uint32_t)kept;
  __syncthreads();
  return true;
}

// A chunk whose candidates overflowed its list, selected again by the
// merge with the row's threshold `thr`: its tokens at or above it or, when
// more than the list holds, its first K (K <= kBlockCandidates) in (key
// desc, id asc) order -- a bisection over keys to a cut that leaves
// K..kBlockCandidates tokens, else the K-th key itself with the lowest ids
// among its ties. The row's first K lie among the chunks' first K, so this
// loses nothing. Rewrites the chunk's list and returns its length. Every
// thread calls it; it clobbers s.prep (and so s.merge).
template <int DT>
__device__ __forceinline__ uint32_t reselect_chunk(const SampleLaunch &a,
                                                   const RowParams &rp,
                                                   uint32_t row, uint32_t chunk,
                                                   uint32_t thr, uint32_t K,
                                                   Lds &s) {
  constexpr int VEC = Geo<DT>::VEC, TPL = Geo<DT>::TPL, SLAB = Geo<DT>::SLAB;
  constexpr uint32_t CHUNK = Geo<DT>::CHUNK;
  const uint32_t tid = threadIdx.x;
  float xs[TPL];
  load_chunk<DT>(a, rp, row, chunk, s, xs);
  const uint32_t lane_base = chunk * CHUNK + tid * VEC;
  uint64_t *dst = a.cands + ((uint64_t)row * a.chunks + chunk) * kBlockCandidates;
  const float tv = thr <= kLowestKey ? -__builtin_inff() : key_logit(thr);
  float bm = -__builtin_inff();
  uint32_t cnt = 0;
#pragma unroll
  for (int i = 0; i < TPL; ++i) {
    cnt += xs[i] >= tv;
    bm = __builtin_fmaxf(bm, xs[i]);
  }
  cnt = block_sum_u32(cnt, s);
  const float bmax = __builtin_fmaxf(block_max_f32(bm, s), -3.402823466e38f);
  uint64_t keep = 0;
  if (cnt <= (uint32_t)kBlockCandidates) {
#pragma unroll
    for (int i = 0; i < TPL; ++i) keep |= (uint64_t)(xs[i] >= tv) << i;
  } else {
    // Invariant: at least K tokens at or above lo, fewer than K at or
    // above hi.
    uint32_t lo_k = thr, hi_k = logit_key(bmax) + 1;
    uint32_t found = 0;
    while (hi_k - lo_k > 1) {
      const uint32_t mid = lo_k + (hi_k - lo_k) / 2;
      const float mv = mid <= kLowestKey ? -__builtin_inff() : key_logit(mid);
      opaque(xs);
      uint32_t cm = 0;
#pragma unroll
      for (int i = 0; i < TPL; ++i) cm += xs[i] >= mv;
      cm = block_sum_u32(cm, s);
      if (cm < K) {
        hi_k = mid;
      } else if (cm <= (uint32_t)kBlockCandidates) {
        found = mid;
        break;
      } else {
        lo_k = mid;
      }
    }
    const uint32_t cut = found ? found : lo_k;
    const float cv = cut <= kLowestKey ? -__builtin_inff() : key_logit(cut);
    opaque(xs);
    uint64_t ge = 0, eq = 0;
#pragma unroll
    for (int i = 0; i < TPL; ++i) {
      ge |= (uint64_t)(xs[i] >= cv) << i;
      eq |= (uint64_t)(xs[i] == cv) << i;
    }
    keep = ge;
    if (!found) {
      // The K-th key itself: of the tokens tied there, the `need` lowest
      // ids stay. L = the largest chunk offset with fewer than `need` ties
      // below it (binary descent); offsets are distinct, so exactly `need`
      // ties lie at offsets <= L. Offset of xs[i] = (i / VEC) * SLAB +
      // (i % VEC) + tid * VEC.
      const uint32_t need = K - block_sum_u32(__popcll(ge & ~eq), s);
      const int toff = (int)(tid * VEC);
      uint32_t L = 0;
#pragma unroll 1
      for (uint32_t bit = CHUNK / 2; bit; bit >>= 1) {
        const int t = (int)(L + bit) - toff;
        uint32_t c = 0;
#pragma unroll
        for (int i = 0; i < TPL; ++i)
          c += ((eq >> i) & 1) && (i / VEC) * SLAB + (i % VEC) < t;
        if (block_sum_u32(c, s) < need) L += bit;
      }
      const int lim = (int)L - toff;
      uint64_t tie_keep = 0;
#pragma unroll
      for (int i = 0; i < TPL; ++i)
        tie_keep |= (uint64_t)(((eq >> i) & 1) && (i / VEC) * SLAB + (i % VEC) <= lim) << i;
      keep = (ge & ~eq) | tie_keep;
    }
  }
  __syncthreads();
  if (tid == 0) s.u32a = 0;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < TPL; ++i)
    if ((keep >> i) & 1) {
      const uint32_t slot = atomicAdd(&s.u32a, 1u);
      dst[slot] = (uint64_t)logit_key(xs[i]) |
                  ((uint64_t)(lane_base + (i / VEC) * SLAB + (i % VEC)) << 32);
    }
  __syncthreads();
  const uint32_t n = s.u32a;
  __syncthreads();
  return n;
}

// Starts the multi-pass stages of a row the merge cannot finish.
__device__ __forceinline__ void begin_stages(const SampleLaunch &a, const RowParams &rp,
                             uint32_t row, float maximum) {
  RowState st = {};
  st.maximum = maximum;
  st.bkey = 0;
  st.bid = 0;
  // The members' count decides whether top-k cuts; a row with neither
  // min-p nor top-k keeps every admitted token.
  if (rp.flags & (kRowMinP | kRowTopK)) {
    st.thr_key = (rp.flags & kRowMinP)
                     ? logit_key(__builtin_fminf(maximum + rp.minp_offset, maximum))
                     : 0u;
    st.stage = kStageCount1;
  } else {
    st.thr_key = 0;
    st.stage = (rp.flags & kRowTopP) ? kStageMass2 : kStageMass3;
  }
  st.drafted = row_draft(a, rp) != kNoToken ? 1u : 0u;
  a.states[row] = st;
}

template <int DT>
__device__ __forceinline__ void merge_sampled(const SampleLaunch &a, const RowParams &rp,
                              uint32_t row, Lds &s) {
  const uint32_t S = a.chunks, tid = threadIdx.x;
  const BlockHeader *hb = a.headers + (uint64_t)row * S;
  // Everything the row needs from memory is requested up front: the chunk
  // summaries (one lane each, S <= 64), the uniform, the draft token and its
  // sparse candidates. The select kernel's writes are visible here because
  // it ended before this launch began.
  const float u = row_uniform(a, row);
  const uint32_t draft = row_draft(a, rp);
  // Rows with a small top-k also fetch the first P slots of every chunk's
  // candidate list now, before the counts are known (S * P <= SPEC items).
  constexpr int SPEC = 10;
  const uint32_t K = rp.top_k;
  const uint32_t P = S <= 20 ? 128u : (S <= 40 ? 64u : 32u);
  const uint32_t pshift = S <= 20 ? 7u : (S <= 40 ? 6u : 5u);
  const bool spec = (rp.flags & kRowTopK) && K <= 64u;
  uint64_t sv[SPEC];
#pragma unroll
  for (int k = 0; k < SPEC; ++k) {
    const uint32_t i = tid + k * kThreads, c = i >> pshift;
    sv[k] = 0;
    if (spec && c < S)
      sv[k] = a.cands[((uint64_t)row * S + c) * kBlockCandidates + (i & (P - 1))];
  }
  for (uint32_t b = tid; b < 1024; b += kThreads) s.merge.bins[b] = 0;
  if (tid < 16) {
    const bool sparse = !a.dense_q && draft != kNoToken;
    s.cids[tid] = sparse ? a.cand_ids[(uint64_t)rp.cand_index * 16 + tid] : kNoToken;
    s.cprobs[tid] = sparse ? a.cand_probs[(uint64_t)rp.cand_index * 16 + tid] : 0.0f;
  }
  if (tid < 64) {
    float hm = -3.402823466e38f;
    uint32_t hc = 0, ha = 0, ho = 0, hf = 0;
    if (tid < S) {
      const BlockHeader h = hb[tid];
      hm = h.maximum;
      hc = h.count;
      ha = h.admitted;
      ho = h.overflow;
      hf = h.floor_key;
    }
    const float mx = wave_max_f32(hm);
    const uint32_t adm = wave_sum_u32(ha), ovf = wave_max_u32(ho),
                   flr = wave_max_u32(hf), hcmax = wave_max_u32(hc);
    const uint32_t incl = wave_incl_scan_u32(hc);
    const uint64_t omask = ballot(ho != 0);
    if (tid < S) {
      s.hoff[tid + 1] = incl;
      s.hcnt[tid] = hc;
      s.hmax[tid] = hm;
    }
    if (tid == 0) {
      s.u64a = omask;
      s.hoff[0] = 0;
      s.row_max = mx;
      s.row_admitted = adm;
      s.row_overflow = ovf;
      s.row_floor = flr;
      s.row_maxcount = hcmax;
    }
  }
  __syncthreads();
  const float maximum = s.row_max;
  const uint32_t admitted = s.row_admitted, overflow = s.row_overflow;
  // The K-th key of the row is at least every block's floor.
  const uint32_t floor_key = s.row_floor;
  if (admitted == 0 || maximum == __builtin_inff()) {
    if (tid == 0) {
      write_result(a, row, kNoToken, 0.0f, 0);
      a.states[row].stage = kStageDone;
    }
    return;
  }
  uint32_t thr = (rp.flags & kRowMinP)
                     ? logit_key(__builtin_fminf(maximum + rp.minp_offset, maximum))
                     : 0u;
  if (rp.flags & kRowTopK) thr = max(thr, floor_key);
  if (overflow && K <= (uint32_t)kBlockCandidates) {
    // Chunks with more candidates than their lists hold (rare: flat or
    // tied values): select each again, then recount.
    uint64_t om = s.u64a;
    while (om) {
      const uint32_t c = (uint32_t)__builtin_ctzll(om);
      om &= om - 1;
      const uint32_t n = reselect_chunk<DT>(a, rp, row, c, thr, K, s);
      if (tid == 0) s.hcnt[c] = n;
    }
    __syncthreads();
    if (tid < 64) {
      const uint32_t incl = wave_incl_scan_u32(tid < S ? s.hcnt[tid] : 0u);
      if (tid < S) s.hoff[tid + 1] = incl;
    }
    for (uint32_t b = tid; b < 1024; b += kThreads) s.merge.bins[b] = 0;
    __syncthreads();
  }
  // A chunk whose maximum is below the threshold holds no item at or above
  // it: the offsets skip its list (every use below wants only such items).
  if (thr > kLowestKey) {
    if (tid < 64) {
      const bool use = tid < S && logit_key(s.hmax[tid]) >= thr;
      const uint32_t incl = wave_incl_scan_u32(use ? s.hcnt[tid] : 0u);
      if (tid < S) s.hoff[tid + 1] = incl;
    }
    __syncthreads();
  }
  const uint32_t n_all = s.hoff[S];
  const bool fits = n_all <= (uint32_t)kMergeCapacity;
  if ((overflow && K > (uint32_t)kBlockCandidates) ||
      (!fits && K > (uint32_t)kMergeCapacity)) {
    if (tid == 0) begin_stages(a, rp, row, maximum);
    return;
  }
  if (tid == 0) a.states[row].stage = kStageDone;
  MergeLds &m = s.merge;
  uint32_t n;
  if (spec && !overflow && s.row_maxcount <= P && thr > kLowestKey) {
    // Every list fits in the slots fetched up front: the items at or above
    // the floor, selected straight from registers.
    uint32_t valid = 0;
#pragma unroll
    for (int k = 0; k < SPEC; ++k) {
      const uint32_t i = tid + k * kThreads, c = i >> pshift;
      if (c < S && (i & (P - 1)) < s.hcnt[c] && (uint32_t)sv[k] >= thr) valid |= 1u << k;
    }
    const int got = spec_select(sv, valid, thr, K, maximum, s);
    if (got >= 0) {
      // At most K items and the boundary bin's: usually 64 or fewer.
      n = (uint32_t)got;
      if (n > 64u && !hist_select(s, n, K, maximum)) {
        lds_sort_by_id(s, n);
        lds_topk(s, n, K);
        if (rp.flags & kRowTopP) lds_topp(s, n, maximum, rp.inv_t, rp.top_p);
        lds_draw(a, rp, row, s, n, maximum, rp.inv_t);
        return;
      }
      if (tid < 64) wave_merge(a, rp, row, s, n, maximum, u, draft);
      return;
    }
  }
  if (fits) {
    // Candidates at or above the floor into LDS: every load issued first,
    // contiguous items per thread, then a compaction.
    constexpr int PER = kMergeCapacity / kThreads;
    uint64_t v[PER];
    const uint32_t first = tid * PER;
    uint32_t c = 0;
    for (uint32_t step = kMaxChunks / 2; step; step >>= 1)
      if (c + step < S && s.hoff[c + step] <= first) c += step;
    uint32_t cnt = 0;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const uint32_t i = first + k;
      v[k] = 0;
      if (i < n_all) {
        while (s.hoff[c + 1] <= i) ++c;
        v[k] = a.cands[((uint64_t)row * S + c) * kBlockCandidates + (i - s.hoff[c])];
      }
    }
    if (K <= 64u && thr > kLowestKey) {
      const int kept = fast_select(v, first, n_all, thr, K, maximum, s);
      if (kept >= 0) {
        if (tid < 64) wave_merge(a, rp, row, s, (uint32_t)kept, maximum, u, draft);
        return;
      }
    }
#pragma unroll
    for (int k = 0; k < PER; ++k)
      cnt += (first + k < n_all) && (uint32_t)v[k] >= thr;
    uint64_t total;
    uint32_t out = (uint32_t)block_excl_scan_u64(cnt, s, &total);
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (first + k < n_all && (uint32_t)v[k] >= thr) {
        m.key[out] = (uint32_t)v[k];
        m.id[out] = (uint32_t)(v[k] >> 32);
        m.fl[out] = 1;
        ++out;
      }
    n = (uint32_t)total;
    __syncthreads();
  } else {
    // More candidates than LDS holds (K fits): select the first K at or
    // above the floor straight from the lists (keys by radix descent, then
    // the lowest ids among the ties), then append them to LDS.
    auto item = [&](uint32_t i) -> uint64_t {
      uint32_t c = 0;
      for (uint32_t step = kMaxChunks / 2; step; step >>= 1)
        if (c + step < S && s.hoff[c + step] <= i) c += step;
      return a.cands[((uint64_t)row * S + c) * kBlockCandidates + (i - s.hoff[c])];
    };
    uint32_t c1 = 0;
    for (uint32_t i = tid; i < n_all; i += kThreads) c1 += (uint32_t)item(i) >= thr;
    const uint32_t n1 = block_sum_u32(c1, s);
    uint32_t kap = 0, iota = kNoToken;  // keep key > kap, or key == kap and id <= iota
    if (K < n1) {
      uint32_t prefix = 0, pmask = 0;
      uint64_t need = K;
      for (int d = 3; d >= 0; --d) {
        s.hist[tid] = 0;
        __syncthreads();
        for (uint32_t i = tid; i < n_all; i += kThreads) {
          const uint32_t k = (uint32_t)item(i);
          if (k >= thr && (k & pmask) == prefix)
            atomicAdd((unsigned long long *)&s.hist[(k >> (8 * d)) & 255u], 1ull);
        }
        __syncthreads();
        crossing_bin(s, need);
        need -= s.sel_excl;
        prefix |= s.sel_bin << (8 * d);
        pmask |= 255u << (8 * d);
        __syncthreads();
      }
      kap = prefix;
      // The need-th smallest id among the ties: the need-th largest of
      // 0xffffff - id, by descent over its three bytes.
      uint32_t ip = 0, im = 0;
      for (int d = 2; d >= 0; --d) {
        s.hist[tid] = 0;
        __syncthreads();
        for (uint32_t i = tid; i < n_all; i += kThreads) {
          const uint64_t v = item(i);
          if ((uint32_t)v != kap) continue;
          const uint32_t ri = 0xffffffu - (uint32_t)(v >> 32);
          if ((ri & im) == ip)
            atomicAdd((unsigned long long *)&s.hist[(ri >> (8 * d)) & 255u], 1ull);
        }
        __syncthreads();
        crossing_bin(s, need);
        need -= s.sel_excl;
        ip |= s.sel_bin << (8 * d);
        im |= 255u << (8 * d);
        __syncthreads();
      }
      iota = 0xffffffu - ip;
    }
    if (tid == 0) s.u32a = 0;
    __syncthreads();
    for (uint32_t i = tid; i < n_all; i += kThreads) {
      const uint64_t v = item(i);
      const uint32_t k = (uint32_t)v, id = (uint32_t)(v >> 32);
      if (k < thr) continue;
      if (k > kap || (k == kap && id <= iota)) {
        const uint32_t slot = atomicAdd(&s.u32a, 1u);
        m.key[slot] = k;
        m.id[slot] = id;
        m.fl[slot] = 1;
      }
    }
    __syncthreads();
    n = s.u32a;
    __syncthreads();
  }
  if (K <= 64u && K < n && hist_select(s, n, K, maximum)) {
    if (tid < 64) wave_merge(a, rp, row, s, n, maximum, u, draft);
    return;
  }
  if (n <= 64u) {
    if (tid < 64) wave_merge(a, rp, row, s, n, maximum, u, draft);
    return;
  }
  if (n <= (uint32_t)kThreads) {
    small_merge(a, rp, row, s, n, maximum);
    return;
  }
  if (K <= (uint32_t)kThreads && hist_select(s, n, K, maximum)) {
    small_merge(a, rp, row, s, n, maximum);
    return;
  }
  lds_sort_by_id(s, n);
  if (K < n) lds_topk(s, n, K);
  if (rp.flags & kRowTopP) lds_topp(s, n, maximum, rp.inv_t, rp.top_p);
  lds_draw(a, rp, row, s, n, maximum, rp.inv_t);
}

// Every thread's device-coherent stores complete, then one arrival; true in
// every thread of the block that arrives last, which returns the counter to
// zero for the next launch.
template <class L>
__device__ __forceinline__ bool arrive_last(uint32_t *counter, uint32_t S,
                                            L &s) {
  wait_memory();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    s.last = prev == S - 1;
    if (s.last) st_dev(counter, 0u);
  }
  __syncthreads();
  return s.last != 0;
}

template <int DT>
__device__ __forceinline__ void merge_row(const SampleLaunch &a,
                                          const RowParams &rp, uint32_t row,
                                          Lds &s) {
  const uint32_t S = a.chunks, tid = threadIdx.x;
  if (uncut_row(rp)) {
    // The uncut kernel draws it; no stage may pick it up.
    if (tid == 0) a.states[row].stage = kStageDone;
    return;
  }
  if (!(rp.flags & kRowSampled)) {
    if (tid < 64) {
      float bv = -__builtin_inff();
      uint32_t bi = kNoToken;
      for (uint32_t c = tid; c < S; c += 64) {
        const BlockHeader *h = a.headers + (uint64_t)row * S + c;
        const float hv = ld_dev(&h->best_value);
        const uint32_t hi = ld_dev(&h->best_id);
        if (hv > bv || (hv == bv && hi < bi)) {
          bv = hv;
          bi = hi;
        }
      }
      wave_argmax(bv, bi);
      if (tid == 0) {
        write_result(a, row, bi, 0.0f, 0);
        a.states[row].stage = kStageDone;
      }
    }
    return;
  }
  merge_sampled<DT>(a, rp, row, s);
}

// ---- the single-pass selection kernel -------------------------------------

#if JF_IN(1)
// A row that keeps every admitted token: its chunk's exact fixed-point mass
// against the chunk's own maximum `bmax` (every value of the chunk is at most
// that maximum), per slice into s.slices[g] (slice g = load g / kWaves of
// wave g % kWaves, 64 x VEC consecutive tokens), and its admitted (non-NaN)
// count per wave into s.wcount. `side` holds the penalized tokens whose own
// registers are dropped (NaN), so every token counts once; their weights join
// their slices through LDS. s.slices is zero on entry (cleared before the
// block's last barrier). Ends with a barrier. Block-uniform. With `wout`
// (fp32 rows, no penalized token: a drafted row's residual pass reads them),
// every token's weight is also stored there as pack_yk, at its offset in
// the chunk.
template <int DT, class L>
__device__ __forceinline__ void uncut_slices(const float (&xs)[Geo<DT>::TPL],
                                             const SideEntries &side, uint32_t base,
                                             float bmax, float inv_t, L &s,
                                             uint32_t *wout = nullptr) {
  constexpr int VEC = Geo<DT>::VEC, LOADS = Geo<DT>::LOADS, SLAB = Geo<DT>::SLAB;
  static_assert(LOADS % 4 == 0, "loads in groups of four");
  const uint32_t tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  uint32_t n = 0;
  // Four loads at a time (fewer live registers than all of them at once).
#pragma unroll
  for (int h = 0; h < LOADS / 4; ++h) {
    uint64_t lv[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      lv[jj] = 0;
      uint32_t pk[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float x = xs[(h * 4 + jj) * VEC + e];
        const WeightYK wy = weight_yk(x, bmax, inv_t);
        lv[jj] += ((uint64_t)wy.Y << 32) >> wy.k;
        pk[e] = pack_yk(wy);
        n += x == x;
      }
      if constexpr (VEC == 4) {
        if (wout) {
          u32x4 v;
          v.x = pk[0];
          v.y = pk[1];
          v.z = pk[2];
          v.w = pk[3];
          *(u32x4 *)(wout + (h * 4 + jj) * SLAB + tid * VEC) = v;
        }
      }
    }
    // Lane l holds the wave's sum of load h * 4 + l / 16.
    const uint64_t sl = wave_sums_u64<4>(lv);
    if (lane % 16 == 0)
      atomicAdd((unsigned long long *)&s.slices[(h * 4 + lane / 16) * kWaves + w],
                (unsigned long long)sl);
  }
#pragma unroll
  for (int k = 0; k < kSideEntries; ++k) {
    const float x = side.val[k];
    n += x == x;
    if (side.tok[k] != kNoToken) {
      const uint32_t o = side.tok[k] - base;
      const uint32_t g = (o / SLAB) * kWaves + (o % SLAB) / VEC / 64;
      atomicAdd((unsigned long long *)&s.slices[g],
                (unsigned long long)quantized_weight(x, bmax, inv_t));
    }
  }
  n = wave_sum_u32(n);
  if (lane == 0) s.wcount[w] = n;
  __syncthreads();
}

// The chunk's summary for the uncut kernel instead of candidates: its
// maximum, whether it admits a token, its admitted count, and its slice
// masses (partial slots v[1 + g]) and total (v[0]) from uncut_slices.
template <int DT, class L>
__device__ __forceinline__ void uncut_summary(const float (&xs)[Geo<DT>::TPL],
                                              const SideEntries &side, uint32_t base,
                                              float bmax, uint32_t badm, float inv_t, L &s,
                                              BlockHeader *hdr, StagePartial *part,
                                              uint32_t *wout = nullptr) {
  constexpr uint32_t G = Geo<DT>::LOADS * kWaves;
  const uint32_t tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  uncut_slices<DT>(xs, side, base, bmax, inv_t, s, wout);
  if (w == 0) {
    const uint64_t v = lane < G ? s.slices[lane] : 0ull;
    if (lane < G) part->v[1 + lane] = v;
    const uint64_t total = wave_sum_u64(v);
    if (lane == 0) {
      hdr->maximum = bmax;
      hdr->admitted = badm;
      hdr->count = s.wcount[0] + s.wcount[1] + s.wcount[2] + s.wcount[3];
      hdr->overflow = 0;
      part->v[0] = total;
    }
  }
}

template <int DT>
__global__ __launch_bounds__(kThreads) void select_kernel(SampleLaunch a) {
  constexpr int VEC = Geo<DT>::VEC, TPL = Geo<DT>::TPL, SLAB = Geo<DT>::SLAB,
                LOADS = Geo<DT>::LOADS;
  constexpr uint32_t CHUNK = Geo<DT>::CHUNK;
  __shared__ SelectLds s;
  const uint32_t S = a.chunks;
  const uint32_t row = blockIdx.x / S, chunk = blockIdx.x % S;
  const uint32_t tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const RowParams rp = a.params[row];
  if (rp.fast_row) return;  // select_fast_kernel's row in a split launch
  float xs[TPL];
  SideEntries side;
  load_chunk<DT, true>(a, rp, row, chunk, s, xs, &side);
  const uint32_t lane_base = chunk * CHUNK + tid * VEC;
  BlockHeader *hdr = a.headers + (uint64_t)row * S + chunk;

  if (!(rp.flags & kRowSampled)) {
    // Largest value, lowest id among equals; NaN never wins and a -inf
    // token wins only over nothing (sampling.metal:1427-1464). A lane's
    // tokens ascend, so the first of equal values stays.
    float best = -__builtin_inff();
    uint32_t bid = kNoToken;
#pragma unroll
    for (int i = 0; i < TPL; ++i) {
      const float v = xs[i];
      const bool take = v > best || (v == best && bid == kNoToken);
      best = take ? v : best;
      bid = take ? lane_base + (i / VEC) * SLAB + (i % VEC) : bid;
    }
    // This thread's penalized tokens (held apart, any id order).
#pragma unroll
    for (int k = 0; k < kSideEntries; ++k) {
      const float v = side.val[k];
      const uint32_t t = side.tok[k];
      const bool take = v > best || (v == best && (bid == kNoToken || t < bid));
      best = take ? v : best;
      bid = take ? t : bid;
    }
    wave_argmax(best, bid);
    if (lane == 0) {
      s.wf[w] = best;
      s.wu[w] = bid;
    }
    __syncthreads();
    if (tid == 0) {
      float bv = s.wf[0];
      uint32_t bi = s.wu[0];
      for (int k = 1; k < kWaves; ++k)
        if (s.wf[k] > bv || (s.wf[k] == bv && s.wu[k] < bi)) {
          bv = s.wf[k];
          bi = s.wu[k];
        }
      hdr->best_value = bv;
      hdr->best_id = bi;
    }
  } else {
    // The lane's largest admitted (non-NaN) value: fmax skips NaN operands,
    // so the NaN it starts from survives only when the lane admits nothing.
    float mx = __builtin_nanf("");
#pragma unroll
    for (int i = 0; i < TPL; ++i) mx = __builtin_fmaxf(mx, xs[i]);
#pragma unroll
    for (int k = 0; k < kSideEntries; ++k) mx = __builtin_fmaxf(mx, side.val[k]);
    const bool any = mx == mx;
    // A bound for the block's top-k: each wave's ceil(k/4)-th largest lane
    // maximum has that many of the wave's tokens at or above it, so the
    // block has at least k tokens at or above the least of the four.
    const uint32_t K = rp.top_k;
    const uint32_t kw = (K + kWaves - 1) / kWaves;
    const bool bound = (rp.flags & kRowTopK) && kw <= 64;
    uint32_t wth = 0;
    if (bound) wth = wave_kth_largest(any ? logit_key(mx) : 0u, kw);
    const float wmax = wave_max_f32(mx);
    const uint32_t wany = ballot(any) != 0 ? 1u : 0u;
    if (lane == 0) {
      s.wf[w] = wmax;
      s.wu[w] = wany;
      s.wu2[w] = wth;
    }
    if (uncut_row(rp) && tid < kWaves * 8) s.slices[tid] = 0;
    __syncthreads();
    const float bmax = __builtin_fmaxf(
        __builtin_fmaxf(__builtin_fmaxf(s.wf[0], s.wf[1]),
                        __builtin_fmaxf(s.wf[2], s.wf[3])),
        -3.402823466e38f);
    const uint32_t badm = s.wu[0] | s.wu[1] | s.wu[2] | s.wu[3];
    if (uncut_row(rp)) {
      uncut_summary<DT>(xs, side, chunk * CHUNK, bmax, badm, rp.inv_t, s, hdr,
                        a.partials + (uint64_t)row * S + chunk);
      return;
    }
    const uint32_t tk =
        bound ? min(min(s.wu2[0], s.wu2[1]), min(s.wu2[2], s.wu2[3])) : 0u;
    uint32_t thr = tk;
    if (rp.flags & kRowMinP)
      thr = max(thr, logit_key(__builtin_fminf(bmax + rp.minp_offset, bmax)));
    // Candidates: each wave appends its hits (raw value, id) to its own
    // LDS list, at slots counted in scalar registers from the ballots;
    // then the block writes the lists to the chunk's list in HBM with
    // their keys. The merge is independent of the order of the list.
    const float tv = thr <= kLowestKey ? -__builtin_inff() : key_logit(thr);
    uint64_t *stage = s.stage[w];
    uint32_t run = 0;
    auto emit = [&](float x, uint32_t token) {
      const bool hit = x >= tv;
      const uint64_t m = ballot(hit);
      if (m) {
        const uint32_t slot = run + mbcnt(m);
        if (hit && slot < kWaveCandidates)
          stage[slot] = (uint64_t)f2u(x) | ((uint64_t)token << 32);
        run += (uint32_t)__popcll(m);
      }
    };
#pragma unroll
    for (int j = 0; j < LOADS; ++j)
#pragma unroll
      for (int e = 0; e < VEC; ++e) emit(xs[j * VEC + e], lane_base + j * SLAB + e);
#pragma unroll
    for (int k = 0; k < kSideEntries; ++k) emit(side.val[k], side.tok[k]);
    if (lane == 0) s.wcount[w] = run;
    __syncthreads();
    uint32_t off[kWaves + 1], over = 0;
    off[0] = 0;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) {
      const uint32_t n = s.wcount[k];
      over |= n > kWaveCandidates;
      off[k + 1] = off[k] + min(n, kWaveCandidates);
    }
    uint64_t *dst = a.cands + ((uint64_t)row * S + chunk) * kBlockCandidates;
    if (!over)
      for (uint32_t i = tid; i < off[kWaves]; i += kThreads) {
        const uint32_t k = (i >= off[1]) + (i >= off[2]) + (i >= off[3]);
        const uint64_t e = s.stage[k][i - off[k]];
        dst[i] = (uint64_t)logit_key(u2f((uint32_t)e)) | (e & 0xffffffff00000000ull);
      }
    const uint32_t c = over ? kBlockCandidates + 1 : off[kWaves];
    if (tid == 0) {
      // More candidates than the list holds: the merge selects this chunk
      // again (with the row's own thresholds) or hands the row to the
      // multi-pass stages.
      hdr->maximum = bmax;
      hdr->count = min(c, (uint32_t)kBlockCandidates);
      hdr->admitted = badm;
      hdr->overflow = c > (uint32_t)kBlockCandidates ? 1u : 0u;
      hdr->floor_key = tk;
    }
  }
}
#endif

// Inside one wave's slice of a chunk (64 lanes x VEC consecutive tokens,
// lane-major): q[e] are the lane's weights in id order and the slice's
// weights sum past `within`. Returns the lane whose running sum first passes
// it, and in that lane the index of the first token that does (the walk of
// sampling.metal:790-829 restricted to the slice).
template <int VEC>
__device__ __forceinline__ uint32_t slice_hit(const uint64_t (&q)[VEC], uint64_t within,
                                              uint32_t &e_hit) {
  uint64_t lsum = 0;
#pragma unroll
  for (int e = 0; e < VEC; ++e) lsum += q[e];
  const uint64_t incl = wave_incl_scan_u64(lsum);
  const uint32_t hl = (uint32_t)__builtin_ctzll(ballot(incl > within));
  uint64_t run = incl - lsum;
  e_hit = VEC;
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    if (e_hit == (uint32_t)VEC && q[e] && run + q[e] > within) e_hit = (uint32_t)e;
    run += q[e];
  }
  return hl;
}

// The slice g that holds `within`, given lane l's slice sum vg (lanes at or
// past G hold 0), and `within` made relative to it; wave-wide, every lane
// gets both.
__device__ __forceinline__ uint32_t pick_slice(uint64_t vg, uint32_t G, uint64_t &within) {
  const uint32_t l = lane_id();
  const bool gin = l < G;
  const uint64_t ginc = wave_incl_scan_u64(vg);
  // The slices of chunk c sum to its mass, which passes `within`.
  const uint32_t g = (uint32_t)__builtin_ctzll(ballot(gin && ginc > within));
  within -= readlane_u64(ginc - vg, g);
  return g;
}

// One wave draws inside slice g of chunk c (load g / kWaves of wave
// g % kWaves: 64 x VEC consecutive tokens): the slice's logits reloaded,
// stop tokens and (constrained rows) masked ones dropped, and the token
// whose running weight first passes `within` written with `pd` and `kept`.
// RESID 0: the plain weights quantized_weight(x, mc) (uncut_draw's walk);
// 1: the residual weights residual_of(floor(w r_c), W, q) against the
// draft's dense q row; 2: against its sparse candidates in s.cids/s.cprobs.
// `q_row`: the draft's row of q (RESID 1) or its candidates' (RESID 2).
template <int DT, int RESID, class L>
__device__ __forceinline__ void draw_in_slice(const SampleLaunch &a, uint32_t row, uint32_t flags,
                                              float inv_t, uint32_t q_row, uint32_t c, uint32_t g,
                                              uint64_t within, float mc, uint64_t Rc,
                                              uint64_t W, float pd, uint32_t kept, const L &s) {
  constexpr int VEC = Geo<DT>::VEC, SLAB = Geo<DT>::SLAB;
  constexpr uint32_t CHUNK = Geo<DT>::CHUNK;
  const uint32_t lane = lane_id(), V = a.vocabulary;
  const uint32_t t0 = c * CHUNK + (g / kWaves) * SLAB + ((g % kWaves) * 64 + lane) * VEC;
  float x[VEC];
  if constexpr (DT == 0) {
    const float *rowp = (const float *)a.logits + (uint64_t)row * a.stride;
    if (t0 + VEC <= V) {
      const f32x4 v = *(const f32x4 *)(rowp + t0);
      x[0] = v.x;
      x[1] = v.y;
      x[2] = v.z;
      x[3] = v.w;
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) x[e] = t0 + e < V ? rowp[t0 + e] : kNotAdmitted;
    }
  } else {
    const uint16_t *rowp = (const uint16_t *)a.logits + (uint64_t)row * a.stride;
    if (t0 + VEC <= V) {
      const u32x4 v = *(const u32x4 *)(rowp + t0);
      const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        x[2 * k] = u2f(vw[k] << 16);
        x[2 * k + 1] = u2f(vw[k] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) x[e] = t0 + e < V ? bf16_to_float(rowp[t0 + e]) : kNotAdmitted;
    }
  }
  float qv[VEC];
  if constexpr (RESID == 1) {
    // A dense q row ends at the vocabulary.
    const float *qrow = a.dense_q + (uint64_t)q_row * a.q_stride;
#pragma unroll
    for (int e = 0; e < VEC; ++e) qv[e] = t0 + e < V ? qrow[t0 + e] : 0.0f;
  } else if constexpr (RESID == 2) {
    // The first candidate that lists the token (sampling.metal:703-708).
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      qv[e] = 0.0f;
      for (int j = 15; j >= 0; --j) qv[e] = s.cids[j] == t0 + e ? s.cprobs[j] : qv[e];
    }
  }
  // The slice's VEC tokens share one mask word (t0 is a multiple of VEC).
  const uint32_t mword =
      (flags & kRowConstrained) && t0 < V ? a.masks[(uint64_t)row * a.mask_stride + (t0 >> 5)] : ~0u;
  uint64_t q[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    const uint32_t t = t0 + e;
    const bool drop = !((mword >> (t & 31)) & 1u) ||
                      ((flags & kRowExcludeStop) && (t == a.stop0 || t == a.stop1));
    const float xe = drop ? kNotAdmitted : x[e];
    if constexpr (RESID == 0)
      q[e] = quantized_weight(xe, mc, inv_t);
    else
      q[e] = residual_of(scaled_weight(xe, mc, inv_t, Rc), W, qv[e]);
  }
  uint32_t e_hit;
  if (lane == slice_hit<VEC>(q, within, e_hit)) write_result(a, row, t0 + e_hit, pd, kept);
}

// finish_acceptance (sampling.metal:1381-1392) on a wave that holds the
// lane's output token t in thread t: the budget min(accepted + 1,
// remaining), then cut after the first stop token within it.
__device__ __forceinline__ uint32_t finish_kept(uint32_t out, uint32_t accepted,
                                                uint32_t remaining, uint32_t stop0,
                                                uint32_t stop1) {
  const uint32_t t = lane_id();
  uint32_t kept = min(accepted + 1, remaining);
  const uint64_t stops = ballot(t < kept && (out == stop0 || out == stop1));
  if (stops) kept = (uint32_t)__builtin_ctzll(stops) + 1;
  return kept;
}

// verify_tree_accept (tree.metal:20-84), on a wave whose thread t holds
// row t's target token `tok` (and, sampled, its p(draft) pv and uniform uv
// of slot 8 + t). From row 0, while the path is shorter than 8: a sampled
// lane's chain row (current + 1 < chain_rows) takes its chain child when
// u[8 + current] q < p; otherwise the lowest row below that is a child of
// the current row and holds the current row's target token (a sampled
// lane's chain child excluded) extends the path; none ends it. Returns the
// path's length; thread i < length holds path[i] in `path`.
__device__ __forceinline__ uint32_t accept_tree_wave(const TreeLaneParams &tr, uint32_t tok,
                                                     float pv, float uv, uint32_t &path) {
  const uint32_t t = lane_id();
  const uint32_t rows = tr.rows, chain = tr.chain_rows;
  const bool sampled = tr.sampled != 0;
  const uint32_t par = t < rows ? tr.parent[t] : kNoToken;
  const uint32_t dtok = t < rows ? tr.token[t] : kNoToken;
  uint32_t length = 1, current = 0;
  path = 0;
  while (length < 8) {
    if (sampled && current + 1 < chain) {
      // Rows 0 .. chain - 1 form a chain (checked by the host), so the
      // chain steps keep current below 7.
      const float q = tr.chain_q[min(current, 7u)];
      const float p = __builtin_bit_cast(float, readlane_u32(__builtin_bit_cast(uint32_t, pv),
                                                             (int)current));
      const float u = __builtin_bit_cast(float, readlane_u32(__builtin_bit_cast(uint32_t, uv),
                                                             (int)current));
      if (u * q < p) {
        if (t == length) path = current + 1;
        ++length;
        ++current;
        continue;
      }
    }
    const uint32_t wanted = readlane_u32(tok, (int)current);
    const bool hit = t > current && t < rows && par == current && dtok == wanted &&
                     !(sampled && t == current + 1 && current + 1 < chain);
    const uint64_t b = ballot(hit);
    if (!b) break;
    current = (uint32_t)__builtin_ctzll(b);
    if (t == length) path = current;
    ++length;
  }
  return length;
}

// Thread i < length: path row i emits its child's token (path[i + 1]) or,
// the last, its own target token (the value for threads past the path is
// not used).
__device__ __forceinline__ uint32_t tree_path_token(const TreeLaneParams &tr, uint32_t tok,
                                                    uint32_t path, uint32_t length) {
  const uint32_t t = lane_id();
  const uint32_t dtok = t < tr.rows ? tr.token[t] : kNoToken;
  const uint32_t next = __shfl_down(path, 1);
  const uint32_t child_tok = __shfl(dtok, (int)next);
  const uint32_t own_tok = __shfl(tok, (int)path);
  return t + 1 < length ? child_tok : own_tok;
}

// The lane's retained and accepted counts and its path rows, from the wave
// whose thread t holds output token `out` and path row `path`.
__device__ __forceinline__ void finish_tree_lane(const AcceptTreeLaunch &a, uint32_t lane,
                                                 const TreeLaneParams &tr, uint32_t out,
                                                 uint32_t path, uint32_t length) {
  const uint32_t t = lane_id();
  const uint32_t kept = finish_kept(out, length - 1, tr.remaining, a.stop0, a.stop1);
  const uint32_t last = readlane_u32(path, (int)(length - 1));
  if (t < 8) a.path_rows[(uint64_t)lane * 8 + t] = t < length ? path : last;
  if (t == 0) {
    a.retained[lane] = kept;
    a.accepted[lane] = length - 1;
  }
}

// ---- the fast selection kernel ---------------------------------------------
//
// select_kernel's results for the rows the host admits (16-byte aligned rows,
// every penalty chunk within its fixed slots, no extra verify tokens), with a
// load phase that requests everything before it waits on anything:
//   1. the chunk's penalty slots (their address needs only the kernel
//      arguments), then the logits with 16-byte loads, then a constrained
//      row's mask words;
//   2. each slot's thread re-reads its token's logit (and mask word): the
//      block's own request for that line is already in flight, so the read
//      merges with it in L2 instead of waiting behind the whole stream. The
//      thread holds the penalized token as a side entry; the lane that loaded
//      the token drops it through a per-thread bitmap (bit i <-> register i);
//   3. greedy rows take the block maximum first and then the lowest id that
//      holds it; sampled rows write the chunk summary and candidates exactly
//      as select_kernel does.

struct __align__(16) FastLds {
  uint32_t bm[kThreads];  // bit i of bm[t]: register i of thread t is dropped
  uint32_t xt[kMaxExtra];  // the row's extra penalty tokens (XTRA launches)
  uint64_t stage[kWaves][kWaveCandidates];
  uint64_t slices[kWaves * 8];  // an uncut row's slice masses
  uint32_t wcount[kWaves];
  float wf[kWaves];
  uint32_t wu[kWaves];
  uint32_t wu2[kWaves];
};

// LDS of the fast kernel's variant that finishes rows with no cut itself:
// the row's chunk slice masses and summaries, gathered by its last chunk's
// block.
struct __align__(16) FusedUncutLds : FastLds {
  uint64_t fsl[kMaxChunks * 32];  // slice masses, G a chunk, chunk-major
  float cmax[kMaxChunks];         // chunk maxima
  uint32_t cinfo[kMaxChunks];     // admitted count << 1 | admits
  uint32_t fail;                  // some wait gave up
};

// The largest multiple of 2^16 with at least k (1..64) lanes holding a value
// >= it: a lower bound of the k-th largest that needs 16 ballots, not 32.
__device__ __forceinline__ uint32_t wave_kth_bound16(uint32_t v, uint32_t k) {
  uint32_t answer = 0;
#pragma unroll
  for (int b = 31; b >= 16; --b) {
    const uint32_t trial = answer | (1u << b);
    if ((uint32_t)__popcll(ballot(v >= trial)) >= k) answer = trial;
  }
  return answer;
}

// A RowParams record read through the scalar cache. The records are written
// only before the launch (by a copy or an earlier kernel), so the record is
// read through the constant address space: the compiler then emits scalar
// loads for the uniform address at this point of the program, counts them
// itself and waits for them before the first use of a field. (A scalar load
// inside inline asm is invisible to the compiler's wait counting: code the
// compiler places between such a load and its wait, such as register copies,
// would read registers the load has not yet written.)
typedef const __attribute__((address_space(4))) uint32_t *ConstWords;
__device__ __forceinline__ RowParams load_row_policy(const RowParams *p) {
  const uint64_t addr = (uint64_t)p;
  const uint64_t u =
      ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(addr >> 32)) << 32) |
      (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)addr);
  const ConstWords w = (ConstWords)u;
  uint32_t v[sizeof(RowParams) / 4];
#pragma unroll
  for (int i = 0; i < (int)(sizeof(RowParams) / 4); ++i) v[i] = w[i];
  RowParams rp;
  __builtin_memcpy(&rp, v, sizeof(rp));
  return rp;
}

// Register i of a thread and the thread that loads chunk offset o.
template <int DT>
__device__ __forceinline__ uint32_t owner_of(uint32_t o) {
  return (o % Geo<DT>::SLAB) / Geo<DT>::VEC;
}
template <int DT>
__device__ __forceinline__ uint32_t register_of(uint32_t o) {
  return (o / Geo<DT>::SLAB) * Geo<DT>::VEC + o % Geo<DT>::VEC;
}

// The thread's 32 tokens of chunk `base`, requested without a wait. A full
// chunk issues its loads unconditionally. The partial last chunk clamps each
// vector load to the last whole vector of the row (always in bounds; the
// host admits V >= 8 only) and reads the tokens past the last whole vector
// into `tail` element by element, after every vector load is out. The
// registers past the vocabulary are the caller's to drop (past_end_bits).
template <int DT>
__device__ __forceinline__ void fast_load(const void *logits, uint64_t stride,
                                          uint32_t V, uint32_t row, uint32_t base,
                                          bool full, float (&xs)[32],
                                          std::conditional_t<DT == 0, float, uint32_t> (&tail)[Geo<DT>::VEC],
                                          uint32_t &tail_j) {
  constexpr int VEC = Geo<DT>::VEC, LOADS = Geo<DT>::LOADS, SLAB = Geo<DT>::SLAB;
  const uint32_t lane_base = base + threadIdx.x * VEC;
  using Raw = std::conditional_t<DT == 0, float, uint16_t>;
  const Raw *rowp = (const Raw *)logits + (uint64_t)row * stride;
  u32x4 v[LOADS];
  const uint32_t vfull = V - V % VEC;  // tokens covered by whole vectors
  // One load sequence for both (a branch here makes the compiler wait
  // between the partial chunk's loads): the address is selected, not the code.
  // Plain loads: the lines stay in L2 for the penalty threads' re-reads
  // (streaming loads would send many of those back to HBM).
#pragma unroll
  for (int j = 0; j < LOADS; ++j) {
    const uint32_t t0 = lane_base + j * SLAB;
    const uint32_t tl = full || t0 + VEC <= vfull ? t0 : vfull - VEC;
    v[j] = *(const u32x4 *)(rowp + tl);
  }
  tail_j = 0xffu;
  if (!full) {
#pragma unroll
    for (int j = 0; j < LOADS; ++j)
      if (lane_base + j * SLAB == vfull && vfull < V) tail_j = (uint32_t)j;
    if (tail_j != 0xffu) {
      // Unconditional loads at clamped indices, kept raw until the caller
      // places them (no wait here); the registers past the vocabulary are
      // dropped by the caller.
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        // A vector load (the uniform index would otherwise make it a scalar
        // load, which the next barrier waits for).
        uint32_t idx = min(vfull + e, V - 1);
        asm volatile("" : "+v"(idx));
        tail[e] = rowp[idx];
      }
    }
  }
#pragma unroll
  for (int j = 0; j < LOADS; ++j) {
    if constexpr (DT == 0) {
      xs[j * 4 + 0] = u2f(v[j].x);
      xs[j * 4 + 1] = u2f(v[j].y);
      xs[j * 4 + 2] = u2f(v[j].z);
      xs[j * 4 + 3] = u2f(v[j].w);
    } else {
      xs[j * 8 + 0] = u2f(v[j].x << 16);
      xs[j * 8 + 1] = u2f(v[j].x & 0xffff0000u);
      xs[j * 8 + 2] = u2f(v[j].y << 16);
      xs[j * 8 + 3] = u2f(v[j].y & 0xffff0000u);
      xs[j * 8 + 4] = u2f(v[j].z << 16);
      xs[j * 8 + 5] = u2f(v[j].z & 0xffff0000u);
      xs[j * 8 + 6] = u2f(v[j].w << 16);
      xs[j * 8 + 7] = u2f(v[j].w & 0xffff0000u);
    }
  }
}

// Drop bits of the thread's registers that hold no token of the vocabulary.
template <int DT>
__device__ __forceinline__ uint32_t past_end_bits(uint32_t V, uint32_t base) {
  constexpr int VEC = Geo<DT>::VEC, LOADS = Geo<DT>::LOADS, SLAB = Geo<DT>::SLAB;
  constexpr uint32_t VMASK = (1u << VEC) - 1u;
  const uint32_t lane_base = base + threadIdx.x * VEC;
  uint32_t bits = 0;
#pragma unroll
  for (int j = 0; j < LOADS; ++j) {
    const uint32_t t0 = lane_base + j * SLAB;
    const uint32_t m = t0 + VEC <= V ? 0u
                       : t0 >= V     ? VMASK
                                     : VMASK & ~((1u << (V - t0)) - 1u);
    bits |= m << (j * VEC);
  }
  return bits;
}

// The arguments a block needs before its first load lead the signature (13
// dwords, no padding; the hardware has 14 to preload): they arrive in scalar
// registers at wave launch, so a wave that starts while the memory system is
// already full of other waves' loads does not wait for its own arguments
// behind them. `packed`: bits 0-7 the uniform flags, 8-15 the chunks per
// row, bit 16 set for 512 penalty slots per chunk (else 256), bits 17-30 the
// first row over 256, bit 31 set when the launch is uniform: every row has
// those flags, reads penalty table row == its own row and the policy values
// that follow; otherwise each row reads its flags and penalty row from
// f.row_info and its policy from f.a.params.
#if JF_IN(1)
// The greedy finish of one row by wave 0 of its finishing block: lane c < S
// reads chunk c's packed best (lane `own` holds `mine`, its own chunk's),
// re-reading up to a.wait_bound times until the word carries this call's
// tag, and returns each word it took to zero. The largest word wins.
// Should a wait reach its bound (a word not written by then: the argument
// that every wait ends has failed), the row gets JF_NO_TOKEN, the sampler's
// status word is set for the host to report, and the words are left for
// the host's clear.
// Returns whether the row finished (its token in `token`, every lane); with
// `write` false the caller writes the result.
__device__ __forceinline__ bool finish_greedy_row(const SampleLaunch &a, uint32_t row,
                                                  uint32_t S, uint32_t own, uint64_t mine,
                                                  uint64_t tag, uint32_t &token,
                                                  bool write = true) {
  const uint32_t lane = lane_id();
  uint64_t best = 0;
  bool ok = true;
  if (lane == own) {
    best = mine;
  } else if (lane < S) {  // S <= kMaxChunks = 64
    uint64_t *word = a.bests + (uint64_t)row * S + lane;
    for (uint32_t n = 0; (best & 0x1fffu) != tag && n < a.wait_bound; ++n) best = ld_dev(word);
    ok = (best & 0x1fffu) == tag;
    if (ok) st_dev(word, 0ull);
  }
  token = kNoToken;
  if (ballot(!ok) != 0) {
    if (lane == 0) {
      if (write) write_result(a, row, kNoToken, 0.0f, 0);
      if (a.status) __hip_atomic_store(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    return false;
  }
  const uint32_t key = wave_max_u32((uint32_t)(best >> 32));
  const uint32_t low = wave_max_u32((uint32_t)(best >> 32) == key ? (uint32_t)best : 0u);
  token = key ? 0x7ffffu - (low >> 13) : kNoToken;
  if (write && lane == 0) write_result(a, row, token, 0.0f, 0);
  return true;
}

// All-greedy rows whose lanes' tree acceptance runs in the select launch
// (the lanes' rows = the launch's rows, R a lane, every lane greedy). Each
// row's finisher publishes its token as a self-validating word (token << 32
// | tag) in partial slot kAcceptSlot of the row's chunk 0; the finisher of
// a lane's last row gathers the lane's tokens (thread t row t, bounded
// waits, each word returned to zero), writes every row's result (the path's
// outputs over the first rows, the selected tokens after them) and the
// lane's counts and path rows. Its waits are for blocks dispatched before
// it (rows in order, chunk fastest), which wait on nothing but their own
// rows' earlier blocks. A wait that gives up leaves the lane's rows
// JF_NO_TOKEN and sets the status word.
constexpr uint32_t kAcceptSlot = 200;
// The walk of lane `row / R` by the finisher of its last row, whose own
// token is `token`; lanes 32 + t of the wave hold row t's published word in
// `early` (t < R - 1) when the caller gathered them already (have_early),
// else they are gathered here.
__device__ __forceinline__ void accept_lane(const SampleLaunch &a, const AcceptTreeLaunch &acc,
                                            uint32_t row, uint32_t S, uint32_t token, bool ok,
                                            uint64_t tag, bool have_early, uint64_t early) {
  const uint32_t t = lane_id();
  const uint32_t R = acc.rows_per_lane, lane = row / R, first = lane * R;
  uint32_t tok = token;
  bool got = ok;
  if (have_early) {
    const uint64_t v = shfl_u64(early, (int)(32 + t));
    if (t + 1 < R) {
      got = (v & 0x1fffu) == tag;
      tok = (uint32_t)(v >> 32);
    }
  } else if (t + 1 < R) {
    uint64_t *word = &a.partials[(uint64_t)(first + t) * S].v[kAcceptSlot];
    uint64_t v = 0;
    for (uint32_t n = 0; (v & 0x1fffu) != tag && n < a.wait_bound; ++n) v = ld_dev(word);
    got = (v & 0x1fffu) == tag;
    if (got) st_dev(word, 0ull);
    tok = (uint32_t)(v >> 32);
  }
  if (ballot(t < R && !got) != 0) {
    if (t < R) write_result(a, first + t, kNoToken, 0.0f, 0);
    if (t == 0 && a.status)
      __hip_atomic_store(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    return;
  }
  if (t >= R) tok = kNoToken;
  const TreeLaneParams &tr = acc.trees[lane];
  uint32_t path;
  const uint32_t length = accept_tree_wave(tr, tok, 0.0f, 0.0f, path);
  const uint32_t out = tree_path_token(tr, tok, path, length);
  if (t < R) write_result(a, first + t, t < length ? out : tok, 0.0f, 0);
  finish_tree_lane(acc, lane, tr, out, path, length);
}

// A row's finisher in a launch with the lanes' tree acceptance: a lane's
// last row gathers its chunk bests (lanes 0 .. S - 1) and, in the same
// round of reads, the lane's other rows' tokens (lanes 32 .. 32 + R - 2)
// when the row has at most 32 chunks, then walks the tree; any other row
// publishes its token.
__device__ __forceinline__ void finish_row_and_lane(const SampleLaunch &a,
                                                    const AcceptTreeLaunch &acc, uint32_t row,
                                                    uint32_t S, uint32_t own, uint64_t mine,
                                                    uint64_t tag) {
  const uint32_t t = lane_id();
  const uint32_t R = acc.rows_per_lane, first = row / R * R;
  const bool lane_last = row + 1 == first + R;
  if (!lane_last || S > 32) {
    uint32_t token;
    const bool ok = finish_greedy_row(a, row, S, own, mine, tag, token, false);
    if (!lane_last) {
      if (ok && t == 0)
        st_dev(&a.partials[(uint64_t)row * S].v[kAcceptSlot], (uint64_t)token << 32 | tag);
      return;
    }
    accept_lane(a, acc, row, S, token, ok, tag, false, 0ull);
    return;
  }
  uint64_t v = 0;
  bool ok = true;
  uint64_t *word = nullptr;
  if (t == own) v = mine;
  else if (t < S) word = a.bests + (uint64_t)row * S + t;
  else if (t >= 32 && t - 32 + 1 < R)
    word = &a.partials[(uint64_t)(first + t - 32) * S].v[kAcceptSlot];
  if (word) {
    for (uint32_t n = 0; (v & 0x1fffu) != tag && n < a.wait_bound; ++n) v = ld_dev(word);
    ok = (v & 0x1fffu) == tag;
    if (ok) st_dev(word, 0ull);
  }
  const bool row_ok = ballot(t < S && !ok) == 0;
  const uint32_t hi = t < S ? (uint32_t)(v >> 32) : 0u;
  const uint32_t key = wave_max_u32(hi);
  const uint32_t low = wave_max_u32(t < S && hi == key ? (uint32_t)v : 0u);
  const uint32_t token = key ? 0x7ffffu - (low >> 13) : kNoToken;
  if (!row_ok && t == 0 && a.status)
    __hip_atomic_store(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  accept_lane(a, acc, row, S, token, row_ok, tag, true, v);
}

// select_fast_kernel's arguments as the kernel-argument segment holds them
// (each at its natural alignment, in order).
// Grids of at most this many blocks warm the scalar cache with the launch
// record (select_fast_kernel).
constexpr uint32_t kWarmGrid = 2048;

struct FastKernelArgs {
  const void *logits;
  const uint32_t *pen_slots;
  uint32_t stride, V, packed, u_top_k;
  float u_minp_offset, u_repetition, u_repetition_inverse, u_presence, u_frequency;
  uint32_t mapped;
  FastLaunch f;
};
static_assert(offsetof(FastKernelArgs, f) == 56, "the launch record follows 14 dwords");

// The fast selection's launch record, read in place in the kernel-argument
// segment: each field by a scalar load where it is used. The segment's
// address passes through an empty asm statement so that the compiler cannot
// trace the loads to the kernel argument: it would otherwise load the whole
// record into scalar registers at the kernel's entry and keep it there,
// which raised the kernel's register use (bf16: 69 to 85 vector registers,
// one wave less per SIMD). (Taking the argument's address instead would
// make the compiler copy the record to private memory.)
__device__ __forceinline__ const SampleLaunch &fast_launch_record() {
  uint64_t u = (uint64_t)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(u));
  typedef const __attribute__((address_space(4))) FastKernelArgs *KernargPtr;
  return ((const FastKernelArgs *)(KernargPtr)u)->f.a;
}
// Whether the launch's row y stores its weights (FastLaunch::lean_bits, read
// in place like the record).
__device__ __forceinline__ bool fast_lean_row(uint32_t y) {
  uint64_t u = (uint64_t)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(u));
  typedef const __attribute__((address_space(4))) FastKernelArgs *KernargPtr;
  return (((const FastKernelArgs *)(KernargPtr)u)->f.lean_bits[y >> 5] >> (y & 31)) & 1u;
}

// Rows with no cut finished in the select launch (every row of the launch
// sampled with no min-p, top-k or top-p cut, no draft, penalty, extra token
// or kept output). Each chunk block publishes its chunk's summary and slice
// masses as self-validating words: the summary in partial slot
// kFusedSummarySlot (the maximum's order key << 32 | admitted count << 14 |
// admits << 13 | tag), slice g in kFusedSliceSlot + g (mass, below 2^54, |
// tag10 << 54); tag = call epoch << 1 | 1 (12 bits of it, 9 for tag10). The
// row's last chunk's block gathers them, waiting word by word (bounded) for
// any not yet written, returns each word it took to zero, and draws as
// uncut_kernel does for a row without a draft: M, the rescales r_c, the
// chunk masses T_c and W; the chunk and slice that hold floor(u W); that
// slice's 64 x VEC logits reloaded (masked and stop tokens dropped) and
// walked. Its waits end: the row's other blocks were dispatched before it
// (in order of block index, chunk fastest) and wait on nothing. Should one
// give up, the row gets JF_NO_TOKEN and the status word is set.
constexpr uint32_t kFusedSummarySlot = 100, kFusedSliceSlot = 101;
template <int DT>
__device__ __forceinline__ void finish_uncut_row(const SampleLaunch &a, const float (&xs)[32],
                                                 const SideEntries &side, uint32_t base,
                                                 float bmax, uint32_t badm, float inv_t,
                                                 FusedUncutLds &s, uint32_t row, uint32_t chunk,
                                                 uint32_t S, uint32_t flags) {
  constexpr uint32_t G = Geo<DT>::LOADS * kWaves;
  const uint32_t tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  StagePartial *parts = a.partials + (uint64_t)row * S;
  const bool finisher = chunk + 1 == S;
  // The row's uniform, requested before the gather.
  const float u = finisher ? row_uniform(a, row) : 0.0f;
  if (tid == 0) s.fail = 0;
  uncut_slices<DT>(xs, side, base, bmax, inv_t, s);
  const uint32_t count = s.wcount[0] + s.wcount[1] + s.wcount[2] + s.wcount[3];
  const uint32_t info = count << 1 | (badm ? 1u : 0u);
  const uint64_t tag = ((uint64_t)(a.epoch & 0xfffu) << 1) | 1ull;
  const uint64_t tag10 = ((uint64_t)(a.epoch & 0x1ffu) << 1) | 1ull;
  constexpr uint64_t kMass54 = (1ull << 54) - 1ull;
  if (!finisher) {
    if (w == 0) {
      if (lane < G) st_dev(&parts[chunk].v[kFusedSliceSlot + lane], s.slices[lane] | tag10 << 54);
      if (lane == 0)
        st_dev(&parts[chunk].v[kFusedSummarySlot],
               (uint64_t)logit_key(bmax) << 32 | (uint64_t)info << 13 | tag);
    }
    return;
  }
  // The gather: every other chunk's slices (all threads) and summaries
  // (threads 0 .. S - 2), each word re-read until it carries this call's tag.
  bool ok = true;
  for (uint32_t k = tid; k < (S - 1) * G; k += kThreads) {
    const uint32_t c = k / G, g = k % G;
    uint64_t *word = &parts[c].v[kFusedSliceSlot + g];
    uint64_t v = 0;
    for (uint32_t n = 0; (v >> 54) != tag10 && n < a.wait_bound; ++n) v = ld_dev(word);
    if ((v >> 54) == tag10) {
      s.fsl[k] = v & kMass54;
      st_dev(word, 0ull);
    } else {
      ok = false;
    }
  }
  if (tid + 1 < S) {
    uint64_t *word = &parts[tid].v[kFusedSummarySlot];
    uint64_t v = 0;
    for (uint32_t n = 0; (v & 0x1fffu) != tag && n < a.wait_bound; ++n) v = ld_dev(word);
    if ((v & 0x1fffu) == tag) {
      s.cmax[tid] = key_logit((uint32_t)(v >> 32));
      s.cinfo[tid] = (uint32_t)(v >> 13) & 0x7fffu;
      st_dev(word, 0ull);
    } else {
      ok = false;
    }
  }
  if (tid < G) s.fsl[(S - 1) * G + tid] = s.slices[tid];
  if (tid == 0) {
    s.cmax[S - 1] = bmax;
    s.cinfo[S - 1] = info;
  }
  if (!ok) s.fail = 1;
  __syncthreads();
  if (s.fail) {
    if (tid == 0) {
      write_result(a, row, kNoToken, 0.0f, 0);
      if (a.status) __hip_atomic_store(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    return;
  }
  if (w != 0) return;
  // Wave 0 draws (uncut_kernel's undrafted row): lane c < S holds chunk c.
  const bool in = lane < S;
  const float m = in ? s.cmax[lane] : -3.402823466e38f;
  const uint32_t ci = in ? s.cinfo[lane] : 0u;
  uint64_t mass = 0;
  if (in)
#pragma unroll
    for (uint32_t g = 0; g < G; ++g) mass += s.fsl[lane * G + g];
  const float M = wave_max_f32(m);
  const uint64_t R = in ? chunk_scale(m, M, inv_t) : kZeroScale;
  const uint64_t T = scale_by(mass, R);
  const uint64_t incl = wave_incl_scan_u64(T);
  const uint64_t W = readlane_u64(incl, 63);
  const uint32_t admitted = wave_sum_u32(ci & 1u), kept = wave_sum_u32(ci >> 1);
  const bool none = admitted == 0 || M == __builtin_inff();
  if (none || W == 0) {
    // The sentinel (a row of -inf keeps every token at probability 0).
    if (lane == 0) write_result(a, row, kNoToken, 0.0f, none ? 0u : kept);
    return;
  }
  uint64_t target = floor_mul(W, u);
  if (target >= W) target = W - 1;
  // incl at the last lane is W > target: some lane passes it.
  const uint32_t c = (uint32_t)__builtin_ctzll(ballot(in && incl > target));
  uint64_t within = unscaled_bound(target - readlane_u64(incl - T, c), readlane_u64(R, c));
  const uint64_t vg = lane < G ? s.fsl[c * G + lane] : 0ull;
  const uint32_t g = pick_slice(vg, G, within);
  draw_in_slice<DT, 0>(a, row, flags, inv_t, 0u, c, g, within, __shfl(m, (int)c, kWave), 0ull,
                       0ull, 0.0f, kept, s);
}

// A launch's per-row fact of row `i`: 0 its sampler row, 1 its flags and
// penalty row, 2 its extra tokens (0 without per-row facts).
template <int F, class R>
__device__ __forceinline__ uint32_t fast_row_fact(const R &fr, uint32_t i) {
  if constexpr (std::is_same_v<R, NoRows>) {
    return 0u;
  } else {
    return F == 0 ? fr.row_of[i] : F == 1 ? fr.row_info[i] : fr.row_extra[i];
  }
}

// XTRA: the launch's rows may carry extra (verify) penalty tokens, read as
// scalars from fr.row_extra's place in SampleLaunch::extra. R: FastRows, or
// NoRows for a uniform launch with no row map and no extra tokens.
template <int DT, bool XTRA, class R, class FIN>
__global__ __launch_bounds__(kThreads) void select_fast_kernel(
    const void *logits, const uint32_t *pen_slots, uint32_t stride, uint32_t V,
    uint32_t packed, uint32_t u_top_k, float u_minp_offset, float u_repetition,
    float u_repetition_inverse, float u_presence, float u_frequency, uint32_t mapped,
    FastLaunch f, R fr, FIN fin) {
  constexpr int VEC = Geo<DT>::VEC, TPL = Geo<DT>::TPL, SLAB = Geo<DT>::SLAB,
                LOADS = Geo<DT>::LOADS;
  constexpr uint32_t CHUNK = Geo<DT>::CHUNK;
  constexpr uint32_t VMASK = (1u << VEC) - 1u;
  constexpr bool kRows = !std::is_same_v<R, NoRows>;
  constexpr bool FUSE = std::is_same_v<FIN, UncutFinish>;
  constexpr bool STORE = std::is_same_v<FIN, StoreWeights>;
  constexpr bool ACCEPT = std::is_same_v<FIN, AcceptTreeLaunch>;
  static_assert(TPL == 32, "one drop bit per register");
  static_assert(kRows || !XTRA, "extra tokens travel in the per-row facts");
  const SampleLaunch &a = fast_launch_record();
  __shared__ std::conditional_t<FUSE, FusedUncutLds, FastLds> s;
  const uint32_t S = (packed >> 8) & 0xffu;
  const uint32_t slot_count = (packed & 0x10000u) ? 512u : 256u;
  const uint32_t row_base = ((packed >> 17) & 0x3fffu) << 8;
  const uint32_t chunk = blockIdx.x, lrow = blockIdx.y;
  const uint32_t row = kRows && mapped ? fast_row_fact<0>(fr, lrow) : row_base + lrow;
  const bool uni = !kRows || (packed >> 31) != 0;
  const uint32_t info = uni ? ((packed & 0xffu) | (row << 8)) : fast_row_fact<1>(fr, lrow);
  const uint32_t flags = info & 0xffu, prow = info >> 8;
  const uint32_t tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const uint32_t base = chunk * CHUNK;
  const uint32_t lane_base = base + tid * VEC;
  const bool full = base + CHUNK <= V;
  const bool penalized = (flags & kRowPenalized) != 0;
  const bool constrained = (flags & kRowConstrained) != 0;

  // 1. Every request of the chunk: penalty slots, logits, mask words.
  constexpr int SPT = kSideEntries;  // slots per thread (slot_count <= 512)
  uint32_t slot[SPT];
#pragma unroll
  for (int k = 0; k < SPT; ++k) slot[k] = 0;
  if (penalized) {
    const uint32_t *sp = pen_slots + ((uint64_t)prow * S + chunk) * slot_count;
#pragma unroll
    for (int k = 0; k < SPT; ++k)
      if (k * kThreads < (int)slot_count) slot[k] = sp[tid + k * kThreads];
    s.bm[tid] = 0;
  }
  // A verify row's extra penalty tokens (penalize_verify, sampling.metal:
  // 978-993: row r counts the draft tokens 1..r): up to 16, lane e of each
  // wave loading extra e, requested with the slots (before the logits) and
  // staged in LDS before the first barrier.
  uint32_t xtok = kNoToken;
  if constexpr (XTRA) {
    const uint32_t xr = fast_row_fact<2>(fr, lrow);
    const uint32_t nx = penalized ? xr >> 27 : 0u;
    if (tid < nx) xtok = a.extra[(xr & kExtraOffsetMask) + tid];
  }
  float xs[TPL];
  std::conditional_t<DT == 0, float, uint32_t> tail[VEC];
  uint32_t tail_j;
  fast_load<DT>(logits, stride, V, row, base, full, xs, tail, tail_j);
  if (w == kWaves - 1 && gridDim.x * gridDim.y <= kWarmGrid) {
    // The last wave, its loads in flight, reads one word of each 64-byte
    // line of the launch record into the scalar cache: the fields the
    // block's end reads (list, header, best and result addresses, the
    // epoch) are then there instead of a round trip to memory each. Only
    // in grids the chip holds at about once: in a larger one the blocks
    // that follow on a CU find the lines there already.
    // (The record starts 56 bytes into the argument segment, whose lines
    // start at multiples of 64.)
    static_assert(offsetof(FastKernelArgs, f) == 56, "the record's offset in the segment");
    const uint32_t *rec = reinterpret_cast<const uint32_t *>(&a);
    uint32_t touched = rec[0];
#pragma unroll
    for (uint32_t k = 2; k < sizeof(SampleLaunch) / 4; k += 16) touched ^= rec[k];
    asm volatile("" ::"s"(touched));
  }
  uint32_t mw[LOADS];
  const uint32_t *mrow = nullptr;
  if (constrained) {
    mrow = a.masks + (uint64_t)row * a.mask_stride;
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const uint32_t t0 = lane_base + j * SLAB;
      mw[j] = t0 < V ? mrow[t0 >> 5] : 0u;
    }
  }
  if constexpr (XTRA) {
    if (tid < kMaxExtra) s.xt[tid] = xtok;
  }
  if (penalized) __syncthreads();  // drop bitmaps cleared (and extras staged)
  // A non-uniform row's policy by scalar loads issued after that barrier
  // (a barrier waits for every outstanding scalar load); their wait sits at
  // the first use.
  // A row with no cut reads its temperature from the record too (a
  // uniform launch's preloaded policy leaves it out).
  const bool uncut = (flags & kRowSampled) && !(flags & (kRowMinP | kRowTopK | kRowTopP));
  RowParams prec{};
  if (!uni || uncut) prec = load_row_policy(a.params + row);
  auto row_policy = [&]() -> RowParams {
    if (!uni) return prec;
    RowParams r{};
    r.flags = flags;
    r.top_k = u_top_k;
    r.minp_offset = u_minp_offset;
    r.repetition = u_repetition;
    r.repetition_inverse = u_repetition_inverse;
    r.presence = u_presence;
    r.frequency = u_frequency;
    return r;
  };

  // 2. Penalized tokens: recorded in the drop bitmaps, re-read by their
  // slot's thread, penalized there (sampling.metal:928-963) and admitted
  // (sampling.metal:33-37).
  uint32_t drop = 0, slot_drop = 0;
  uint32_t xin = 0, xmine = kNoToken, xcnt = 0;  // this chunk's extras (XTRA launches)
  SideEntries side;
#pragma unroll
  for (int k = 0; k < SPT; ++k) {
    side.tok[k] = kNoToken;
    side.val[k] = kNotAdmitted;
  }
  RowParams rp;
  if (penalized) {
    uint32_t raw[SPT], mword[SPT];
#pragma unroll
    for (int k = 0; k < SPT; ++k) {
      raw[k] = 0;
      mword[k] = 0;
      if (slot[k]) {
        const uint32_t o = slot[k] >> kSlotOffsetShift, t = base + o;
        atomicOr(&s.bm[owner_of<DT>(o)], 1u << register_of<DT>(o));
        if constexpr (DT == 0)
          raw[k] = f2u(((const float *)logits)[(uint64_t)row * stride + t]);
        else
          raw[k] = (uint32_t)((const uint16_t *)logits)[(uint64_t)row * stride + t];
        if (constrained) mword[k] = mrow[t >> 5];
      }
    }
    __syncthreads();  // bitmaps complete
    drop = s.bm[tid];
    slot_drop = drop;
    rp = row_policy();
    if constexpr (XTRA) {
      // Lane e < 16 of every wave: extra e, whether it lies in this chunk and
      // is the first of its equal ones (bit e of xin, the same in every
      // wave), and how many of the row's extras equal it (xcnt).
      const uint32_t le = lane & (kMaxExtra - 1);
      xmine = s.xt[le];
      bool first = lane < kMaxExtra && xmine - base < CHUNK && xmine < V;
      for (uint32_t e2 = 0; e2 < (uint32_t)kMaxExtra; ++e2) {
        const uint32_t o2 = s.xt[e2];
        xcnt += o2 == xmine ? 1u : 0u;
        first = first && !(e2 < le && o2 == xmine);
      }
      xin = (uint32_t)ballot(first);
    }
#pragma unroll
    for (int k = 0; k < SPT; ++k) {
      if (slot[k]) {
        const uint32_t o = slot[k] >> kSlotOffsetShift, t = base + o;
        uint32_t count = slot[k] & kSlotCountMask;
        if constexpr (XTRA) {
          for (uint32_t bits = xin; bits; bits &= bits - 1) {
            const int e = __builtin_ctz(bits);
            count += readlane_u32(xmine, e) == t ? readlane_u32(xcnt, e) : 0u;
          }
        }
        const float x = DT == 0 ? u2f(raw[k]) : bf16_to_float(raw[k]);
        float v = penalize(x, count, rp.repetition, rp.repetition_inverse,
                           rp.presence, rp.frequency);
        if (constrained && !((mword[k] >> (t & 31)) & 1u)) v = kNotAdmitted;
        if ((flags & kRowExcludeStop) && (t == a.stop0 || t == a.stop1)) v = kNotAdmitted;
        side.tok[k] = t;
        side.val[k] = v;
      }
    }
  }
  // The constraint mask and the stop tokens join the drop bits.
  if (constrained) {
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const uint32_t t0 = lane_base + j * SLAB;
      const uint32_t keep = (mw[j] >> (t0 & 31)) & VMASK;
      drop |= (~keep & VMASK) << (j * VEC);
    }
  }
  bool stop_here = false;
  if (flags & kRowExcludeStop) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const uint32_t st = k ? a.stop1 : a.stop0;
      if (st >= base && st < base + CHUNK) {
        stop_here = true;
        const uint32_t o = st - base;
        if (owner_of<DT>(o) == tid) drop |= 1u << register_of<DT>(o);
      }
    }
  }
  if (!full) {
    drop |= past_end_bits<DT>(V, base);
    if (tail_j != 0xffu)
#pragma unroll
      for (int j = 0; j < LOADS; ++j)
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          xs[j * VEC + e] = (uint32_t)j == tail_j ? (DT == 0 ? (float)tail[e] : bf16_to_float((uint32_t)tail[e]))
                                                  : xs[j * VEC + e];
  }
  if constexpr (XTRA) {
    // An extra token with no fixed slot in this chunk holds no table entry
    // (a row on this kernel has every entry in a slot): its penalty is its
    // extras' count alone (sampling.metal:941-963), applied in place by the
    // thread that loaded it.
    for (uint32_t bits = xin; bits; bits &= bits - 1) {
      const int e = __builtin_ctz(bits);
      const uint32_t o = readlane_u32(xmine, e) - base, reg = register_of<DT>(o);
      float xv = 0.0f;
#pragma unroll
      for (int i = 0; i < TPL; ++i) xv = (uint32_t)i == reg ? xs[i] : xv;
      const float pv = penalize(xv, readlane_u32(xcnt, e), rp.repetition, rp.repetition_inverse,
                                rp.presence, rp.frequency);
      const bool mine = tid == owner_of<DT>(o) && !((slot_drop >> reg) & 1u);
#pragma unroll
      for (int i = 0; i < TPL; ++i) xs[i] = mine && (uint32_t)i == reg ? pv : xs[i];
    }
  }
  if (penalized || constrained || stop_here || !full) {
    // A dropped register becomes NaN: its exponent bits and quiet bit set.
#pragma unroll
    for (int i = 0; i < TPL; ++i) {
      const uint32_t m = (uint32_t)((int32_t)(drop << (31 - i)) >> 31);
      xs[i] = u2f(f2u(xs[i]) | (m & 0x7fc00000u));
    }
  }

  if (!penalized) rp = row_policy();

  // 3. The lane's largest admitted value (fmax skips NaN operands, so the NaN
  // it starts from survives only when the lane admits nothing).
  float mx = kNotAdmitted;
#pragma unroll
  for (int i = 0; i < TPL; ++i) mx = __builtin_fmaxf(mx, xs[i]);
#pragma unroll
  for (int k = 0; k < SPT; ++k) mx = __builtin_fmaxf(mx, side.val[k]);
  BlockHeader *hdr = a.headers + (uint64_t)row * S + chunk;

  if (!(flags & kRowSampled)) {
    // Greedy (sampling.metal:1427-1464): the block maximum, then the lowest
    // id holding it. NaN never wins; a -inf token wins only over nothing.
    const float wmax = wave_max_f32(mx);
    if (lane == 0) s.wf[w] = wmax;
    __syncthreads();
    const float M = __builtin_fmaxf(__builtin_fmaxf(s.wf[0], s.wf[1]),
                                    __builtin_fmaxf(s.wf[2], s.wf[3]));
    uint32_t id = kNoToken;
    if (mx == M) {
#pragma unroll
      for (int i = TPL - 1; i >= 0; --i)
        id = xs[i] == M ? lane_base + (i / VEC) * SLAB + (i % VEC) : id;
#pragma unroll
      for (int k = 0; k < SPT; ++k)
        id = side.val[k] == M ? min(id, side.tok[k]) : id;
    }
    const uint32_t wid = wave_min_u32(id);
    if (lane == 0) s.wu[w] = wid;
    __syncthreads();
    const float bv = M == M ? M : -__builtin_inff();
    const uint32_t bi = min(min(s.wu[0], s.wu[1]), min(s.wu[2], s.wu[3]));
    if (!f.fuse_greedy) {
      if (tid == 0) {
        hdr->best_value = bv;
        hdr->best_id = bi;
      }
      return;
    }
    // Each block's best as one 64-bit word: the value's order key in bits
    // 63..32, 0x7FFFF - id in 31..13 (ids stay below 2^19, so the larger
    // word holds the larger value, then the lower id), the call's epoch in
    // 12..1 and bit 0 set (the tag: nothing admitted is the tag alone,
    // below every admitted key). A reader takes a word as this call's only
    // when its tag matches, so neither a cleared word nor a late store of an
    // earlier call passes for it.
    const uint64_t tag = ((uint64_t)(a.epoch & 0xfffu) << 1) | 1ull;
    const uint64_t mine =
        bi == kNoToken ? tag
                       : ((uint64_t)logit_key(bv) << 32) | ((uint64_t)(0x7ffffu - bi) << 13) | tag;
    if (f.fuse_greedy == 2u) {
      // The row's last chunk finishes it: every other block stores its word
      // and ends; this one reads the row's words, waiting word by word for
      // any not yet written, and returns them to zero. Its wait ends: blocks
      // are dispatched in the order of their index (chunk fastest), so the
      // row's other blocks were dispatched before it, and they wait on
      // nothing.
      if (chunk + 1 < S) {
        if (tid == 0) st_dev(a.bests + (uint64_t)row * S + chunk, mine);
        return;
      }
      if (w == 0) {
        if constexpr (ACCEPT) {
          finish_row_and_lane(a, fin, row, S, chunk, mine, tag);
        } else {
          uint32_t token;
          finish_greedy_row(a, row, S, chunk, mine, tag, token);
        }
      }
      return;
    }
    // Every row greedy: the row's last block to arrive takes the largest
    // chunk best, the lowest id among equals (the reference's last-arriving
    // group, split_reduce.h:14-45). The word's store and the arrival go out
    // together; the last block reads the row's words and waits, word by
    // word, for any not yet visible. Each such store was issued before its
    // block's arrival, so every wait ends. The last block returns the words
    // and the counter to zero.
    if (tid == 0) {
      st_dev(a.bests + (uint64_t)row * S + chunk, mine);
      const uint32_t prev = __hip_atomic_fetch_add(a.counters + row, 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
      s.wcount[0] = prev == S - 1 ? 1u : 0u;
      if (prev == S - 1) st_dev(a.counters + row, 0u);
    }
    __syncthreads();
    if (s.wcount[0] && w == 0) {
      uint32_t token;
      finish_greedy_row(a, row, S, S, 0ull, tag, token);
    }
    return;
  }

  const bool any = mx == mx;
  // The chunk's top-k bound, as select_kernel (each wave's ceil(k/4)-th
  // largest lane maximum, rounded down to a multiple of 2^16 of its key).
  const uint32_t K = rp.top_k;
  const uint32_t kw = (K + kWaves - 1) / kWaves;
  const bool bound = (flags & kRowTopK) && kw <= 64;
  uint32_t wth = 0;
  if (bound) wth = wave_kth_bound16(any ? logit_key(mx) : 0u, kw);
  const float wmax = wave_max_f32(mx);
  const uint32_t wany = ballot(any) != 0 ? 1u : 0u;
  if (lane == 0) {
    s.wf[w] = wmax;
    s.wu[w] = wany;
    s.wu2[w] = wth;
  }
  if (uncut && tid < kWaves * 8) s.slices[tid] = 0;
  __syncthreads();
  const float bmax = __builtin_fmaxf(
      __builtin_fmaxf(__builtin_fmaxf(s.wf[0], s.wf[1]),
                      __builtin_fmaxf(s.wf[2], s.wf[3])),
      -3.402823466e38f);
  const uint32_t badm = s.wu[0] | s.wu[1] | s.wu[2] | s.wu[3];
  const uint32_t tk =
      bound ? min(min(s.wu2[0], s.wu2[1]), min(s.wu2[2], s.wu2[3])) : 0u;
  if (uncut) {
    // The row keeps every admitted token: the uncut kernel's chunk summary,
    // or (FUSE) the row finished here.
    const float inv_t = uni ? prec.inv_t : rp.inv_t;
    if constexpr (FUSE) {
      finish_uncut_row<DT>(a, xs, side, base, bmax, badm, inv_t, s, row, chunk, S, flags);
    } else {
      // A drafted row's weights for its residual pass (fp32, no penalty).
      uint32_t *wout = nullptr;
      if (STORE && fast_lean_row(lrow))
        wout = a.lean_weights + (uint64_t)row * a.lean_stride + (uint64_t)chunk * CHUNK;
      uncut_summary<DT>(xs, side, base, bmax, badm, inv_t, s, hdr,
                        a.partials + (uint64_t)row * S + chunk, wout);
    }
    return;
  }
  uint32_t thr = tk;
  if (flags & kRowMinP)
    thr = max(thr, logit_key(__builtin_fminf(bmax + rp.minp_offset, bmax)));
  const float tv = thr <= kLowestKey ? -__builtin_inff() : key_logit(thr);
  uint64_t *stage = s.stage[w];
  uint32_t run = 0;
  auto emit = [&](float x, uint32_t token) {
    const bool hit = x >= tv;
    const uint64_t m = ballot(hit);
    if (m) {
      // Hits past the wave's list land on its last entry: the wave's count
      // then exceeds the list and the chunk is flagged as overflowed, so
      // its staged list is never copied out.
      const uint32_t slot_i = min(__builtin_amdgcn_mbcnt_hi(
                                      (uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, run)),
                                  (uint32_t)kWaveCandidates - 1u);
      if (hit) stage[slot_i] = (uint64_t)f2u(x) | ((uint64_t)token << 32);
      run += (uint32_t)__popcll(m);
    }
  };
#pragma unroll
  for (int j = 0; j < LOADS; ++j)
#pragma unroll
    for (int e = 0; e < VEC; ++e) emit(xs[j * VEC + e], lane_base + j * SLAB + e);
#pragma unroll
  for (int k = 0; k < SPT; ++k) emit(side.val[k], side.tok[k]);
  if (lane == 0) s.wcount[w] = run;
  __syncthreads();
  uint32_t off[kWaves + 1], over = 0;
  off[0] = 0;
#pragma unroll
  for (int k = 0; k < kWaves; ++k) {
    const uint32_t n = s.wcount[k];
    over |= n > kWaveCandidates;
    off[k + 1] = off[k] + min(n, kWaveCandidates);
  }
  uint64_t *dst = a.cands + ((uint64_t)row * S + chunk) * kBlockCandidates;
  if (!over)
    for (uint32_t i = tid; i < off[kWaves]; i += kThreads) {
      const uint32_t k = (i >= off[1]) + (i >= off[2]) + (i >= off[3]);
      const uint64_t e = s.stage[k][i - off[k]];
      dst[i] = (uint64_t)logit_key(u2f((uint32_t)e)) | (e & 0xffffffff00000000ull);
    }
  const uint32_t c = over ? kBlockCandidates + 1 : off[kWaves];
  if (tid == 0) {
    hdr->maximum = bmax;
    hdr->count = min(c, (uint32_t)kBlockCandidates);
    hdr->admitted = badm;
    hdr->overflow = c > (uint32_t)kBlockCandidates ? 1u : 0u;
    hdr->floor_key = tk;
  }
}
#endif

// One block per row merges the row's chunk summaries (the reduction the
// reference's last-arriving group does, split_reduce.h:14-45; here the
// kernel boundary orders the partials before their reader).
#if JF_IN(2)
template <int DT>
__global__ __launch_bounds__(kThreads) void merge_kernel(SampleLaunch a) {
  __shared__ Lds s;
  const uint32_t row = blockIdx.x;
  const RowParams rp = a.params[row];
  merge_row<DT>(a, rp, row, s);
}
#endif

// ---- the small-K merge -----------------------------------------------------
//
// One block per row, for launches whose sampled rows all keep at most 64
// tokens (top-k <= 64) and take their draft probabilities, if any, from the
// sparse candidates. It computes what merge_kernel computes, built for
// latency: every kernel argument in one round trip, then every load the row
// needs in one batch (its policy, the chunk summaries, the first slots of
// every chunk's candidate list, the uniform, the draft and its candidates);
// the 1024-bin histogram that leaves the top K and the boundary bin; and a
// finish by one wave in registers. Rows the speculative fetch does not cover
// (an overflowed chunk, a list longer than the slots fetched, values that do
// not spread over the bins) take merge_kernel's general path.

// The exact top-K (K <= 64) of a row's candidates held in registers (v[k] =
// key | id << 32; bit k of `valid` set for an item at or above the floor),
// written to s.merge.key/id[0, n) in (key desc, id asc) order, n = min(K,
// items). A 1024-bin histogram of the values over [value(thr), maximum] and
// its suffix sums give each item its rank up to the items of its own bin,
// which it compares directly; no sort. Returns n, or -1 when the values do
// not spread over the bins, the boundary bin holds more than 64 items, or
// more than 64 items would be kept (K above 64).
// The caller zeroed s.merge.bins and s.merge.key[1024, 2048) before a
// barrier. Every thread calls it. Uses s.merge.id[1024, 2048) and s.hist.
template <int PER>
__device__ __forceinline__ int rank_select(const uint64_t (&v)[PER], uint32_t valid,
                                           uint32_t thr, uint32_t K, float maximum,
                                           Lds &s) {
  MergeLds &m = s.merge;
  uint32_t *excl = m.id + 1024;   // items in the bins above each bin
  uint32_t *fill = m.key + 1024;  // items placed per bin
  uint64_t *seg = s.hist;         // items of the kept bins, grouped by bin
  const uint32_t tid = threadIdx.x;
  const float lo = key_logit(thr);
  const float scale = 1023.0f / (maximum - lo);
  if (!(scale > 0.0f && scale < 3.0e38f)) return -1;
  auto bin_of = [&](uint32_t key) -> uint32_t {
    return min(1023u, (uint32_t)((key_logit(key) - lo) * scale));
  };
  uint32_t bins[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    bins[k] = bin_of((uint32_t)v[k]);
    if ((valid >> k) & 1) atomicAdd(&m.bins[bins[k]], 1u);
  }
  __syncthreads();
  // Suffix sums: thread t owns bins 4t .. 4t+3; excl(b) counts the items in
  // the bins above b. (The scan's barriers order the flag's reset before the
  // boundary thread sets it.)
  const uint4 c4 = *(const uint4 *)&m.bins[4 * tid];
  const uint32_t own = c4.x + c4.y + c4.z + c4.w;
  if (tid == 0) s.hit = 0;
  uint64_t total64;
  const uint32_t before = (uint32_t)block_excl_scan_u64(own, s, &total64);
  const uint32_t total = (uint32_t)total64;
  const uint32_t e3 = total - before - own, e2 = e3 + c4.w, e1 = e2 + c4.z,
                 e0 = e1 + c4.y;
  // The boundary bin: where the count from the top reaches K.
  const uint32_t need = min(K, total);
  if (need > 64u) return -1;  // more than one wave finishes (K above 64)
  uint32_t bstar = 0xffffffffu, bcount = 0;
  if (e3 < need && e3 + c4.w >= need) { bstar = 4 * tid + 3; bcount = c4.w; }
  else if (e2 < need && e2 + c4.z >= need) { bstar = 4 * tid + 2; bcount = c4.z; }
  else if (e1 < need && e1 + c4.y >= need) { bstar = 4 * tid + 1; bcount = c4.y; }
  else if (e0 < need && e0 + c4.x >= need) { bstar = 4 * tid; bcount = c4.x; }
  *(uint4 *)&excl[4 * tid] = make_uint4(e0, e1, e2, e3);
  if (bstar != 0xffffffffu) {
    s.sel_bin = bstar;
    s.hit = bcount > 64u ? 1u : 0u;
  }
  __syncthreads();
  if (s.hit) return -1;
  const uint32_t bs = need ? s.sel_bin : 1024u;
  // Items of the kept bins, grouped by bin in rank order of the bins.
#pragma unroll
  for (int k = 0; k < PER; ++k)
    if (((valid >> k) & 1) && bins[k] >= bs) {
      const uint32_t pos = excl[bins[k]] + atomicAdd(&fill[bins[k]], 1u);
      seg[pos] = ((uint64_t)(uint32_t)v[k] << 32) | (uint32_t)~(uint32_t)(v[k] >> 32);
    }
  __syncthreads();
  const uint32_t nsel = need ? excl[bs] + fill[bs] : 0u;
  if (tid < nsel) {
    const uint64_t me = seg[tid];
    const uint32_t b = bin_of((uint32_t)(me >> 32));
    const uint32_t e = excl[b], cnt = fill[b];
    uint32_t rank = e;
    for (uint32_t j = e; j < e + cnt; ++j) rank += seg[j] > me ? 1u : 0u;
    if (rank < need) {
      m.key[rank] = (uint32_t)(me >> 32);
      m.id[rank] = ~(uint32_t)me;
    }
  }
  __syncthreads();
  return (int)need;
}

// The last steps of a row with at most 64 items left, s.merge.key/id[0, n)
// in (key desc, id asc) order (rank_select), by one wave in registers. Rank
// order gives the top-k cut and the walk of top-p (sampling.metal:585-650);
// sorting the kept items by id gives the draw's order and the kept outputs
// (sampling.metal:700-829). The results equal wave_merge's.
__device__ __forceinline__ void wave_finish(const SampleLaunch &a, const RowParams &rp,
                                            uint32_t row, const Lds &s, uint32_t n,
                                            float maximum, float u, uint32_t draft) {
  const MergeLds &m = s.merge;
  const uint32_t lane = lane_id();
  const uint32_t key = lane < n ? m.key[lane] : 0u;
  const uint32_t id = lane < n ? m.id[lane] : kNoToken;
  const uint32_t n2 = min(rp.top_k, n);
  const bool in2 = lane < n2;
  const float w = in2 ? weight_of(key_logit(key), maximum, rp.inv_t) : 0.0f;
  const uint64_t wq = quantize(w);
  uint32_t n3 = n2;
  if (rp.flags & kRowTopP) {
    const uint64_t incl = wave_incl_scan_u64(wq);
    const uint64_t mass2 = readlane_u64(incl, 63);
    if (mass2) {
      const uint64_t nucleus = floor_mul(mass2, rp.top_p);
      const uint64_t hm = ballot(in2 && incl - wq <= nucleus && incl > nucleus);
      if (hm) n3 = (uint32_t)__builtin_ctzll(hm) + 1;
    }
  }
  const bool kept = lane < n3;
  const uint64_t mass3 = wave_sum_u64(kept ? wq : 0);
  const double scale = (double)mass3 * 0x1p-44;
  const bool drafted = draft != kNoToken;
  uint64_t d = kept ? wq : 0;
  if (drafted) {
    float q = 0.0f;
    for (int j = 15; j >= 0; --j) q = s.cids[j] == id ? s.cprobs[j] : q;
    const uint64_t r = kept ? residual_of(wq, mass3, q) : 0;
    if (ballot(r > 0)) d = r;
  }
  const uint64_t fm = ballot(drafted && kept && id == draft);
  const float fw = u2f(readlane_u32(f2u(w), fm ? (int)__builtin_ctzll(fm) : 0));
  // Id order of the kept items, each carrying the lane of its rank (ids are
  // below 2^19, so id and lane share 32 bits).
  uint32_t e = kept ? (id << 6) | lane : 0xffffffffu;
  e = wave_sort_asc_u32(e);
  const uint32_t src = e & 63u, iid = e >> 6;
  const uint64_t dq = shfl_u64(d, (int)src);
  const float wi = __shfl(w, (int)src, kWave);
  if (a.out_kept_ids && kept && lane < a.kept_cap) {
    a.out_kept_ids[(uint64_t)row * a.kept_cap + lane] = iid;
    a.out_kept_probs[(uint64_t)row * a.kept_cap + lane] =
        mass3 ? (float)((double)wi / scale) : 0.0f;
  }
  if (mass3 == 0) {
    if (lane == 0) write_result(a, row, kNoToken, 0.0f, n3);
    return;
  }
  const uint64_t dd = kept ? dq : 0ull;
  const uint64_t incl = wave_incl_scan_u64(dd);
  const uint64_t total = readlane_u64(incl, 63);
  uint64_t target = floor_mul(total, u);
  if (target >= total) target = total - 1;
  const uint64_t hm = ballot(kept && incl - dd <= target && incl > target);
  const uint32_t token = hm ? readlane_u32(iid, (int)__builtin_ctzll(hm)) : kNoToken;
  if (lane == 0)
    write_result(a, row, token, drafted && fm ? (float)((double)fw / scale) : 0.0f, n3);
}

// The general merge of a row for merge_small_kernel, out of line so that
// its register pressure stays out of the fast path's schedule. A called
// function cannot reach the kernel's arguments (its kernel-argument segment
// pointer is null), so the kernel copies the launch record into LDS first;
// the function works in the kernel's LDS record.
#if JF_IN(2)
__shared__ Lds g_small_lds;
__shared__ SampleLaunch g_small_launch;
template <int DT>
__device__ __noinline__ void merge_small_general(uint32_t row) {
  const SampleLaunch &a = g_small_launch;
  const RowParams rp = a.params[row];
  merge_sampled<DT>(a, rp, row, g_small_lds);
}
#endif

// The arguments the first loads need lead the signature (14 dwords, no
// padding): the hardware preloads them into scalar registers at wave launch
// (14 of its 16 user registers; the argument segment's address takes two).
// They repeat fields of `a` (drafted_rows is 0 when there are no drafts);
// bit 31 of `chunks_bits` says the row's draft is addressed through its
// record (the chunk count below it), so that no later argument is read
// from memory at the row's start.
#if JF_IN(2)
// SPEC: speculatively fetched list slots a thread. 10 gives floor(2560 / S)
// slots a chunk (134 at 19 chunks); 20 gives floor(5120 / S) (165 at 31
// chunks), for vocabularies past 163,840 tokens whose cut rows have no
// min-p floor (their lists average about 75 candidates and reach 130).
template <int DT, int SPEC>
__global__ __launch_bounds__(kThreads) void merge_small_kernel(
    const BlockHeader *headers, const uint64_t *cands, const RowParams *params,
    const float *uniforms, const uint32_t *uniform_index, uint32_t chunks_bits,
    uint32_t uniform_offset, uint32_t uniform_stride, uint32_t drafted_rows, SampleLaunch a) {
  Lds &s = g_small_lds;
  const uint32_t row = blockIdx.x, tid = threadIdx.x;
  const uint32_t S = chunks_bits & 0x7fffffffu;
  const bool row_indexed = (chunks_bits >> 31) != 0;
  // Every address of the row, computed once and held in vector registers:
  // the general path's register pressure would otherwise have the compiler
  // reload (and wait for) kernel arguments between the loads below. A load
  // with nothing to read targets the row's first chunk summary instead (its
  // value is ignored), so no load sits in a branch.
  typedef __attribute__((address_space(1))) const u32x4 GlobalU32x4;
  typedef __attribute__((address_space(1))) const uint64_t GlobalU64;
  typedef __attribute__((address_space(1))) const uint32_t GlobalU32;
  typedef __attribute__((address_space(1))) const float GlobalF32;
  const bool has_draft = row < drafted_rows;
  const bool has_index = uniform_index != nullptr, has_uniform = uniforms != nullptr;
  const BlockHeader *hrow = headers + (uint64_t)row * S;
  uint64_t hbase = (uint64_t)(hrow + (tid < S ? tid : 0u));
  uint64_t cbase = (uint64_t)(cands + (uint64_t)row * S * kBlockCandidates);
  uint64_t uaddr = has_index     ? (uint64_t)(uniform_index + row)
                   : has_uniform ? (uint64_t)(uniforms + uniform_offset + (uint64_t)row * uniform_stride)
                                 : (uint64_t)hrow;
  uint64_t ubase = has_uniform ? (uint64_t)uniforms : (uint64_t)hrow;
  uint64_t daddr = (uint64_t)hrow, qaddr = (uint64_t)hrow, paddr = (uint64_t)hrow;
  if (has_draft) {
    daddr = (uint64_t)(a.draft_tokens + row);
    qaddr = (uint64_t)(a.cand_ids + (uint64_t)row * 16 + (tid & 15));
    paddr = (uint64_t)(a.cand_probs + (uint64_t)row * 16 + (tid & 15));
  }
  uint64_t pbase = (uint64_t)(params + row);
  asm volatile("" : "+v"(hbase), "+v"(cbase), "+v"(uaddr), "+v"(ubase), "+v"(daddr),
               "+v"(qaddr), "+v"(paddr), "+s"(pbase));
  // Every load of the row, before any wait: the uniform (or its index), the
  // policy, the chunk summaries, the first P slots of every chunk's list,
  // the draft token and its 16 candidates.
  uint32_t ubits = *(GlobalU32 *)uaddr;
  const RowParams prec = load_row_policy((const RowParams *)pbase);
  // BlockHeader: maximum, count, admitted, overflow | best_value, best_id,
  // floor_key, reserved.
  const u32x4 h0 = ((GlobalU32x4 *)hbase)[0], h1 = ((GlobalU32x4 *)hbase)[1];
  constexpr uint32_t kSlots = SPEC * kThreads;
  // P = floor(kSlots / S) slots a chunk (at most a list's capacity), the
  // slots left over to the last chunk: slot i of the fetch is item i - c P
  // of chunk c = min(i / P, S - 1), read within the chunk's list. i / P as
  // the high word of i * ceil(2^32 / P), exact for i P < 2^32.
  const uint32_t P = min(kSlots / S, (uint32_t)kBlockCandidates);
  const uint32_t last_cap = min(kSlots - (S - 1) * P, (uint32_t)kBlockCandidates);
  const uint32_t pinv = (uint32_t)((0xffffffffull + P) / P);
  auto chunk_of = [&](uint32_t i) { return min(__umulhi(i, pinv), S - 1); };
  uint64_t sv[SPEC];
#pragma unroll
  for (int k = 0; k < SPEC; ++k) {
    const uint32_t i = tid + k * kThreads, c = chunk_of(i);
    const uint32_t j = min(i - c * P, (uint32_t)kBlockCandidates - 1);
    sv[k] = ((GlobalU64 *)cbase)[(uint64_t)c * kBlockCandidates + j];
  }
  const uint32_t draft_raw = *(GlobalU32 *)daddr;
  const uint32_t cid_raw = *(GlobalU32 *)qaddr;
  const float cpr_raw = *(GlobalF32 *)paddr;
  // A uniform through an index: its second load, once the index is in.
  if (has_index) {
    uint64_t a2 = ubase + (uint64_t)ubits * sizeof(float);
    asm volatile("" : "+v"(a2));
    ubits = *(GlobalU32 *)a2;
  }
  uint32_t draft = has_draft ? draft_raw : kNoToken;
  uint32_t cid = has_draft && tid < 16 ? cid_raw : kNoToken;
  float cpr = has_draft && tid < 16 ? cpr_raw : 0.0f;
  const bool hv = tid < S;
  const float hmax = hv ? u2f(h0.x) : -3.402823466e38f;
  const float hbest = hv ? u2f(h1.x) : -__builtin_inff();
  const uint32_t hcount = hv ? h0.y : 0u, hadm = hv ? h0.z : 0u, hovf = hv ? h0.w : 0u,
                 hfloor = hv ? h1.z : 0u, hbid = hv ? h1.y : kNoToken;
  if (tid >= 64) {
    // Waves 1..3, idle until the summaries' barrier, read the launch
    // record's output fields into the scalar cache, where wave 0's reads at
    // the end of the row then find them (a read there from memory would be
    // a round trip on the row's critical path).
    const void *o0 = a.out_tokens, *o1 = a.out_draft, *o2 = a.out_kept_counts,
               *o3 = a.out_kept_ids, *o4 = a.out_kept_probs;
    const uint32_t o5 = a.kept_cap;
    asm volatile("" ::"s"(o0), "s"(o1), "s"(o2), "s"(o3), "s"(o4), "s"(o5));
  }
  const float u = u2f(ubits);
  for (uint32_t b = tid; b < 1024; b += kThreads) {
    s.merge.bins[b] = 0;
    s.merge.key[1024 + b] = 0;
  }
  const RowParams rp = prec;
  if (row_indexed) {
    // Drafts addressed through the row's record (a batch of verify lanes):
    // their loads wait for the policy (the launch passed drafted_rows 0).
    draft = row_draft(a, rp);
    if (draft != kNoToken && tid < 16) {
      cid = a.cand_ids[(uint64_t)rp.cand_index * 16 + tid];
      cpr = a.cand_probs[(uint64_t)rp.cand_index * 16 + tid];
    }
  }
  if (uncut_row(rp)) {
    // The uncut kernel draws it.
    if (tid == 0) a.states[row].stage = kStageDone;
    return;
  }

  if (!(rp.flags & kRowSampled)) {
    // Greedy: the largest chunk best, the lowest id among equals.
    if (tid < 64) {
      float bv = hbest;
      uint32_t bi = hbid;
      wave_argmax(bv, bi);
      if (tid == 0) write_result(a, row, bi, 0.0f, 0);
    }
    return;
  }
  // The chunk summaries (wave 0): the row maximum, admission, overflow, the
  // top-k floor (the K-th key is at least every chunk's floor) and whether
  // some list is longer than its fetched slots.
  // Also each chunk's offset among the candidates of the chunks whose
  // maximum reaches the row's threshold (hoff; the others hold none at or
  // above it), for a compact refetch.
  if (tid < 64) {
    const float mx = wave_max_f32(hmax);
    const bool long_list = hv && hcount > (tid + 1 == S ? last_cap : P);
    const uint32_t adm = wave_max_u32(hadm), ovf = wave_max_u32(hovf),
                   flr = wave_max_u32(hfloor), longer = ballot(long_list) ? 1u : 0u;
    const uint32_t wthr =
        max((prec.flags & kRowMinP) ? logit_key(__builtin_fminf(mx + prec.minp_offset, mx)) : 0u,
            flr);
    const bool use = hv && logit_key(hmax) >= wthr;
    const uint32_t incl = wave_incl_scan_u32(use ? hcount : 0u);
    if (tid < S) {
      s.hcnt[tid] = hcount;
      s.hoff[tid + 1] = incl;
    }
    if (tid == 0) {
      s.hoff[0] = 0;
      s.row_max = mx;
      s.row_admitted = adm;
      s.row_overflow = ovf;
      s.row_floor = flr;
      s.row_long = longer;
    }
  }
  if (tid < 16) {
    s.cids[tid] = draft != kNoToken ? cid : kNoToken;
    s.cprobs[tid] = draft != kNoToken ? cpr : 0.0f;
  }
  __syncthreads();
  const float maximum = s.row_max;
  if (s.row_admitted == 0 || maximum == __builtin_inff()) {
    if (tid == 0) write_result(a, row, kNoToken, 0.0f, 0);
    return;
  }
  uint32_t thr = (rp.flags & kRowMinP)
                     ? logit_key(__builtin_fminf(maximum + rp.minp_offset, maximum))
                     : 0u;
  thr = max(thr, s.row_floor);
  const uint32_t K = rp.top_k;
  const uint32_t n_all = s.hoff[S];
  if (!s.row_overflow && thr > kLowestKey && (!s.row_long || n_all <= kSlots)) {
    uint32_t valid = 0;
    if (!s.row_long) {
#pragma unroll
      for (int k = 0; k < SPEC; ++k) {
        const uint32_t i = tid + k * kThreads, c = chunk_of(i);
        if (i - c * P < s.hcnt[c] && (uint32_t)sv[k] >= thr) valid |= 1u << k;
      }
    } else {
      // A list longer than its fetched slots, but every candidate at or
      // above the threshold fits the registers: item i = tid + k * threads
      // of the chunks that reach the threshold, its chunk the last c with
      // hoff[c] <= i (binary searches, all items at once), fetched now.
      uint32_t cc[SPEC];
#pragma unroll
      for (int k = 0; k < SPEC; ++k) cc[k] = 0;
      for (uint32_t step = kMaxChunks / 2; step; step >>= 1) {
#pragma unroll
        for (int k = 0; k < SPEC; ++k) {
          const uint32_t i = tid + k * kThreads;
          if (cc[k] + step < S && s.hoff[cc[k] + step] <= i) cc[k] += step;
        }
      }
#pragma unroll
      for (int k = 0; k < SPEC; ++k) {
        const uint32_t i = tid + k * kThreads;
        sv[k] = i < n_all ? ((GlobalU64 *)cbase)[(uint64_t)cc[k] * kBlockCandidates +
                                                 (i - s.hoff[cc[k]])]
                          : 0ull;
      }
#pragma unroll
      for (int k = 0; k < SPEC; ++k) {
        const uint32_t i = tid + k * kThreads;
        if (i < n_all && (uint32_t)sv[k] >= thr) valid |= 1u << k;
      }
    }
    const int got = rank_select(sv, valid, thr, K, maximum, s);
    if (got >= 0) {
      if (tid < 64) wave_finish(a, rp, row, s, (uint32_t)got, maximum, u, draft);
      return;
    }
    __syncthreads();
  }
  // What the speculative fetch does not cover: the general merge. The
  // launch record is copied word by word from the argument segment here
  // (one word a thread), so no field of it stays live from the kernel's
  // entry (the compiler otherwise kept some in private memory for this).
  {
    const uint32_t *src = reinterpret_cast<const uint32_t *>(&a);
    uint32_t *dst = reinterpret_cast<uint32_t *>(&g_small_launch);
    for (uint32_t k = tid; k < sizeof(SampleLaunch) / 4; k += kThreads) dst[k] = src[k];
  }
  __syncthreads();
  merge_small_general<DT>(row);
}
#endif

// ---- multi-pass stages ---------------------------------------------------

// A drafted row's dense q over this thread's tokens of a chunk, in the
// order of the chunk's logits; 16-byte loads when the rows are aligned.
template <int DT>
__device__ __forceinline__ void load_dense_q(const SampleLaunch &a, const RowParams &rp,
                                             uint32_t chunk,
                                             float (&qv)[Geo<DT>::TPL]) {
  constexpr int VEC = Geo<DT>::VEC, SLAB = Geo<DT>::SLAB, LOADS = Geo<DT>::LOADS;
  constexpr uint32_t CHUNK = Geo<DT>::CHUNK;
  const uint32_t lane_base = chunk * CHUNK + threadIdx.x * VEC;
  const float *q = a.dense_q + (uint64_t)rp.cand_index * a.q_stride;
  if (a.q_aligned && chunk * CHUNK + CHUNK <= a.vocabulary) {
#pragma unroll
    for (int j = 0; j < LOADS; ++j)
#pragma unroll
      for (int h = 0; h < VEC / 4; ++h) {
        const float4 f = *reinterpret_cast<const float4 *>(q + lane_base + j * SLAB + 4 * h);
        qv[j * VEC + 4 * h + 0] = f.x;
        qv[j * VEC + 4 * h + 1] = f.y;
        qv[j * VEC + 4 * h + 2] = f.z;
        qv[j * VEC + 4 * h + 3] = f.w;
      }
  } else {
#pragma unroll
    for (int j = 0; j < LOADS; ++j)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const uint32_t t = lane_base + j * SLAB + e;
        qv[j * VEC + e] = t < a.vocabulary ? q[t] : 0.0f;
      }
  }
}

// The draw inside chunk `c` of a row: the first member, in id order, whose
// running weight (the residual weight when `residual`) passes `within`
// (sampling.metal:790-829 walks the whole row the same way). Members are the
// admitted tokens at or above `thr_key` and at or before the kept boundary
// (bkey, bid). Every thread of the block calls it; every thread gets the
// token.
template <int DT, class L>
__device__ __forceinline__ uint32_t walk_chunk(const SampleLaunch &a, const RowParams &rp,
                                               uint32_t row, uint32_t c, float M,
                                               uint32_t thr_key, uint32_t bkey, uint32_t bid,
                                               bool residual, uint64_t mass3,
                                               uint64_t within, L &s) {
  constexpr int VEC = Geo<DT>::VEC, TPL = Geo<DT>::TPL, SLAB = Geo<DT>::SLAB,
                LOADS = Geo<DT>::LOADS;
  constexpr uint32_t CHUNK = Geo<DT>::CHUNK;
  // A dense draft row is requested ahead of the chunk's logits.
  const bool dq = residual && a.dense_q;
  float qv[TPL];
  if (dq) load_dense_q<DT>(a, rp, c, qv);
  float xs[TPL];
  load_chunk<DT>(a, rp, row, c, s, xs);
  const uint32_t lane_base = c * CHUNK + threadIdx.x * VEC;
  const float inv_t = rp.inv_t;
  auto tok = [&](int i) -> uint32_t {
    return lane_base + (i / VEC) * SLAB + (i % VEC);
  };
  auto d_of = [&](float v, float q, uint32_t t) -> uint64_t {
    if (v != v) return 0;
    const uint32_t k = logit_key(v);
    if (k < thr_key || !at_or_before(k, t, bkey, bid)) return 0;
    const uint64_t wq = quantize(weight_of(v, M, inv_t));
    return residual ? residual_of(wq, mass3, dq ? q : draft_q(a, rp, t, s)) : wq;
  };
  uint64_t lsum[LOADS], offs[LOADS];
#pragma unroll
  for (int j = 0; j < LOADS; ++j) {
    lsum[j] = 0;
#pragma unroll
    for (int e = 0; e < VEC; ++e)
      lsum[j] += d_of(xs[j * VEC + e], dq ? qv[j * VEC + e] : 0.0f, tok(j * VEC + e));
  }
  if (threadIdx.x == 0) s.hit = kNoToken;
  order_offsets<LOADS>(lsum, offs, s);
  // The load whose range holds `within` recomputes its weights: its VEC
  // values are picked out first, so only VEC weights are live at once.
  int jsel = -1;
  uint64_t acc = 0;
#pragma unroll
  for (int j = 0; j < LOADS; ++j)
    if (offs[j] <= within && offs[j] + lsum[j] > within) {
      jsel = j;
      acc = offs[j];
    }
  if (jsel >= 0) {
    float xv[VEC], qq[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) xv[e] = qq[e] = 0.0f;
#pragma unroll
    for (int j = 0; j < LOADS; ++j)
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        if (j == jsel) {
          xv[e] = xs[j * VEC + e];
          if (dq) qq[e] = qv[j * VEC + e];
        }
    const uint32_t tbase = lane_base + (uint32_t)jsel * SLAB;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const uint32_t t = tbase + e;
      const uint64_t d = d_of(xv[e], qq[e], t);
      if (d && acc + d > within) {
        s.hit = t;
        break;
      }
      acc += d;
    }
  }
  __syncthreads();
  return s.hit;
}

// The stage kernel is compiled once per class of stages, so each launch
// carries only its stage's code and registers.
#if JF_IN(3)
template <int DT, int CLS>
__global__ __launch_bounds__(kThreads) void stage_kernel(SampleLaunch a) {
  constexpr int VEC = Geo<DT>::VEC, TPL = Geo<DT>::TPL, SLAB = Geo<DT>::SLAB,
                LOADS = Geo<DT>::LOADS;
  constexpr uint32_t CHUNK = Geo<DT>::CHUNK;
  constexpr uint32_t VMASK = (1u << VEC) - 1u;
  __shared__ Lds s;
  const uint32_t S = a.chunks;
  const uint32_t row = blockIdx.x / S, chunk = blockIdx.x % S;
  const uint32_t tid = threadIdx.x;
  const uint32_t stage = a.stage;
  if (stage_class(stage) != CLS) return;
  // The row's parameters are requested with its state, in one round trip.
  const RowParams rp = a.params[row];
  RowState st = a.states[row];
  if (st.stage != stage) return;
  const bool single = stage == kStageTopKLocate || stage == kStageTopPLocate;
  if (single && chunk != st.chunk) return;
  // The draw stage's dense q is requested ahead of the chunk's logits.
  float qv[CLS == kClsDraw ? TPL : 1];
  if constexpr (CLS == kClsDraw)
    if (a.dense_q) load_dense_q<DT>(a, rp, chunk, qv);
  float xs[TPL];
  load_chunk<DT>(a, rp, row, chunk, s, xs);
  stage_candidates(a, rp, s);
  const uint32_t lane_base = chunk * CHUNK + tid * VEC;
  const float M = st.maximum, inv_t = rp.inv_t;
  // Members: admitted (non-NaN), at or above the min-p floor, at or before
  // the kept boundary.
  uint64_t mem = 0;
#pragma unroll
  for (int i = 0; i < TPL; ++i) {
    const float v = xs[i];
    if (v != v) continue;
    const uint32_t k = logit_key(v);
    const uint32_t t = lane_base + (i / VEC) * SLAB + (i % VEC);
    if (k >= st.thr_key && at_or_before(k, t, st.bkey, st.bid)) mem |= 1ull << i;
  }
  StagePartial *part = a.partials + (uint64_t)row * S + chunk;
  const uint32_t draft = row_draft(a, rp);

  auto wq_of = [&](int i) -> uint64_t {
    return quantize(weight_of(xs[i], M, inv_t));
  };
  auto tok_of = [&](int i) -> uint32_t {
    return lane_base + (i / VEC) * SLAB + (i % VEC);
  };
  // The `within`-th (0-based) token with a set bit, in id order; returns
  // its token in every thread.
  auto locate = [&](uint64_t bits, uint64_t within) -> uint32_t {
    if (tid == 0) s.hit = kNoToken;
    uint32_t nb[LOADS], off[LOADS];
#pragma unroll
    for (int j = 0; j < LOADS; ++j) nb[j] = __popc((uint32_t)(bits >> (j * VEC)) & VMASK);
    order_offsets<LOADS>(nb, off, s);
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      uint64_t idx = off[j];
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        if ((bits >> (j * VEC + e)) & 1u) {
          if (idx == within) s.hit = tok_of(j * VEC + e);
          ++idx;
        }
    }
    __syncthreads();
    return s.hit;
  };

  switch (stage) {
    case kStageCount1: {
      if constexpr (CLS == kClsCount) {
      const uint32_t c = block_sum_u32(__popcll(mem), s);
      if (tid == 0) st_dev(&part->v[0], (uint64_t)c);
      }
      break;
    }
    case kStageTopK3: case kStageTopK3 + 1: case kStageTopK3 + 2: case kStageTopK0:
    case kStageTopP3: case kStageTopP3 + 1: case kStageTopP3 + 2: case kStageTopP0: {
      if constexpr (CLS == kClsDigits) {
      const bool by_mass = stage >= kStageTopP3;
      const int d = by_mass ? (int)(kStageTopP0 - stage) : (int)(kStageTopK0 - stage);
      s.hist[tid] = 0;
      __syncthreads();
#pragma unroll
      for (int i = 0; i < TPL; ++i) {
        if (!((mem >> i) & 1)) continue;
        const uint32_t k = logit_key(xs[i]);
        if ((k & st.pmask) != st.prefix) continue;
        const uint64_t v = by_mass ? wq_of(i) : 1ull;
        if (v) atomicAdd((unsigned long long *)&s.hist[(k >> (8 * d)) & 255u],
                         (unsigned long long)v);
      }
      __syncthreads();
      st_dev(&part->v[tid], s.hist[tid]);
      }
      break;
    }
    case kStageTopKTie:
    case kStageTopPTie: {
      if constexpr (CLS == kClsTie) {
      uint32_t c = 0;
#pragma unroll
      for (int i = 0; i < TPL; ++i)
        c += ((mem >> i) & 1) && logit_key(xs[i]) == st.tie_key;
      c = block_sum_u32(c, s);
      if (tid == 0) st_dev(&part->v[0], (uint64_t)c);
      }
      break;
    }
    case kStageTopKLocate:
    case kStageTopPLocate:
      break;
    case kStageMass2:
    case kStageMass3:
    case kStageKeptCount: {
      if constexpr (CLS == kClsMass) {
      uint64_t sum = 0;
      uint32_t c = 0;
      if (tid == 0) {
        s.found_w = 0.0f;
        s.u32a = 0;
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < TPL; ++i)
        if ((mem >> i) & 1) {
          sum += wq_of(i);
          ++c;
        }
      if (stage == kStageMass3 && draft != kNoToken) {
#pragma unroll
        for (int i = 0; i < TPL; ++i)
          if (((mem >> i) & 1) && tok_of(i) == draft) {
            s.found_w = weight_of(xs[i], M, inv_t);
            s.u32a = 1;
          }
      }
      sum = block_sum_u64(sum, s);
      c = block_sum_u32(c, s);
      if (tid == 0) {
        st_dev(&part->v[0], stage == kStageKeptCount ? (uint64_t)c : sum);
        st_dev(&part->v[1], (uint64_t)s.u32a);
        st_dev(&part->v[2], (uint64_t)__float_as_uint(s.found_w));
      }
      }
      break;
    }
    case kStageDraw: {
      if constexpr (CLS == kClsDraw) {
      uint64_t dsum = 0, wsum = 0;
      uint32_t any = 0;
#pragma unroll
      for (int i = 0; i < TPL; ++i)
        if ((mem >> i) & 1) {
          const uint64_t wq = wq_of(i);
          wsum += wq;
          if (st.drafted) {
            const float q = a.dense_q ? qv[i] : draft_q(a, rp, tok_of(i), s);
            const uint64_t d = residual_of(wq, st.mass3, q);
            dsum += d;
            any |= d > 0;
          }
        }
      dsum = block_sum_u64(dsum, s);
      wsum = block_sum_u64(wsum, s);
      any = block_max_u32(any, s);
      if (tid == 0) {
        st_dev(&part->v[0], dsum);
        st_dev(&part->v[1], wsum);
        st_dev(&part->v[2], (uint64_t)any);
      }
      }
      break;
    }
    case kStageKeptWrite: {
      if constexpr (CLS == kClsKeptWrite) {
      // Offset of this chunk: the kept counts of the chunks before it.
      uint64_t off = 0;
      for (uint32_t c = 0; c < chunk; ++c) off += a.partials[(uint64_t)row * S + c].v[0];
      const double scale = (double)st.mass3 * 0x1p-44;
      uint32_t nb[LOADS], offs[LOADS];
#pragma unroll
      for (int j = 0; j < LOADS; ++j) nb[j] = __popc((uint32_t)(mem >> (j * VEC)) & VMASK);
      order_offsets<LOADS>(nb, offs, s);
#pragma unroll
      for (int j = 0; j < LOADS; ++j) {
        uint64_t idx = off + offs[j];
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          if ((mem >> (j * VEC + e)) & 1u) {
            if (idx < a.kept_cap) {
              const int i = j * VEC + e;
              a.out_kept_ids[(uint64_t)row * a.kept_cap + idx] = tok_of(i);
              a.out_kept_probs[(uint64_t)row * a.kept_cap + idx] =
                  st.mass3 ? (float)((double)weight_of(xs[i], M, inv_t) / scale)
                           : 0.0f;
            }
            ++idx;
          }
      }
      }
      break;
    }
    default:
      break;
  }

  if constexpr (CLS == kClsLocate) {
  if (stage == kStageTopKLocate || stage == kStageTopPLocate) {
    // The within-th tie of this chunk closes the kept set.
    uint64_t ties = 0;
#pragma unroll
    for (int i = 0; i < TPL; ++i)
      if (((mem >> i) & 1) && logit_key(xs[i]) == st.tie_key) ties |= 1ull << i;
    const uint32_t id = locate(ties, st.within);
    if (tid == 0) {
      RowState &ns = a.states[row];
      ns.bkey = st.tie_key;
      ns.bid = id;
      ns.prefix = 0;
      ns.pmask = 0;
      if (stage == kStageTopKLocate && (rp.flags & kRowTopP))
        ns.stage = kStageMass2;
      else
        ns.stage = kStageMass3;
    }
    return;
  }
  }
  if (!arrive_last(a.counters + row, S, s)) return;

  // Finalize the stage for this row. The chunks' partials are read with
  // every load in flight at once: a runtime loop of device-coherent loads
  // would wait a round trip per chunk.
  const StagePartial *parts = a.partials + (uint64_t)row * S;
  if constexpr (CLS == kClsDigits) {
  if ((stage >= kStageTopK3 && stage <= kStageTopK0) ||
      (stage >= kStageTopP3 && stage <= kStageTopP0)) {
    uint64_t h = 0;
    for (uint32_t c0 = 0; c0 < S; c0 += 8) {
      uint64_t t[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) t[k] = ld_dev(&parts[min(c0 + k, S - 1)].v[tid]);
#pragma unroll
      for (int k = 0; k < 8; ++k) h += c0 + k < S ? t[k] : 0ull;
    }
    s.hist[tid] = h;
    __syncthreads();
    crossing_bin(s, st.remaining);
    if (tid == 0) {
      const bool by_mass = stage >= kStageTopP3;
      const int d = by_mass ? (int)(kStageTopP0 - stage) : (int)(kStageTopK0 - stage);
      RowState &ns = a.states[row];
      ns.remaining = st.remaining - s.sel_excl;
      ns.prefix = st.prefix | (s.sel_bin << (8 * d));
      ns.pmask = st.pmask | (255u << (8 * d));
      if (d > 0) {
        ns.stage = stage + 1;
      } else {
        ns.tie_key = ns.prefix;
        if (by_mass) {
          // Tied tokens weigh the same; keep as many as reach the mass.
          const uint64_t wk = quantize(weight_of(key_logit(ns.prefix), M, inv_t));
          ns.remaining = (ns.remaining + wk - 1) / wk;
          ns.stage = kStageTopPTie;
        } else {
          ns.stage = kStageTopKTie;
        }
      }
    }
    return;
  }
  }
  // The other stages: wave 0, one lane per chunk (S <= 64).
  if (tid >= 64) return;
  const bool in = tid < S;
  const StagePartial *pl = parts + min(tid, S - 1);
  auto lane_v = [&](int f) -> uint64_t {
    const uint64_t v = ld_dev(&pl->v[f]);
    return in ? v : 0ull;
  };
  // The first chunk whose running total passes `target` (strictly when
  // `strict`), and the total before it; the last chunk and the whole total
  // when none does.
  auto pick = [&](uint64_t v, uint64_t target, bool strict, uint32_t &chunk_out,
                  uint64_t &before) {
    const uint64_t incl = wave_incl_scan_u64(v);
    const uint64_t m = ballot(in && (strict ? incl > target : incl >= target));
    if (m) {
      const int c = (int)__builtin_ctzll(m);
      chunk_out = (uint32_t)c;
      before = readlane_u64(incl - v, c);
    } else {
      chunk_out = S - 1;
      before = readlane_u64(incl, 63);
    }
  };
  RowState &ns = a.states[row];
  const bool lead = tid == 0;
  switch (stage) {
    case kStageCount1: {
      if constexpr (CLS == kClsCount) {
      const uint64_t n1 = wave_sum_u64(lane_v(0));
      if (lead) {
        ns.n1 = n1;
        if (rp.top_k < n1) {
          ns.stage = kStageTopK3;
          ns.remaining = rp.top_k;
        } else {
          ns.stage = (rp.flags & kRowTopP) ? kStageMass2 : kStageMass3;
        }
      }
      }
      break;
    }
    case kStageTopKTie:
    case kStageTopPTie: {
      if constexpr (CLS == kClsTie) {
      uint32_t c;
      uint64_t cum;
      pick(lane_v(0), st.remaining, false, c, cum);
      if (lead) {
        ns.chunk = c;
        ns.within = st.remaining - cum - 1;
        ns.stage = stage == kStageTopKTie ? kStageTopKLocate : kStageTopPLocate;
      }
      }
      break;
    }
    case kStageMass2: {
      if constexpr (CLS == kClsMass) {
      const uint64_t mass = wave_sum_u64(lane_v(0));
      if (lead) {
        ns.mass2 = mass;
        if (mass == 0) {
          ns.stage = kStageMass3;
        } else {
          ns.nucleus = floor_mul(mass, rp.top_p);
          ns.remaining = ns.nucleus + 1;
          ns.prefix = 0;
          ns.pmask = 0;
          ns.stage = kStageTopP3;
        }
      }
      }
      break;
    }
    case kStageMass3: {
      if constexpr (CLS == kClsMass) {
      const uint64_t v0 = lane_v(0), v1 = lane_v(1), v2 = lane_v(2);
      const uint64_t mass = wave_sum_u64(v0);
      // The chunk holding the draft token reports its weight.
      const uint64_t fm = ballot(v1 != 0);
      const uint32_t fw = fm ? (uint32_t)readlane_u64(v2, 63 - __builtin_clzll(fm)) : 0u;
      uint32_t c = 0;
      uint64_t cum = 0, target = 0;
      const bool walk = mass != 0 && !st.drafted;
      if (walk) {
        // Without a draft the chunk masses already place the draw.
        target = floor_mul(mass, row_uniform(a, row));
        if (target >= mass) target = mass - 1;
        pick(v0, target, true, c, cum);
      }
      if (lead) {
        if (fm) ns.draft_w = __uint_as_float(fw);
        ns.mass3 = mass;
        if (mass == 0) {
          write_result(a, row, kNoToken, 0.0f, 0);
          ns.stage = a.out_kept_ids ? kStageKeptCount : kStageDone;
        } else if (st.drafted) {
          ns.stage = kStageDraw;
        } else {
          ns.residual = 0;
          ns.chunk = c;
          ns.within = target - cum;
          ns.target = target;
          ns.stage = kStageWalk;
        }
      }
      }
      break;
    }
    case kStageDraw: {
      if constexpr (CLS == kClsDraw) {
      const uint64_t v0 = lane_v(0), v1 = lane_v(1), v2 = lane_v(2);
      const bool residual = st.drafted && ballot(v2 != 0) != 0;
      const uint64_t v = residual ? v0 : v1;
      const uint64_t total = wave_sum_u64(v);
      uint64_t target = floor_mul(total, row_uniform(a, row));
      if (target >= total) target = total - 1;
      uint32_t c;
      uint64_t cum;
      pick(v, target, true, c, cum);
      if (lead) {
        ns.residual = residual ? 1u : 0u;
        ns.chunk = c;
        ns.within = target - cum;
        ns.target = target;
        ns.stage = kStageWalk;
      }
      }
      break;
    }
    case kStageKeptCount: {
      if constexpr (CLS == kClsMass) {
      const uint64_t kept = wave_sum_u64(lane_v(0));
      if (lead) {
        if (a.out_kept_counts) a.out_kept_counts[row] = (uint32_t)kept;
        ns.stage = kStageKeptWrite;
      }
      }
      break;
    }
    case kStageKeptWrite:
      if (lead) ns.stage = kStageDone;
      break;
    default:
      break;
  }
}
#endif

// The draw inside the chunk the row's last stage chose: one block per row.
#if JF_IN(3)
template <int DT>
__global__ __launch_bounds__(kThreads) void walk_kernel(SampleLaunch a) {
  __shared__ Lds s;
  const uint32_t row = blockIdx.x;
  const RowParams rp = a.params[row];
  const RowState st = a.states[row];
  if (st.stage != kStageWalk) return;
  stage_candidates(a, rp, s);
  const uint32_t hit = walk_chunk<DT>(a, rp, row, st.chunk, st.maximum, st.thr_key,
                                      st.bkey, st.bid, st.residual != 0, st.mass3,
                                      st.within, s);
  if (threadIdx.x == 0) {
    const double scale = (double)st.mass3 * 0x1p-44;
    write_result(a, row, hit,
                 st.drafted ? (float)((double)st.draft_w / scale) : 0.0f, 0);
    a.states[row].stage = a.out_kept_ids ? kStageKeptCount : kStageDone;
  }
}
#endif

// ---- rows that keep every admitted token -----------------------------------
//
// A sampled row with no min-p, top-k or top-p cut keeps every admitted token.
// The select pass left, per chunk, the chunk's maximum m_c, its admitted
// count and its exact fixed-point mass S_c against m_c (partials v[0]). The
// row's mass is W = sum of T_c = floor(S_c * r_c) with the rescale
// r_c = exp((m_c - M) / T) carried as R_c * 2^-s_c (chunk_scale: a 32-bit
// significand and a shift, relative precision 2^-32 at any offset), so the
// mass costs one read of the logits. One block per row draws: the chunk whose
// running T_c passes u * W, that chunk reloaded, and its first token (id
// order) whose running mass P has floor(P * r_c) past the remainder
// (sampling.metal:694-829 on these weights). A drafted row's blocks, one per
// chunk, sum the residual weights residual_of(floor(w * r_c), W, q) per slice;
// the row's last block draws from them, or plainly when no residual mass
// remains, and writes p(draft). Drafted rows with no penalty, mask or extra
// tokens (kRowLean) take that pass in residual_kernel, launched before, and
// their chunk 0 block here draws. Chunk 0's block writes the row's kept
// outputs, each probability w * r_c / W from the token's float weight.
// Greedy rows take the argmax of the chunk bests when no merge runs.
//
// Partial slots per (row, chunk): v[0] S_c; v[kDraftSlot] the draft token's
// float weight against m_c; v[kResidualSlot] the chunk's residual mass and
// v[kResidualSlot + 1 + g] its slices' (slice g = load g / kWaves of wave
// g % kWaves, 64 x VEC consecutive tokens, so g runs in id order).
struct __align__(16) UncutLds {
  PrepLds prep;
  uint64_t wj[kWaves][8];
  uint64_t wl[kWaves];
  uint32_t cids[16];
  float cprobs[16];
  float cmax[kMaxChunks];       // the row's chunk maxima
  uint64_t cscale[kMaxChunks];  // r_c, packed s_c << 32 | R_c
  uint64_t ctot[kMaxChunks];    // T_c
  uint32_t ccount[kMaxChunks];  // admitted (non-NaN) tokens per chunk
  uint64_t slices[kWaves * 8];  // one chunk's slice masses
  float row_max;
  uint64_t row_mass;
  uint32_t row_admitted;
  uint32_t row_kept;
  float pd;                     // p(draft)
  uint32_t residual;
  uint32_t last;
  uint32_t sel_bin;
  uint64_t sel_excl;
  uint32_t slice;
  uint64_t slice_within;
};

#if JF_IN(4)
constexpr uint32_t kDraftSlot = 40;
constexpr uint32_t kResidualSlot = 63;

// The reported probability of a token of float weight w (against its
// chunk's maximum) in a chunk of packed rescale s << 32 | R: w R 2^-s over the
// row mass W (units of 2^-44), in double; below FLT_MIN it reports 0, so no
// denormal conversion is involved.
__device__ __forceinline__ float uncut_probability(float w, uint64_t scale, uint64_t W) {
  if (!W) return 0.0f;
  const double r = __builtin_ldexp((double)(uint32_t)scale, -(int)(scale >> 32));
  const double p = ((double)w * r) / ((double)W * 0x1p-44);
  return p >= 0x1p-126 ? (float)p : 0.0f;
}

// The first kept_cap admitted tokens of the row in id order with their
// probabilities (chunk 0's block; block-uniform).
template <int DT>
__device__ __forceinline__ void uncut_kept(const SampleLaunch &a, const RowParams &rp, uint32_t row,
                           UncutLds &s, uint64_t W) {
  constexpr int TPL = Geo<DT>::TPL, VEC = Geo<DT>::VEC, LOADS = Geo<DT>::LOADS,
                SLAB = Geo<DT>::SLAB;
  constexpr uint32_t CHUNK = Geo<DT>::CHUNK;
  const uint32_t cap = a.kept_cap, tid = threadIdx.x;
  uint32_t *ids = a.out_kept_ids + (uint64_t)row * cap;
  float *probs = a.out_kept_probs + (uint64_t)row * cap;
  uint32_t written = 0;
  for (uint32_t c = 0; c < a.chunks && written < cap; ++c) {
    if (s.ccount[c] == 0) continue;
    float xs[TPL];
    load_chunk<DT>(a, rp, row, c, s, xs);
    const float mc = s.cmax[c];
    const uint64_t R = s.cscale[c];
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      uint32_t n = 0;
#pragma unroll
      for (int e = 0; e < VEC; ++e) n += xs[j * VEC + e] == xs[j * VEC + e];
      uint64_t total;
      uint32_t pos = written + (uint32_t)block_excl_scan_u64(n, s, &total);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float x = xs[j * VEC + e];
        if (x == x) {
          if (pos < cap) {
            ids[pos] = c * CHUNK + j * SLAB + tid * VEC + e;
            probs[pos] = uncut_probability(weight_of(x, mc, rp.inv_t), R, W);
          }
          ++pos;
        }
      }
      written += (uint32_t)total;
    }
  }
}

// The plain draw of an uncut row from its chunk masses (one block; block-
// uniform): the chunk, its reload together with its slice masses (which the
// select pass wrote), the slice, the token.
template <int DT>
__device__ __forceinline__ void uncut_draw(const SampleLaunch &a, const RowParams &rp,
                                           uint32_t row, UncutLds &s, uint64_t W, float u) {
  constexpr int TPL = Geo<DT>::TPL, VEC = Geo<DT>::VEC, LOADS = Geo<DT>::LOADS,
                SLAB = Geo<DT>::SLAB;
  constexpr uint32_t CHUNK = Geo<DT>::CHUNK, G = LOADS * kWaves;
  const uint32_t S = a.chunks, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (w == 0) {
    const bool in = lane < S;
    const uint64_t T = in ? s.ctot[lane] : 0ull;
    const uint64_t incl = wave_incl_scan_u64(T);
    uint64_t target = floor_mul(W, u);
    if (target >= W) target = W - 1;
    // incl at the last lane is W > target: some lane passes it.
    const uint32_t c = (uint32_t)__builtin_ctzll(ballot(in && incl > target));
    const uint64_t within = target - readlane_u64(incl - T, c);
    if (lane == 0) {
      s.sel_bin = c;
      // The running mass inside chunk c (against m_c) that the token's
      // prefix must pass: floor(P * r_c) > within <=> P > this.
      s.sel_excl = unscaled_bound(within, s.cscale[c]);
    }
  }
  __syncthreads();
  const uint32_t c = s.sel_bin;
  uint64_t vg = 0;
  if (w == 0 && lane < G) vg = a.partials[(uint64_t)row * S + c].v[1 + lane];
  float xs[TPL];
  load_chunk<DT>(a, rp, row, c, s, xs);
  if (w == 0) {
    uint64_t wi = s.sel_excl;
    const uint32_t gg = pick_slice(vg, G, wi);
    if (lane == 0) {
      s.slice = gg;
      s.slice_within = wi;
    }
  }
  __syncthreads();
  const uint32_t g = s.slice, jg = g / kWaves;
  if (w == g % kWaves) {
    const float mc = s.cmax[c];
    uint64_t q[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float x = 0.0f;
#pragma unroll
      for (int j = 0; j < LOADS; ++j) x = (uint32_t)j == jg ? xs[j * VEC + e] : x;
      q[e] = quantized_weight(x, mc, rp.inv_t);
    }
    uint32_t e_hit;
    if (lane == slice_hit<VEC>(q, s.slice_within, e_hit))
      write_result(a, row, c * CHUNK + jg * SLAB + tid * VEC + e_hit, s.pd, s.row_kept);
  }
}

struct __align__(16) LeanLds {
  uint32_t cids[16];
  float cprobs[16];
  uint64_t wl[kWaves];
  float mc;      // this chunk's maximum
  uint64_t rc;   // its rescale r_c, packed
  uint64_t W;    // the row's mass
  uint32_t ok;   // the row has mass to draw from
  uint32_t kept; // its admitted tokens
  // (drawing launches) every chunk's maximum, rescale and scaled mass T_c;
  // the finisher's gather: every chunk's slice residual masses, the draft
  // token's float weight, and whether a wait gave up
  float cmax[kMaxChunks];
  uint64_t cscale[kMaxChunks];
  uint64_t ctot[kMaxChunks];
  alignas(16) uint64_t fsl[kMaxChunks * 32];
  uint32_t dw;
  uint32_t fail;
};

// One wave: a row's chunk summaries (lane c < S holds chunk c's maximum m,
// rescale R against the row maximum M and scaled mass T), and W = sum T,
// the admitted and kept counts, as uncut_kernel computes them.
struct RowSums {
  float m, M;
  uint64_t R, T, W;
  uint32_t admitted, kept;
};
__device__ __forceinline__ RowSums row_sums_of(uint32_t S, float hm, uint32_t hadm,
                                               uint32_t hcnt, uint64_t hmass, float inv_t) {
  const bool in = lane_id() < S;
  RowSums r;
  r.m = in ? hm : -3.402823466e38f;
  r.M = wave_max_f32(r.m);
  r.R = in ? chunk_scale(r.m, r.M, inv_t) : kZeroScale;
  r.T = scale_by(in ? hmass : 0ull, r.R);
  r.W = wave_sum_u64(r.T);
  r.admitted = wave_sum_u32(in ? hadm : 0u);
  r.kept = wave_sum_u32(in ? hcnt : 0u);
  return r;
}
__device__ __forceinline__ RowSums row_sums(const SampleLaunch &a, uint32_t row, float inv_t) {
  const uint32_t S = a.chunks, at = lane_id() < S ? lane_id() : 0u;
  const BlockHeader *h = a.headers + (uint64_t)row * S + at;
  return row_sums_of(S, h->maximum, h->admitted, h->count,
                     a.partials[(uint64_t)row * S + at].v[0], inv_t);
}

// One wave: the plain draw of an uncut row (uncut_draw's): the chunk and
// slice that hold floor(u W) by the chunk masses and the slice masses the
// selection wrote, then the token inside the slice.
template <int DT, class L>
__device__ __forceinline__ void plain_draw_wave(const SampleLaunch &a, uint32_t row,
                                                uint32_t flags, float inv_t, const RowSums &r,
                                                float u, float pd, const L &s) {
  constexpr uint32_t G = Geo<DT>::LOADS * kWaves;
  const uint32_t S = a.chunks, lane = lane_id();
  const uint64_t incl = wave_incl_scan_u64(r.T);
  uint64_t target = floor_mul(r.W, u);
  if (target >= r.W) target = r.W - 1;
  // incl at the last lane is W > target: some lane passes it.
  const uint32_t c = (uint32_t)__builtin_ctzll(ballot(lane < S && incl > target));
  uint64_t within = unscaled_bound(target - readlane_u64(incl - r.T, c), readlane_u64(r.R, c));
  const uint64_t vg = lane < G ? a.partials[(uint64_t)row * S + c].v[1 + lane] : 0ull;
  const uint32_t g = pick_slice(vg, G, within);
  draw_in_slice<DT, 0>(a, row, flags, inv_t, 0u, c, g, within, u2f(readlane_u32(f2u(r.m), c)),
                       0ull, 0ull, pd, r.kept, s);
}

// A drawing launch's block for a row with no residual pass (one wave): a
// greedy row's argmax of the chunk bests (sampling.metal:1478-1512), or a
// sampled row's plain draw, or the sentinel.
template <int DT>
__device__ __forceinline__ void plain_row_block(const SampleLaunch &a, uint32_t row, LeanLds &s) {
  const uint32_t S = a.chunks, lane = lane_id();
  // Every load the row needs first, none waiting on another: the record,
  // the uniform, the chunk summaries (lane c < S).
  const bool in = lane < S;
  const uint32_t at = in ? lane : 0u;
  const RowParams rp = a.params[row];
  const float u = row_uniform(a, row);
  const BlockHeader *h = a.headers + (uint64_t)row * S + at;
  const float hm = h->maximum, hbv = h->best_value;
  const uint32_t hadm = h->admitted, hcnt = h->count, hbi = h->best_id;
  const uint64_t hmass = a.partials[(uint64_t)row * S + at].v[0];
  if (!(rp.flags & kRowSampled)) {
    float hv = in ? hbv : -__builtin_inff();
    uint32_t hi = in ? hbi : kNoToken;
    wave_argmax(hv, hi);
    if (lane == 0) write_result(a, row, hi, 0.0f, 0);
    return;
  }
  const RowSums r = row_sums_of(S, hm, hadm, hcnt, hmass, rp.inv_t);
  const bool none = r.admitted == 0 || r.M == __builtin_inff();
  if (none || r.W == 0) {
    // The sentinel (a row of -inf keeps every token at probability 0).
    if (lane == 0) write_result(a, row, kNoToken, 0.0f, none ? 0u : r.kept);
    return;
  }
  plain_draw_wave<DT>(a, row, rp.flags, rp.inv_t, r, u, 0.0f, s);
}

// The residual pass of the rows flagged kRowLean (drafted, no cut, no
// penalty, mask or extra tokens), one block per (row, chunk): the same
// partial slots as uncut_kernel's pass (the chunk's residual mass and its
// slices', the draft token's float weight), from the same arithmetic, but
// with nothing else in the kernel and half a chunk's logits and q held at
// a time, so it keeps few registers and many waves per SIMD. Without
// l.draw, uncut_kernel then finishes these rows in one block each (this
// launch ends first). With it, the launch finishes every row itself: the
// lean rows' last chunk blocks also draw the rows without a residual pass
// (plain_row_block), and each lean row's last chunk block (its finisher)
// draws it as uncut_kernel would. The row's other blocks publish their
// slice masses (below 2^54) as self-validating words, mass | tag10 << 54,
// and the draft token's weight as tag12 << 32 | its bits (tag = call
// epoch << 1 | 1, 10 and 12 bits of it); the finisher gathers them, each
// word re-read until it carries this
// call's tag (at most a.wait_bound reads), and returns each to zero. Its
// waits end: the row's other blocks were dispatched before it (block
// index order) and wait on nothing. Should one give up, the row gets
// JF_NO_TOKEN and the status word is set.
template <int DT, bool DENSE, bool PACKED>
__global__ __launch_bounds__(kThreads) void residual_kernel(LeanLaunch l) {
  static_assert(!PACKED || DT == 0, "packed weights come from fp32 select passes");
  constexpr int VEC = Geo<DT>::VEC, LOADS = Geo<DT>::LOADS, SLAB = Geo<DT>::SLAB;
  constexpr uint32_t CHUNK = Geo<DT>::CHUNK, G = LOADS * kWaves;
  constexpr int HL = LOADS / 2, HV = HL * VEC;  // loads and values per half
  static_assert(HL == 2 || HL == 4, "two or four loads a half");
  const SampleLaunch &a = l.a;
  __shared__ LeanLds s;
  const uint32_t S = a.chunks;
  const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint32_t lean = blockIdx.x / S, chunk = blockIdx.x % S;
  const uint32_t row = l.row_of[lean];
  // A drawing launch's last chunk blocks also draw the rows without a
  // residual pass: waves 1-3 of lean row j's block take rows
  // n_lean + j + k n_lean, one per wave at a time, while wave 0 reads the
  // row's summaries, before the block's own chunk. That chunk is the row's
  // partial one when the vocabulary does not fill the last chunk, so this
  // mostly takes time the block would spend waiting for the row's other
  // blocks.
  const bool finisher = l.draw && chunk + 1 == S;
  const auto draw_plain_share = [&]() {
    for (uint32_t i = lean + (w - 1) * l.n_lean; i < l.n_plain; i += (kWaves - 1) * l.n_lean)
      plain_row_block<DT>(a, l.row_of[l.n_lean + i], s);
  };
  const RowParams rp = a.params[row];
  const uint32_t draft = row_draft(a, rp);
  if (draft == kNoToken) {
    // Drawn plainly: by uncut_kernel, or here by chunk 0's block.
    if (l.draw && chunk == 0 && w == 0) plain_row_block<DT>(a, row, s);
    if (finisher && w != 0) draw_plain_share();
    return;
  }
  const uint64_t tag10 = ((uint64_t)(a.epoch & 0x1ffu) << 1) | 1ull;
  const uint64_t tag12 = ((uint64_t)(a.epoch & 0x7ffu) << 1) | 1ull;
  if (tid == 0) s.fail = 0;
  const float inv_t = rp.inv_t;
  // The row's maximum, this chunk's rescale and the row's mass from the
  // chunk summaries (wave 0, S <= 64).
  StagePartial *parts = a.partials + (uint64_t)row * S;
  if (w == 0) {
    const RowSums r = row_sums(a, row, inv_t);
    if (lane == chunk) {
      s.mc = r.m;
      s.rc = r.R;
    }
    if (lane < S) {
      s.cmax[lane] = r.m;
      s.cscale[lane] = r.R;
      s.ctot[lane] = r.T;
    }
    if (lane == 0) {
      const bool none = r.admitted == 0 || r.M == __builtin_inff();
      s.W = r.W;
      s.ok = !none && r.W != 0 ? 1u : 0u;
      s.kept = none ? 0u : r.kept;
    }
  } else if (finisher) {
    draw_plain_share();
  }
  stage_candidates(a, rp, s);  // ends with a barrier
  if (!s.ok) {
    // The sentinel: uncut_kernel's, or here chunk 0's block's.
    if (l.draw && chunk == 0 && tid == 0) write_result(a, row, kNoToken, 0.0f, s.kept);
    return;
  }
  const float mc = s.mc;
  const uint64_t Rc = s.rc, W = s.W;
  const uint32_t V = a.vocabulary, base = chunk * CHUNK;
  const uint32_t lane_base = base + tid * VEC;
  const bool full = base + CHUNK <= V;
  const bool vec_x = full && a.aligned, vec_q = full && a.q_aligned;
  const float *qrow = DENSE ? a.dense_q + (uint64_t)rp.cand_index * a.q_stride : nullptr;
  const bool stops = (rp.flags & kRowExcludeStop) &&
                     ((a.stop0 >= base && a.stop0 < base + CHUNK) ||
                      (a.stop1 >= base && a.stop1 < base + CHUNK));
  uint64_t total = 0;
  // PACKED: the select pass stored each token's weight (pack_yk), read in
  // place of the logit; the draft token's float weight still comes from
  // its logit, requested here.
  const uint32_t *wrow = PACKED ? a.lean_weights + (uint64_t)row * a.lean_stride : nullptr;
  float xdraft = 0.0f;
  if (PACKED && draft < V && draft / CHUNK == chunk && tid == ((draft - base) % SLAB) / VEC)
    xdraft = ((const float *)a.logits)[(uint64_t)row * a.stride + draft];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float xv[HV], qv[HV];
    uint32_t pv[HV];
#pragma unroll
    for (int jj = 0; jj < HL; ++jj) {
      const uint32_t t0 = lane_base + (h * HL + jj) * SLAB;
      if constexpr (PACKED) {
        // The weights cover whole chunks (past the vocabulary: zero weights).
        const u32x4 v = *(const u32x4 *)(wrow + t0);
        pv[jj * 4 + 0] = v.x;
        pv[jj * 4 + 1] = v.y;
        pv[jj * 4 + 2] = v.z;
        pv[jj * 4 + 3] = v.w;
      } else if constexpr (DT == 0) {
        const float *rowp = (const float *)a.logits + (uint64_t)row * a.stride;
        if (vec_x) {
          const f32x4 v = *(const f32x4 *)(rowp + t0);
          xv[jj * 4 + 0] = v.x;
          xv[jj * 4 + 1] = v.y;
          xv[jj * 4 + 2] = v.z;
          xv[jj * 4 + 3] = v.w;
        } else {
#pragma unroll
          for (int e = 0; e < VEC; ++e)
            xv[jj * VEC + e] = t0 + e < V ? rowp[t0 + e] : kNotAdmitted;
        }
      } else {
        const uint16_t *rowp = (const uint16_t *)a.logits + (uint64_t)row * a.stride;
        if (vec_x) {
          const u32x4 v = *(const u32x4 *)(rowp + t0);
          const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            xv[jj * 8 + 2 * k] = u2f(vw[k] << 16);
            xv[jj * 8 + 2 * k + 1] = u2f(vw[k] & 0xffff0000u);
          }
        } else {
#pragma unroll
          for (int e = 0; e < VEC; ++e)
            xv[jj * VEC + e] = t0 + e < V ? bf16_to_float(rowp[t0 + e]) : kNotAdmitted;
        }
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const uint32_t t = t0 + e;
        if constexpr (DENSE) {
          if (vec_q) {
            if (e % 4 == 0) {
              const float4 f = *reinterpret_cast<const float4 *>(qrow + t);
              qv[jj * VEC + e] = f.x;
              qv[jj * VEC + e + 1] = f.y;
              qv[jj * VEC + e + 2] = f.z;
              qv[jj * VEC + e + 3] = f.w;
            }
          } else {
            qv[jj * VEC + e] = t < V ? qrow[t] : 0.0f;
          }
        } else {
          qv[jj * VEC + e] = draft_q(a, rp, t, s);
        }
        if (stops && (t == a.stop0 || t == a.stop1)) {
          if constexpr (PACKED)
            pv[jj * VEC + e] = 63u << 25;
          else
            xv[jj * VEC + e] = kNotAdmitted;
        }
      }
    }
    uint64_t lv[4] = {0, 0, 0, 0};
#pragma unroll
    for (int jj = 0; jj < HL; ++jj)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        uint64_t wq;
        if constexpr (PACKED) {
          const WeightYK wy = unpack_yk(pv[jj * VEC + e]);
          wq = scale_yk(wy.Y, wy.k, Rc);
        } else {
          wq = scaled_weight(xv[jj * VEC + e], mc, inv_t, Rc);
        }
        lv[jj] += residual_of(wq, W, qv[jj * VEC + e]);
      }
    // Lane l holds the wave's sum of load h * HL + l / 16 (l / 16 < HL).
    const uint64_t sl = wave_sums_u64<4>(lv);
    if (lane % 16 == 0 && lane / 16 < (uint32_t)HL) {
      const uint32_t gi = (h * HL + lane / 16) * kWaves + w;
      if (finisher)
        s.fsl[chunk * G + gi] = sl;
      else
        st_dev(&parts[chunk].v[kResidualSlot + 1 + gi], l.draw ? sl | tag10 << 54 : sl);
    }
    uint64_t t = sl + xor_u64<16>(sl);
    total += t + xor_u64<32>(t);
    // The draft token's float weight, from the thread that holds it.
    if (draft < V && draft / CHUNK == chunk) {
      const uint32_t o = draft - base, j = o / SLAB;
      if (j / HL == (uint32_t)h && tid == (o % SLAB) / VEC) {
        float xd = 0.0f;
        if constexpr (PACKED) {
          xd = stops && (draft == a.stop0 || draft == a.stop1) ? kNotAdmitted : xdraft;
        } else {
          const uint32_t i = (j % HL) * VEC + o % VEC;
#pragma unroll
          for (int k = 0; k < HV; ++k) xd = (uint32_t)k == i ? xv[k] : xd;
        }
        const uint32_t wd = f2u(weight_of(xd, mc, inv_t));
        if (finisher)
          s.dw = wd;
        else
          st_dev(&parts[chunk].v[kDraftSlot], l.draw ? tag12 << 32 | wd : (uint64_t)wd);
      }
    }
  }
  if (!l.draw) {
    if (lane == 0) s.wl[w] = total;
    __syncthreads();
    if (tid == 0) parts[chunk].v[kResidualSlot] = s.wl[0] + s.wl[1] + s.wl[2] + s.wl[3];
    return;
  }
  if (!finisher) return;

  // The finisher's gather: the other chunks' slice masses (word k is slice
  // k % G of chunk k / G) and, in the last thread, the draft token's
  // weight (its word PER). Each round re-reads every word of the thread
  // not yet seen with this call's tag, all requested before any is checked.
  constexpr uint64_t kMass54 = (1ull << 54) - 1ull;
  constexpr int PER = (kMaxChunks * G + kThreads - 1) / kThreads;
  const uint32_t n_words = chunk * G;
  const uint32_t cd = draft < V ? draft / CHUNK : chunk;
  uint32_t pending = 0;  // bit i: word i still to be seen
#pragma unroll
  for (int i = 0; i < PER; ++i)
    pending |= tid + i * kThreads < n_words ? 1u << i : 0u;
  if (cd != chunk && tid == kThreads - 1) pending |= 1u << PER;
  uint64_t vw[PER + 1];
  for (uint32_t n = 0; pending && n < a.wait_bound; ++n) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const uint32_t k = tid + i * kThreads;
      if ((pending >> i) & 1u) vw[i] = ld_dev(&parts[k / G].v[kResidualSlot + 1 + k % G]);
    }
    if ((pending >> PER) & 1u) vw[PER] = ld_dev(&parts[cd].v[kDraftSlot]);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const uint32_t k = tid + i * kThreads;
      if (((pending >> i) & 1u) && (vw[i] >> 54) == tag10) {
        s.fsl[k] = vw[i] & kMass54;
        st_dev(&parts[k / G].v[kResidualSlot + 1 + k % G], 0ull);
        pending &= ~(1u << i);
      }
    }
    if (((pending >> PER) & 1u) && (vw[PER] >> 32) == tag12) {
      s.dw = (uint32_t)vw[PER];
      st_dev(&parts[cd].v[kDraftSlot], 0ull);
      pending &= ~(1u << PER);
    }
  }
  const bool ok = pending == 0;
  if (!ok) s.fail = 1;
  __syncthreads();
  if (w != 0) return;
  if (s.fail) {
    if (lane == 0) {
      write_result(a, row, kNoToken, 0.0f, 0);
      if (a.status) __hip_atomic_store(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    return;
  }

  // Wave 0: p(draft), then the residual draw, or the plain one when no
  // residual mass remains (uncut_kernel's last block). Lane c < S sums
  // chunk c's slices.
  const float u = row_uniform(a, row);
  const bool in = lane < S;
  uint64_t rv = 0;
  if (in) {
    const ulonglong2 *f = reinterpret_cast<const ulonglong2 *>(&s.fsl[lane * G]);
#pragma unroll
    for (uint32_t g2 = 0; g2 < G / 2; ++g2) {
      const ulonglong2 p2 = f[g2];
      rv += p2.x + p2.y;
    }
  }
  const float pd = draft < V ? uncut_probability(u2f(s.dw), s.cscale[cd], W) : 0.0f;
  const uint64_t incl = wave_incl_scan_u64(rv);
  const uint64_t tot = readlane_u64(incl, 63);
  if (!tot) {
    RowSums r;
    r.m = in ? s.cmax[lane] : -3.402823466e38f;
    r.R = in ? s.cscale[lane] : kZeroScale;
    r.T = in ? s.ctot[lane] : 0ull;
    r.W = W;
    r.kept = s.kept;
    plain_draw_wave<DT>(a, row, rp.flags, inv_t, r, u, pd, s);
    return;
  }
  uint64_t target = floor_mul(tot, u);
  if (target >= tot) target = tot - 1;
  const uint32_t c = (uint32_t)__builtin_ctzll(ballot(in && incl > target));
  uint64_t within = target - readlane_u64(incl - rv, c);
  const uint64_t vg = lane < G ? s.fsl[c * G + lane] : 0ull;
  const uint32_t g = pick_slice(vg, G, within);
  draw_in_slice<DT, DENSE ? 1 : 2>(a, row, rp.flags, inv_t, rp.cand_index, c, g, within,
                                   s.cmax[c], s.cscale[c], W, pd, s.kept, s);
}

template <int DT>
__global__ __launch_bounds__(kThreads) void uncut_kernel(SampleLaunch a, uint32_t per_row) {
  constexpr int TPL = Geo<DT>::TPL, VEC = Geo<DT>::VEC, LOADS = Geo<DT>::LOADS,
                SLAB = Geo<DT>::SLAB;
  constexpr uint32_t CHUNK = Geo<DT>::CHUNK, G = LOADS * kWaves;
  __shared__ UncutLds s;
  const uint32_t S = a.chunks;
  const uint32_t row = blockIdx.x / per_row, chunk = blockIdx.x % per_row;
  const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const BlockHeader *hb = a.headers + (uint64_t)row * S;
  StagePartial *parts = a.partials + (uint64_t)row * S;
  // Requested together before anything waits: the row's record, its
  // uniform, and (wave 0) its chunk summaries, one per lane (S <= 64).
  const RowParams rp = a.params[row];
  const float u = row_uniform(a, row);
  const bool in = w == 0 && lane < S;
  const BlockHeader *hl = hb + (in ? lane : 0u);
  const float hm = hl->maximum, hbv = hl->best_value;
  const uint32_t hadm = hl->admitted, hcnt = hl->count, hbi = hl->best_id;
  const uint64_t hmass = parts[in ? lane : 0u].v[0];
  if (!(rp.flags & kRowSampled)) {
    // Greedy (sampling.metal:1478-1512), when no merge runs: the largest
    // chunk best, the lowest id among equals.
    if (a.finish_greedy && chunk == 0 && tid < 64) {
      float hv = in ? hbv : -__builtin_inff();
      uint32_t hi = in ? hbi : kNoToken;
      wave_argmax(hv, hi);
      if (tid == 0) write_result(a, row, hi, 0.0f, 0);
    }
    return;
  }
  if (!uncut_row(rp)) return;  // the merge's
  const uint32_t draft = row_draft(a, rp);
  const bool drafted = draft != kNoToken;
  if (!drafted && chunk != 0) return;
  const float inv_t = rp.inv_t;
  // The row's chunk summaries.
  if (w == 0) {
    const float m = in ? hm : -3.402823466e38f;
    const uint32_t adm = in ? hadm : 0u;
    const uint32_t cnt = in ? hcnt : 0u;
    const uint64_t mass = in ? hmass : 0ull;
    const float M = wave_max_f32(m);
    const uint64_t R = in ? chunk_scale(m, M, inv_t) : kZeroScale;
    const uint64_t T = scale_by(mass, R);
    const uint64_t W = wave_sum_u64(T);
    const uint32_t admitted = wave_sum_u32(adm), kept = wave_sum_u32(cnt);
    if (in) {
      s.cmax[lane] = m;
      s.cscale[lane] = R;
      s.ctot[lane] = T;
      s.ccount[lane] = cnt;
    }
    if (lane == 0) {
      s.row_max = M;
      s.row_mass = W;
      // Nothing admitted, or a +inf maximum: the sentinel with nothing kept.
      const bool none = admitted == 0 || M == __builtin_inff();
      s.row_admitted = none ? 0u : 1u;
      s.row_kept = none ? 0u : kept;
      s.pd = 0.0f;
    }
  }
  __syncthreads();
  const uint64_t W = s.row_mass;
  if (chunk == 0 && a.out_kept_ids && s.row_admitted && a.kept_cap)
    uncut_kept<DT>(a, rp, row, s, W);
  if (!s.row_admitted || W == 0) {
    // The sentinel (a row of -inf keeps every token at probability 0).
    if (chunk == 0 && tid == 0) write_result(a, row, kNoToken, 0.0f, s.row_kept);
    return;
  }
  if (!drafted) {
    uncut_draw<DT>(a, rp, row, s, W, u);
    return;
  }

  float xs[TPL];
  if (rp.flags & kRowLean) {
    // residual_kernel summed this row's residual masses (its launch ended
    // before this one began): chunk 0's block draws.
    if (chunk != 0) return;
    stage_candidates(a, rp, s);
  } else {
    // A drafted row: this chunk's residual masses per slice.
    float qv[TPL];
    if (a.dense_q) load_dense_q<DT>(a, rp, chunk, qv);
    load_chunk<DT>(a, rp, row, chunk, s, xs);
    stage_candidates(a, rp, s);
    const float mc = s.cmax[chunk];
    const uint64_t Rc = s.cscale[chunk];
    const uint32_t lane_base = chunk * CHUNK + tid * VEC;
    uint64_t total = 0;
    // Four loads at a time (fewer live registers than all of them at once).
#pragma unroll
    for (int h = 0; h < LOADS / 4; ++h) {
      uint64_t lv[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int j = h * 4 + jj;
        lv[jj] = 0;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const int i = j * VEC + e;
          const float q = a.dense_q ? qv[i] : draft_q(a, rp, lane_base + j * SLAB + e, s);
          lv[jj] += residual_of(scaled_weight(xs[i], mc, inv_t, Rc), W, q);
        }
      }
      // Lane l holds the wave's sum of load h * 4 + l / 16.
      const uint64_t sl = wave_sums_u64<4>(lv);
      if (lane % 16 == 0)
        st_dev(&parts[chunk].v[kResidualSlot + 1 + (h * 4 + lane / 16) * kWaves + w], sl);
      uint64_t t = sl + xor_u64<16>(sl);
      total += t + xor_u64<32>(t);
    }
    // The draft token's float weight, from the thread that holds it.
    if (draft < a.vocabulary && draft / CHUNK == chunk) {
      const uint32_t o = draft - chunk * CHUNK;
      if (tid == (o % SLAB) / VEC) {
        const uint32_t i = (o / SLAB) * VEC + o % VEC;
        float xd = 0.0f;
#pragma unroll
        for (int k = 0; k < TPL; ++k) xd = (uint32_t)k == i ? xs[k] : xd;
        st_dev(&parts[chunk].v[kDraftSlot], (uint64_t)f2u(weight_of(xd, mc, inv_t)));
      }
    }
    if (lane == 0) s.wl[w] = total;
    __syncthreads();
    if (tid == 0)
      st_dev(&parts[chunk].v[kResidualSlot], s.wl[0] + s.wl[1] + s.wl[2] + s.wl[3]);
    if (!arrive_last(a.counters + row, S, s)) return;
  }

  // The row's last block: p(draft), then the residual draw when it has mass.
  if (w == 0) {
    const bool in = lane < S;
    const uint64_t rv = in ? ld_dev(&parts[lane].v[kResidualSlot]) : 0ull;
    const uint64_t incl = wave_incl_scan_u64(rv);
    const uint64_t tot = readlane_u64(incl, 63);
    uint64_t target = floor_mul(tot, u);
    if (tot && target >= tot) target = tot - 1;
    const uint32_t c = tot ? (uint32_t)__builtin_ctzll(ballot(in && incl > target)) : 0u;
    const uint64_t before = readlane_u64(incl - rv, c);
    if (lane == 0) {
      s.residual = tot ? 1u : 0u;
      s.sel_bin = c;
      s.sel_excl = target - before;
      if (draft < a.vocabulary) {
        const uint32_t cd = draft / CHUNK;
        s.pd = uncut_probability(u2f((uint32_t)ld_dev(&parts[cd].v[kDraftSlot])),
                                 s.cscale[cd], W);
      }
    }
  }
  __syncthreads();
  if (!s.residual) {
    uncut_draw<DT>(a, rp, row, s, W, u);
    return;
  }
  const uint32_t c = s.sel_bin;
  uint64_t vg = 0;
  if (w == 0 && lane < G) vg = ld_dev(&parts[c].v[kResidualSlot + 1 + lane]);
  load_chunk<DT>(a, rp, row, c, s, xs);
  if (w == 0) {
    uint64_t wi = s.sel_excl;
    const uint32_t gg = pick_slice(vg, G, wi);
    if (lane == 0) {
      s.slice = gg;
      s.slice_within = wi;
    }
  }
  __syncthreads();
  const uint32_t g = s.slice, jg = g / kWaves;
  if (w == g % kWaves) {
    const float mcc = s.cmax[c];
    const uint64_t Rcc = s.cscale[c];
    const uint32_t tbase = c * CHUNK + jg * SLAB + tid * VEC;
    uint64_t q[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float x = 0.0f;
#pragma unroll
      for (int j = 0; j < LOADS; ++j) x = (uint32_t)j == jg ? xs[j * VEC + e] : x;
      // Past the vocabulary (a partial last chunk) the weight is zero and no
      // q is read: a dense q row ends at the vocabulary.
      const float qe = tbase + e < a.vocabulary ? draft_q(a, rp, tbase + e, s) : 0.0f;
      q[e] = residual_of(scaled_weight(x, mcc, inv_t, Rcc), W, qe);
    }
    uint32_t e_hit;
    if (lane == slice_hit<VEC>(q, s.slice_within, e_hit))
      write_result(a, row, tbase + e_hit, s.pd, s.row_kept);
  }
}
#endif

// ---- acceptance --------------------------------------------------------
//
// One wave per lane. Everything the lane's walk can read goes out in one
// round of loads (thread t holds row or proposal t); the walk itself then
// runs on registers: readlane for the current row, a ballot for a child
// search or for the leading run of accepted proposals. The result is that
// of the reference's one-thread loops, step for step.

// decode_accept_dflash (sampling.metal:1399-1423, 1514-1558). Greedy:
// the leading proposals equal to the target's tokens. Sampled: the leading
// proposals that pass u q < p (q the draft's probability of the proposal
// among its 16 candidates, the first that lists it; 0 when none does), each
// replacing the target's token; a proposal of JF_NO_TOKEN ends the run.
#if JF_IN(4)
__global__ __launch_bounds__(64) void accept_chain_kernel(AcceptChainLaunch a) {
  const uint32_t lane = blockIdx.x, t = threadIdx.x;
  const AcceptChainLane lp = a.lane_params[lane];
  const uint32_t VR = a.verify_rows, P = VR - 1;
  uint32_t *tokens = a.target_tokens + (uint64_t)lane * VR;
  const uint32_t tok = t < VR ? tokens[t] : kNoToken;
  const uint32_t d = t < P ? a.proposed[(uint64_t)lane * P + t] : kNoToken;
  bool ok;
  if (lp.sampled) {
    uint32_t ids[16];
    float probs[16];
    float p = 0.0f, u = 0.0f;
    if (t < P) {
      const uint64_t c = ((uint64_t)lane * P + t) * 16;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        ids[j] = a.candidates[c + j];
        probs[j] = a.proposal_probs[c + j];
      }
      p = a.target_draft_probs[(uint64_t)lane * VR + t];
      u = a.uniforms[(uint64_t)lane * 40 + (t < 7 ? 8 + t : 16 + t - 7)];
    }
    float q = 0.0f;
    bool seen = false;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const bool m = t < P && !seen && ids[j] == d;
      q = m ? probs[j] : q;
      seen |= m;
    }
    ok = t < P && d != kNoToken && u * q < p;
  } else {
    ok = t < P && d == tok;
  }
  // Bit P of ~ballot is set (no thread at or past P is ok): accepted <= P.
  const uint32_t accepted = (uint32_t)__builtin_ctzll(~ballot(ok));
  const bool replace = lp.sampled && t < accepted;
  if (replace) tokens[t] = d;
  const uint32_t out = replace ? d : tok;
  const uint32_t kept = finish_kept(out, accepted, lp.remaining, a.stop0, a.stop1);
  if (t == 0) {
    a.retained[lane] = kept;
    a.accepted[lane] = accepted;
  }
}
#endif

#if JF_IN(4)
__global__ __launch_bounds__(64) void accept_tree_kernel(AcceptTreeLaunch a) {
  const uint32_t lane = blockIdx.x, t = threadIdx.x;
  const TreeLaneParams &tr = a.trees[lane];
  const uint32_t R = a.rows_per_lane;
  uint32_t *tokens = a.target_tokens + (uint64_t)lane * R;
  const uint32_t tok = t < R ? tokens[t] : kNoToken;
  float pv = 0.0f, uv = 0.0f;
  if (tr.sampled) {
    if (t < R) pv = a.target_draft_probs[(uint64_t)lane * R + t];
    if (t < 16) uv = a.uniforms[(uint64_t)lane * 40 + 8 + t];
  }
  uint32_t path;
  const uint32_t length = accept_tree_wave(tr, tok, pv, uv, path);
  // Thread i < length: path row i's output; the rows past the path keep
  // their selected tokens.
  const uint32_t out = tree_path_token(tr, tok, path, length);
  if (t < length) tokens[t] = out;
  finish_tree_lane(a, lane, tr, out, path, length);
}
#endif

// ---- launchers -------------------------------------------------------

#if JF_IN(1)
int launch_select(const SampleLaunch &a, uint32_t dtype, void *stream,
                  void *start_event, void *stop_event) {
  const dim3 grid(a.rows * a.chunks), block(kThreads);
  const hipStream_t st = (hipStream_t)stream;
  if (start_event) {
    const hipEvent_t e0 = (hipEvent_t)start_event, e1 = (hipEvent_t)stop_event;
    if (dtype == 0)
      hipExtLaunchKernelGGL(select_kernel<0>, grid, block, 0, st, e0, e1, 0, a);
    else
      hipExtLaunchKernelGGL(select_kernel<1>, grid, block, 0, st, e0, e1, 0, a);
  } else if (dtype == 0) {
    hipLaunchKernelGGL(select_kernel<0>, grid, block, 0, st, a);
  } else {
    hipLaunchKernelGGL(select_kernel<1>, grid, block, 0, st, a);
  }
  return (int)hipGetLastError();
}
#endif

#if JF_IN(1)
// Blocks of select_fast_kernel<dtype> the current device holds at once
// (0 when the query fails), cached per device; the cache is shared by every
// host thread, so it is read and filled under a lock.
static uint32_t fast_resident_blocks(uint32_t dtype) {
  constexpr int kDevices = 64;
  static std::mutex lock;
  static uint32_t cache[kDevices][2];
  static bool known[kDevices][2];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kDevices) return 0;
  std::lock_guard<std::mutex> guard(lock);
  if (!known[dev][dtype]) {
    int per_cu = 0, cus = 0;
    const hipError_t e1 =
        dtype == 0
            ? hipOccupancyMaxActiveBlocksPerMultiprocessor(
                  &per_cu, select_fast_kernel<0, false, FastRows, NoFinish>, kThreads, 0)
            : hipOccupancyMaxActiveBlocksPerMultiprocessor(
                  &per_cu, select_fast_kernel<1, false, FastRows, NoFinish>, kThreads, 0);
    const hipError_t e2 = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    cache[dev][dtype] = e1 == hipSuccess && e2 == hipSuccess && per_cu > 0 && cus > 0
                            ? (uint32_t)per_cu * (uint32_t)cus
                            : 0u;
    known[dev][dtype] = true;
  }
  return cache[dev][dtype];
}

int launch_select_fast(const FastLaunch &f, const FastRows *fr, uint32_t rows, uint32_t dtype,
                       const RowParams *uniform, bool extras, bool fuse_uncut,
                       const AcceptTreeLaunch *accept, bool *accepted, void *stream,
                       void *start_event, void *stop_event) {
  if (accepted) *accepted = false;
  if (f.fuse_greedy == 1u && f.a.chunks > 1 && rows < fast_resident_blocks(dtype)) {
    // Each row's last chunk can wait for the row's other blocks instead of
    // counting arrivals: only those finishers (one a row) ever wait, and
    // they are fewer than the blocks the device holds at once, so some
    // slot always remains for the blocks they wait for, which never wait.
    FastLaunch g = f;
    g.fuse_greedy = 2u;
    return launch_select_fast(g, fr, rows, dtype, uniform, extras, fuse_uncut, accept, accepted,
                              stream, start_event, stop_event);
  }
  if (!fr && (!uniform || f.mapped || extras)) return (int)hipErrorInvalidValue;
  if (fuse_uncut && (extras || f.mapped)) return (int)hipErrorInvalidValue;
  const dim3 grid(f.a.chunks, rows), block(kThreads);
  const hipStream_t st = (hipStream_t)stream;
  const hipEvent_t e0 = (hipEvent_t)start_event, e1 = (hipEvent_t)stop_event;
  const RowParams u = uniform ? *uniform : RowParams{};
  const uint32_t packed = (uniform ? 0x80000000u | (u.flags & 0xffu) : 0u) |
                          (f.a.chunks << 8) | (f.slot_count == 512u ? 0x10000u : 0u) |
                          ((f.row_base >> 8) << 17);
  auto go = [&](auto kernel, const auto &rows_arg, const auto &fin) {
    hipExtLaunchKernelGGL(kernel, grid, block, 0, st, e0, e1, 0, f.a.logits, f.pen_slots,
                          (uint32_t)f.a.stride, f.a.vocabulary, packed, u.top_k,
                          u.minp_offset, u.repetition, u.repetition_inverse, u.presence,
                          u.frequency, f.mapped, f, rows_arg, fin);
  };
  // The lanes' tree acceptance rides on the row finishers (each row's last
  // chunk block) of a uniform all-greedy launch.
  if (accept && f.fuse_greedy == 2u && !fr && !extras && !f.mapped && f.row_base == 0) {
    dtype == 0 ? go(select_fast_kernel<0, false, NoRows, AcceptTreeLaunch>, NoRows{}, *accept)
               : go(select_fast_kernel<1, false, NoRows, AcceptTreeLaunch>, NoRows{}, *accept);
    if (accepted) *accepted = true;
  } else if (fuse_uncut) {
    if (!fr)
      dtype == 0 ? go(select_fast_kernel<0, false, NoRows, UncutFinish>, NoRows{}, UncutFinish{})
                 : go(select_fast_kernel<1, false, NoRows, UncutFinish>, NoRows{}, UncutFinish{});
    else
      dtype == 0 ? go(select_fast_kernel<0, false, FastRows, UncutFinish>, *fr, UncutFinish{})
                 : go(select_fast_kernel<1, false, FastRows, UncutFinish>, *fr, UncutFinish{});
  } else if (f.a.lean_weights) {
    // Stored weights: fp32 rows with no extra token only.
    if (dtype != 0 || extras) return (int)hipErrorInvalidValue;
    !fr ? go(select_fast_kernel<0, false, NoRows, StoreWeights>, NoRows{}, StoreWeights{})
        : go(select_fast_kernel<0, false, FastRows, StoreWeights>, *fr, StoreWeights{});
  } else if (!fr) {
    dtype == 0 ? go(select_fast_kernel<0, false, NoRows, NoFinish>, NoRows{}, NoFinish{})
               : go(select_fast_kernel<1, false, NoRows, NoFinish>, NoRows{}, NoFinish{});
  } else if (dtype == 0) {
    extras ? go(select_fast_kernel<0, true, FastRows, NoFinish>, *fr, NoFinish{})
           : go(select_fast_kernel<0, false, FastRows, NoFinish>, *fr, NoFinish{});
  } else {
    extras ? go(select_fast_kernel<1, true, FastRows, NoFinish>, *fr, NoFinish{})
           : go(select_fast_kernel<1, false, FastRows, NoFinish>, *fr, NoFinish{});
  }
  return (int)hipGetLastError();
}
#endif

#if JF_IN(2)
int launch_merge(const SampleLaunch &a, uint32_t dtype, void *stream) {
  const dim3 grid(a.rows), block(kThreads);
  if (dtype == 0)
    hipLaunchKernelGGL(merge_kernel<0>, grid, block, 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(merge_kernel<1>, grid, block, 0, (hipStream_t)stream, a);
  return (int)hipGetLastError();
}
#endif

#if JF_IN(4)
int launch_residual(const LeanLaunch &l, uint32_t dtype, void *stream) {
  const dim3 grid(l.n_lean * l.a.chunks), block(kThreads);
  const hipStream_t st = (hipStream_t)stream;
  // A sparse draft's 16-candidate lookup per token takes about 30 more
  // registers than a dense q row: separate instantiations. With the select
  // pass's stored weights (fp32 rows), the weights are read in place of the
  // logits.
  const bool packed = l.a.lean_weights != nullptr;
  if (l.a.dense_q) {
    if (dtype == 0 && packed)
      hipLaunchKernelGGL((residual_kernel<0, true, true>), grid, block, 0, st, l);
    else if (dtype == 0)
      hipLaunchKernelGGL((residual_kernel<0, true, false>), grid, block, 0, st, l);
    else
      hipLaunchKernelGGL((residual_kernel<1, true, false>), grid, block, 0, st, l);
  } else {
    if (dtype == 0 && packed)
      hipLaunchKernelGGL((residual_kernel<0, false, true>), grid, block, 0, st, l);
    else if (dtype == 0)
      hipLaunchKernelGGL((residual_kernel<0, false, false>), grid, block, 0, st, l);
    else
      hipLaunchKernelGGL((residual_kernel<1, false, false>), grid, block, 0, st, l);
  }
  return (int)hipGetLastError();
}

int launch_uncut(const SampleLaunch &a, uint32_t dtype, uint32_t per_row, void *stream) {
  const dim3 grid(a.rows * per_row), block(kThreads);
  if (dtype == 0)
    hipLaunchKernelGGL(uncut_kernel<0>, grid, block, 0, (hipStream_t)stream, a, per_row);
  else
    hipLaunchKernelGGL(uncut_kernel<1>, grid, block, 0, (hipStream_t)stream, a, per_row);
  return (int)hipGetLastError();
}
#endif

#if JF_IN(2)
int launch_merge_small(const SampleLaunch &a, uint32_t dtype, bool wide, void *stream) {
  const dim3 grid(a.rows), block(kThreads);
  const hipStream_t st = (hipStream_t)stream;
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, block, 0, st, a.headers, (const uint64_t *)a.cands,
                       a.params, a.uniforms, a.uniform_index,
                       a.chunks | (a.row_indexed ? 0x80000000u : 0u),
                       (uint32_t)a.uniform_offset, (uint32_t)a.uniform_stride,
                       a.draft_tokens && !a.row_indexed ? a.drafted_rows : 0u, a);
  };
  // The wider fetch past 20 chunks (fewer than 128 slots a chunk otherwise).
  const bool w = wide && a.chunks > 20;
  if (dtype == 0)
    w ? go(merge_small_kernel<0, 20>) : go(merge_small_kernel<0, 10>);
  else
    w ? go(merge_small_kernel<1, 20>) : go(merge_small_kernel<1, 10>);
  return (int)hipGetLastError();
}
#endif

#if JF_IN(3)
int launch_stage(const SampleLaunch &a, uint32_t dtype, void *stream) {
  const dim3 grid(a.rows * a.chunks), block(kThreads);
  const hipStream_t st = (hipStream_t)stream;
  auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, block, 0, st, a); };
  const int cls = stage_class(a.stage);
  if (cls == kClsWalk) {
    if (dtype == 0)
      hipLaunchKernelGGL(walk_kernel<0>, dim3(a.rows), block, 0, st, a);
    else
      hipLaunchKernelGGL(walk_kernel<1>, dim3(a.rows), block, 0, st, a);
    return (int)hipGetLastError();
  }
#define JF_STAGE_CASE(C)                              \
  case C:                                             \
    if (dtype == 0)                                   \
      go(stage_kernel<0, C>);                         \
    else                                              \
      go(stage_kernel<1, C>);                         \
    break;
  switch (cls) {
    JF_STAGE_CASE(kClsCount)
    JF_STAGE_CASE(kClsDigits)
    JF_STAGE_CASE(kClsTie)
    JF_STAGE_CASE(kClsLocate)
    JF_STAGE_CASE(kClsMass)
    JF_STAGE_CASE(kClsDraw)
    JF_STAGE_CASE(kClsKeptWrite)
    default:
      return (int)hipErrorInvalidValue;
  }
#undef JF_STAGE_CASE
  return (int)hipGetLastError();
}
#endif

#if JF_IN(4)
int launch_accept_chain(const AcceptChainLaunch &a, void *stream) {
  const dim3 grid(a.lanes), block(64);
  hipLaunchKernelGGL(accept_chain_kernel, grid, block, 0, (hipStream_t)stream, a);
  return (int)hipGetLastError();
}
#endif

#if JF_IN(4)
int launch_accept_tree(const AcceptTreeLaunch &a, void *stream) {
  const dim3 grid(a.lanes), block(64);
  hipLaunchKernelGGL(accept_tree_kernel, grid, block, 0, (hipStream_t)stream, a);
  return (int)hipGetLastError();
}
#endif

}  // namespace jf
