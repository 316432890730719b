// Device helpers of the gfx950 sampler: the logit order, the weight, exact
// fixed-point arithmetic and wave64 primitives. Everything here is plain
// IEEE fp32 (the library is compiled with -ffp-contract=off) or integer
// code, so a host restatement of the same steps produces the same bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jf {

constexpr uint32_t kNoToken = 0xffffffffu;
constexpr uint32_t kPromptBit = 0x80000000u;
constexpr uint32_t kCountMask = 0x7fffffffu;
constexpr int kWave = 64;
// Fixed-point weight: floor(w * 2^44). A row holds < 2^18 tokens of weight
// <= 1, so every sum of weights stays below 2^62.
constexpr int kWeightBits = 44;

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// The order of the logits as an unsigned key (sampling.metal:167-171): a
// larger logit has a larger key and -0, +0 share one.
__device__ __forceinline__ uint32_t logit_key(float value) {
  uint32_t bits = f2u(value);
  bits = (bits << 1) ? bits : 0u;
  return (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
}
__device__ __forceinline__ float key_logit(uint32_t key) {
  return u2f((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

// e^x by the Cephes expf method (S. L. Moshier): n = rint(x log2 e),
// r = x - n ln2 with the two-constant Cody-Waite split of ln2,
// e^r = 1 + r + r^2 P(r) with Cephes' degree-5 P, times 2^n. Zero below
// -86, so every nonzero result is a normal float.
__device__ __forceinline__ float exp_weight(float x) {
  if (!(x >= -86.0f)) return 0.0f;
  if (x > 88.0f) return __builtin_inff();
  const float n = __builtin_rintf(x * 1.44269504088896341f);
  float r = __builtin_fmaf(n, -0.693359375f, x);
  r = __builtin_fmaf(n, 2.12194440e-4f, r);
  float p = 1.9875691500e-4f;
  p = __builtin_fmaf(p, r, 1.3981999507e-3f);
  p = __builtin_fmaf(p, r, 8.3334519073e-3f);
  p = __builtin_fmaf(p, r, 4.1665795894e-2f);
  p = __builtin_fmaf(p, r, 1.6666665459e-1f);
  p = __builtin_fmaf(p, r, 5.0000001201e-1f);
  const float r2 = r * r;
  const float y = __builtin_fmaf(p, r2, r) + 1.0f;
  const int ni = (int)n;
  return y * u2f((uint32_t)(ni + 127) << 23);
}

// A token's softmax weight relative to the row maximum (sampling.metal:38-40,
// with the division by the temperature taken as a product by its inverse).
__device__ __forceinline__ float weight_of(float value, float maximum,
                                           float inv_t) {
  return exp_weight((value - maximum) * inv_t);
}
__device__ __forceinline__ uint64_t quantize(float w) {
  return (uint64_t)(w * 0x1p44f);
}

// floor(a * f) exactly for f in [0, 1]; NaN and f <= 0 give 0, f >= 1 gives a.
__device__ __forceinline__ uint64_t floor_mul(uint64_t a, float f) {
  if (!(f > 0.0f)) return 0;
  if (f >= 1.0f) return a;
  const uint32_t b = f2u(f);
  const uint32_t e = b >> 23;
  const uint64_t m = e ? ((b & 0x7fffffu) | 0x800000u) : (b & 0x7fffffu);
  const int sh = e ? 150 - (int)e : 149;
  const unsigned __int128 p = (unsigned __int128)a * m;
  return sh >= 128 ? 0 : (uint64_t)(p >> sh);
}

// penalize_logit (sampling.metal:928-935): repetition divides a positive
// logit and multiplies a negative one, presence and frequency lower it by
// the count, and the result saturates (a NaN becomes -FLT_MAX).
__device__ __forceinline__ float penalize(float value, uint32_t count,
                                          float repetition, float inverse,
                                          float presence, float frequency) {
  value *= value > 0.0f ? inverse : repetition;
  if (count) {
    const float scaled = frequency * (float)count;
    const float lowered = scaled + presence;
    value = value - lowered;
  }
  return __builtin_fminf(__builtin_fmaxf(value, -3.402823466e38f),
                         3.402823466e38f);
}

__device__ __forceinline__ float bf16_to_float(uint32_t bits16) {
  return u2f(bits16 << 16);
}

// ---- cross-block scratch -------------------------------------------------
// Blocks of one row exchange partial results through device memory. The
// writers store with device-coherent (L2 write-through) stores and wait for
// them to complete before they count their arrival; the reader loads with
// device-coherent (L2-bypassing) loads. No cache writeback or invalidate of
// the whole L2 is needed, which a device-scope fence would issue per block.
__device__ __forceinline__ void st_dev(uint32_t *p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(uint64_t *p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(float *p, float v) {
  st_dev((uint32_t *)p, __float_as_uint(v));
}
__device__ __forceinline__ uint32_t ld_dev(const uint32_t *p) {
  return __hip_atomic_load((uint32_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_dev(const uint64_t *p) {
  return __hip_atomic_load((uint64_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float *p) {
  return __uint_as_float(ld_dev((const uint32_t *)p));
}
// Waits until every memory access this thread issued has completed.
__device__ __forceinline__ void wait_memory() { __builtin_amdgcn_s_waitcnt(0); }

// ---- wave64 primitives ------------------------------------------------

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

// Lanes below this one whose bit is set in `mask`.
__device__ __forceinline__ uint32_t mbcnt(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(
      (uint32_t)(mask >> 32),
      __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor((uint32_t)v, m, kWave);
  const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m, kWave);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t shfl_down_u64(uint64_t v, int d) {
  const uint32_t lo = __shfl_down((uint32_t)v, d, kWave);
  const uint32_t hi = __shfl_down((uint32_t)(v >> 32), d, kWave);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t shfl_up_u64(uint64_t v, int d) {
  const uint32_t lo = __shfl_up((uint32_t)v, d, kWave);
  const uint32_t hi = __shfl_up((uint32_t)(v >> 32), d, kWave);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
  const uint32_t lo = __shfl((uint32_t)v, src, kWave);
  const uint32_t hi = __shfl((uint32_t)(v >> 32), src, kWave);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v += shfl_xor_u64(v, m);
  return v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v = max(v, (uint32_t)__shfl_xor(v, m, kWave));
  return v;
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v = min(v, (uint32_t)__shfl_xor(v, m, kWave));
  return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}
// Inclusive prefix sum over lanes.
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t v) {
  const uint32_t lane = lane_id();
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint64_t o = shfl_up_u64(v, d);
    if (lane >= (uint32_t)d) v += o;
  }
  return v;
}
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  const uint32_t lane = lane_id();
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t o = __shfl_up(v, d, kWave);
    if (lane >= (uint32_t)d) v += o;
  }
  return v;
}

// The largest greedy candidate of the wave: larger value, then lower id.
__device__ __forceinline__ void wave_argmax(float &value, uint32_t &id) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const float ov = __shfl_xor(value, m, kWave);
    const uint32_t oi = __shfl_xor(id, m, kWave);
    if (ov > value || (ov == value && oi < id)) {
      value = ov;
      id = oi;
    }
  }
}

// The k-th largest (1-based) of the wave's 64 values, by bitwise descent:
// the largest v with at least k lanes holding a value >= v. k in 1..64.
__device__ __forceinline__ uint32_t wave_kth_largest(uint32_t v, uint32_t k) {
  uint32_t answer = 0;
#pragma unroll 1
  for (int b = 31; b >= 0; --b) {
    const uint32_t trial = answer | (1u << b);
    if ((uint32_t)__popcll(ballot(v >= trial)) >= k) answer = trial;
  }
  return answer;
}

}  // namespace jf
