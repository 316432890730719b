// Device helpers of the gfx950 sampler: the logit order, the weight, exact
// fixed-point arithmetic and wave64 primitives. Everything here is plain
// IEEE fp32 (the library is compiled with -ffp-contract=off) or integer
// code, so a host restatement of the same steps produces the same bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

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
// Branch-free: the polynomial runs on the argument clamped to [-87, 88]
// (equal to it inside the range), and the two range ends are selected
// afterwards, so a wave runs no exec-mask branches per token.
__device__ __forceinline__ float exp_weight(float x_in) {
  const float x = __builtin_fminf(__builtin_fmaxf(x_in, -87.0f), 88.0f);
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
  const float e = y * u2f((uint32_t)(ni + 127) << 23);
  const float hi = x_in > 88.0f ? __builtin_inff() : e;
  return x_in >= -86.0f ? hi : 0.0f;  // NaN and below -86: zero
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

// quantize(weight_of(value, maximum, inv_t)) for value <= maximum or NaN
// (every member of a row: the maximum is the row's largest admitted value),
// without the float scaling and the float-to-u64 conversion. exp_weight's
// result is y * 2^n exactly (y in [0.70, 1.42], n in [-124, 0], a normal
// float), so floor(y * 2^(n + 44)) is the integer Y = y * 2^30 (exact: y
// has 24 mantissa bits and exponent -1 or 0) shifted by n + 14, here
// (Y << 32) >> (18 - n); a shift of 63 gives zero, below -86 or for NaN.
// Checked equal to quantize(exp_weight(x)) for every float x in [-90, 0]
// and NaN. weight_yk returns Y and that shift k = min(18 - n, 63).
struct WeightYK {
  uint32_t Y;
  int k;
};
__device__ __forceinline__ WeightYK weight_yk(float value, float maximum, float inv_t) {
  const float x_in = (value - maximum) * inv_t;
  const float x = __builtin_fminf(__builtin_fmaxf(x_in, -87.0f), 88.0f);
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
  WeightYK w;
  w.Y = (uint32_t)(y * 0x1p30f);
  w.k = x_in >= -86.0f ? min(18 - (int)n, 63) : 63;
  return w;
}
__device__ __forceinline__ uint64_t quantized_weight(float value, float maximum,
                                                     float inv_t) {
  const WeightYK w = weight_yk(value, maximum, inv_t);
  return ((uint64_t)w.Y << 32) >> w.k;
}

// scale_by of the weight (Y << 32) >> k by a packed chunk scale s << 32 | R
// (R < 2^32, s >= 31, or R = 0 with s = 64) in one 32 x 32-bit product: the
// weight is Y (< 2^31) with k in [18, 63], so for k <= 32 it is
// Y * 2^(32 - k) and the scaled weight is (Y * R) >> (s + k - 32); for k > 32
// it is m = Y >> (k - 32) and the scaled weight (m * R) >> s. Both products
// stay below 2^63, so a shift clamped to 63 gives the zero that any larger
// shift would.
__device__ __forceinline__ uint64_t scale_yk(uint32_t Y, int k, uint64_t scale) {
  const uint32_t m = Y >> max(k - 32, 0);
  const int sh = min((int)(scale >> 32) - 32 + min(k, 32), 63);
  return ((uint64_t)m * (uint32_t)scale) >> sh;
}
// scale_by(quantized_weight(value, maximum, inv_t), scale).
__device__ __forceinline__ uint64_t scaled_weight(float value, float maximum, float inv_t,
                                                  uint64_t scale) {
  const WeightYK w = weight_yk(value, maximum, inv_t);
  return scale_yk(w.Y, w.k, scale);
}

// A weight's Y and k in one word: Y's low 6 bits are zero (Y = y * 2^30
// with y's 24-bit mantissa at exponent -1 or 0), so Y >> 6 takes 25 bits,
// and k (at most 63) the 6 above them.
__device__ __forceinline__ uint32_t pack_yk(const WeightYK &w) {
  return (w.Y >> 6) | ((uint32_t)w.k << 25);
}
__device__ __forceinline__ WeightYK unpack_yk(uint32_t p) {
  WeightYK w;
  w.Y = (p & 0x1ffffffu) << 6;
  w.k = (int)(p >> 25);
  return w;
}

// e^x in double: the Cody-Waite reduction x = n ln2 + r (n = rint(x log2 e),
// ln2 split into a 28-bit head, so n * head is exact, and the rounded rest),
// then e^r by its Taylor series to degree 13 in Horner form with fused
// multiply-adds, times 2^n. Each step is one IEEE double operation, so a host
// restatement of the same steps gives the same bits. Zero below -708 (where
// 2^n would leave the normal range) and for NaN.
__device__ __forceinline__ double exp64(double x) {
  if (!(x >= -708.0)) return 0.0;
  if (x > 709.0) return __builtin_inf();
  const double n = __builtin_rint(x * 0x1.71547652b82fep+0);
  double r = __builtin_fma(n, -0x1.62e42ffp-1, x);
  r = __builtin_fma(n, 0x1.718432a1b0e26p-35, r);
  double p = 0x1.6124613a86d09p-33;  // 1/13!
  p = __builtin_fma(p, r, 0x1.1eed8eff8d898p-29);
  p = __builtin_fma(p, r, 0x1.ae64567f544e4p-26);
  p = __builtin_fma(p, r, 0x1.27e4fb7789f5cp-22);
  p = __builtin_fma(p, r, 0x1.71de3a556c734p-19);
  p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-16);
  p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-13);
  p = __builtin_fma(p, r, 0x1.6c16c16c16c17p-10);
  p = __builtin_fma(p, r, 0x1.1111111111111p-7);
  p = __builtin_fma(p, r, 0x1.5555555555555p-5);
  p = __builtin_fma(p, r, 0x1.5555555555555p-3);
  p = __builtin_fma(p, r, 0x1p-1);
  p = __builtin_fma(p, r, 1.0);
  p = __builtin_fma(p, r, 1.0);
  return p * __longlong_as_double((long long)((int64_t)n + 1023) << 52);
}

// A chunk mass's rescale from the chunk's maximum to the row's,
// r = exp64((chunk_max - row_max) * inv_t) (difference and product in double),
// as R * 2^-s with R the significand rounded half up to 32 bits: R in
// [2^31, 2^32), relative error at most 2^-32 at any offset. Packed s << 32 | R;
// r = 0 gives R = 0, s = 64.
__device__ __forceinline__ uint64_t chunk_scale(float chunk_max, float row_max, float inv_t) {
  const double r = exp64(((double)chunk_max - (double)row_max) * (double)inv_t);
  if (!(r > 0.0)) return 64ull << 32;
  const uint64_t bits = (uint64_t)__double_as_longlong(r);
  const int e = (int)(bits >> 52) - 1023;  // r normal: e in [-1022, 0]
  uint64_t R = (((bits & 0xfffffffffffffull) | (1ull << 52)) + (1ull << 20)) >> 21;
  uint64_t s = (uint64_t)(31 - e);
  if (R >> 32) {
    R >>= 1;
    s -= 1;
  }
  return s << 32 | R;
}
// The packed scale of nothing (R = 0).
constexpr uint64_t kZeroScale = 64ull << 32;
// floor(x * R * 2^-s) for x < 2^63 and a packed scale: the 96-bit product
// shifted right by s (s >= 31; at or past 128 nothing remains).
__device__ __forceinline__ uint64_t scale_by(uint64_t x, uint64_t scale) {
  const uint64_t R = scale & 0xffffffffull;
  const uint32_t s = (uint32_t)(scale >> 32);
  const uint64_t lo = x * R, hi = __umul64hi(x, R);
  if (s >= 128) return 0;
  if (s >= 64) return hi >> (s - 64);
  return (hi << (64 - s)) | (lo >> s);
}
// The largest P with scale_by(P, scale) <= within, for R > 0 and a within
// below scale_by(x, scale) for some x < 2^63 (the chunk the draw chose):
// floor(((within + 1) * 2^s - 1) / R). The numerator N stays below
// x * R < 2^95, so N is built as two 64-bit words and divided by R in four
// 32-bit digits (each partial dividend below R * 2^32 < 2^64).
__device__ __forceinline__ uint64_t unscaled_bound(uint64_t within, uint64_t scale) {
  const uint64_t R = scale & 0xffffffffull;
  const uint32_t s = (uint32_t)(scale >> 32);
  const uint64_t n = within + 1;
  uint64_t hi, lo;
  if (s >= 64) {
    hi = n << (s - 64);
    lo = 0;
  } else {
    hi = n >> (64 - s);  // s >= 31
    lo = n << s;
  }
  // N - 1 (N >= 2^31 > 0).
  if (lo == 0) --hi;
  --lo;
  uint64_t q = 0, rem = 0;
  const uint32_t digit[4] = {(uint32_t)(hi >> 32), (uint32_t)hi, (uint32_t)(lo >> 32),
                             (uint32_t)lo};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint64_t cur = (rem << 32) | digit[d];
    q = (q << 32) | (cur / R);
    rem = cur % R;
  }
  return q;
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

// Lane exchanges without the LDS crossbar: DPP quad permutes for xor 1 and
// 2, DPP row shifts for xor 4 and 8 (both partners lie in the same 16-lane
// row), and gfx950's lane swaps for xor 16 and 32. v_permlane16_swap of a
// value with itself leaves, in every lane, the value of the even row of its
// row pair (rows 0,1 and 2,3) in the first result and the odd row's in the
// second; v_permlane32_swap likewise the lower half's and the upper half's.
// The partner's is the one of the other row (half). Exchanges are made with
// the whole wave active.
template <int M>
__device__ __forceinline__ uint32_t xor_u32(uint32_t v) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32);
  if constexpr (M == 1) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);
  } else if constexpr (M == 2) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);
  } else if constexpr (M == 4 || M == 8) {
    // row_shl:M reads lane i + M, row_shr:M reads lane i - M.
    const uint32_t up = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x100 + M, 0xF, 0xF, false);
    const uint32_t dn = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x110 + M, 0xF, 0xF, false);
    return (lane_id() & M) ? dn : up;
  } else if constexpr (M == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (lane_id() & 16) ? (uint32_t)p[0] : (uint32_t)p[1];
  } else {
    const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (lane_id() & 32) ? (uint32_t)p[0] : (uint32_t)p[1];
  }
}
template <int M>
__device__ __forceinline__ float xor_f32(float v) {
  return __uint_as_float(xor_u32<M>(__float_as_uint(v)));
}
template <int M>
__device__ __forceinline__ uint64_t xor_u64(uint64_t v) {
  return ((uint64_t)xor_u32<M>((uint32_t)(v >> 32)) << 32) | xor_u32<M>((uint32_t)v);
}
// Lane i - D within its 16-lane row, or 0 for the first D lanes of a row.
template <int D>
__device__ __forceinline__ uint32_t row_shr_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x110 + D, 0xF, 0xF, true);
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
__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
  const uint32_t lo = __shfl((uint32_t)v, src, kWave);
  const uint32_t hi = __shfl((uint32_t)(v >> 32), src, kWave);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
  return ((uint64_t)readlane_u32((uint32_t)(v >> 32), l) << 32) | readlane_u32((uint32_t)v, l);
}

// Butterfly reductions: every lane ends with the wave's result.
#define JF_BUTTERFLY(T, XOR, OP)                                   \
  v = OP(v, XOR<1>(v));                                            \
  v = OP(v, XOR<2>(v));                                            \
  v = OP(v, XOR<4>(v));                                            \
  v = OP(v, XOR<8>(v));                                            \
  v = OP(v, XOR<16>(v));                                           \
  v = OP(v, XOR<32>(v));                                           \
  return v;

__device__ __forceinline__ uint32_t add_u32(uint32_t a, uint32_t b) { return a + b; }
__device__ __forceinline__ uint64_t add_u64(uint64_t a, uint64_t b) { return a + b; }
__device__ __forceinline__ uint32_t max_u32(uint32_t a, uint32_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint32_t min_u32(uint32_t a, uint32_t b) { return a < b ? a : b; }
__device__ __forceinline__ float max_f32(float a, float b) { return __builtin_fmaxf(a, b); }

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) { JF_BUTTERFLY(uint32_t, xor_u32, add_u32) }
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) { JF_BUTTERFLY(uint64_t, xor_u64, add_u64) }
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) { JF_BUTTERFLY(uint32_t, xor_u32, max_u32) }
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) { JF_BUTTERFLY(uint32_t, xor_u32, min_u32) }
__device__ __forceinline__ float wave_max_f32(float v) { JF_BUTTERFLY(float, xor_f32, max_f32) }
#undef JF_BUTTERFLY

// Several wave totals at once: v[j] are the lane's N (4 or 8) values, and
// lane l gets the wave's total of v[j] for j = l / (64 / N). Each exchange
// step halves what a lane carries: a lane whose bit is clear keeps the
// lower half of its values and sends the upper half to its partner, which
// does the opposite. The lanes that share a j then add up their partials.
// About a third of the instructions of N separate butterflies.
template <int N>
__device__ __forceinline__ uint64_t wave_sums_u64(const uint64_t (&v)[N]) {
  static_assert(N == 4 || N == 8, "four or eight values per lane");
  const uint32_t l = lane_id();
  const bool h5 = (l >> 5) & 1u, h4 = (l >> 4) & 1u;
  constexpr int H = N / 2;
  uint64_t a[H];
#pragma unroll
  for (int k = 0; k < H; ++k) {
    const uint64_t keep = h5 ? v[H + k] : v[k], send = h5 ? v[k] : v[H + k];
    a[k] = keep + xor_u64<32>(send);
  }
  uint64_t c;
  if constexpr (N == 8) {
    const bool h3 = (l >> 3) & 1u;
    uint64_t b[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const uint64_t keep = h4 ? a[2 + k] : a[k], send = h4 ? a[k] : a[2 + k];
      b[k] = keep + xor_u64<16>(send);
    }
    c = (h3 ? b[1] : b[0]) + xor_u64<8>(h3 ? b[0] : b[1]);
  } else {
    c = (h4 ? a[1] : a[0]) + xor_u64<16>(h4 ? a[0] : a[1]);
    c += xor_u64<8>(c);
  }
  c += xor_u64<4>(c);
  c += xor_u64<2>(c);
  c += xor_u64<1>(c);
  return c;
}

// Inclusive prefix sums over lanes: row-wise by DPP shifts, then the
// totals of the rows before (lanes 15, 31, 47) added.
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  v += row_shr_u32<1>(v);
  v += row_shr_u32<2>(v);
  v += row_shr_u32<4>(v);
  v += row_shr_u32<8>(v);
  const uint32_t r0 = readlane_u32(v, 15), r1 = readlane_u32(v, 31),
                 r2 = readlane_u32(v, 47);
  const uint32_t row = lane_id() >> 4;
  return v + (row >= 1 ? r0 : 0u) + (row >= 2 ? r1 : 0u) + (row >= 3 ? r2 : 0u);
}
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t v) {
  auto shr = [](uint64_t x, auto d) -> uint64_t {
    constexpr int D = decltype(d)::value;
    return ((uint64_t)row_shr_u32<D>((uint32_t)(x >> 32)) << 32) | row_shr_u32<D>((uint32_t)x);
  };
  v += shr(v, std::integral_constant<int, 1>{});
  v += shr(v, std::integral_constant<int, 2>{});
  v += shr(v, std::integral_constant<int, 4>{});
  v += shr(v, std::integral_constant<int, 8>{});
  const uint64_t r0 = readlane_u64(v, 15), r1 = readlane_u64(v, 31),
                 r2 = readlane_u64(v, 47);
  const uint32_t row = lane_id() >> 4;
  return v + (row >= 1 ? r0 : 0ull) + (row >= 2 ? r1 : 0ull) + (row >= 3 ? r2 : 0ull);
}

// The largest greedy candidate of the wave: larger value, then lower id.
__device__ __forceinline__ void wave_argmax(float &value, uint32_t &id) {
  auto step = [&](float ov, uint32_t oi) {
    if (ov > value || (ov == value && oi < id)) {
      value = ov;
      id = oi;
    }
  };
  step(xor_f32<1>(value), xor_u32<1>(id));
  step(xor_f32<2>(value), xor_u32<2>(id));
  step(xor_f32<4>(value), xor_u32<4>(id));
  step(xor_f32<8>(value), xor_u32<8>(id));
  step(xor_f32<16>(value), xor_u32<16>(id));
  step(xor_f32<32>(value), xor_u32<32>(id));
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

// Bitonic sort of one 32-bit value per lane over the wave, ascending.
__device__ __forceinline__ uint32_t wave_sort_asc_u32(uint32_t v) {
  const uint32_t lane = lane_id();
#pragma unroll
  for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      uint32_t o;
      switch (j) {
        case 1: o = xor_u32<1>(v); break;
        case 2: o = xor_u32<2>(v); break;
        case 4: o = xor_u32<4>(v); break;
        case 8: o = xor_u32<8>(v); break;
        case 16: o = xor_u32<16>(v); break;
        default: o = xor_u32<32>(v); break;
      }
      const bool lower = (lane & j) == 0;
      const bool block_asc = (lane & k) == 0;
      const bool take_smaller = lower == block_asc;
      v = take_smaller ? min(v, o) : max(v, o);
    }
  }
  return v;
}

}  // namespace jf
