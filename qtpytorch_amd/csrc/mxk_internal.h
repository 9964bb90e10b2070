// Internal helpers shared by the libmxk HIP sources (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bfloat16.h>
#include <stdint.h>
#include <string>

#include "../../include/mxk.h"

namespace mxk {

// ---------------------------------------------------------------- errors
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }
inline int64_t next_pow2(int64_t v) {
  int64_t p = 1;
  while (p < v) p <<= 1;
  return p;
}
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Number of CUs of the current device (cached per device).
int num_cus();

// ---------------------------------------------------------------- device math
// Quantizer modes.
enum QMode : int { Q_INT = 0, Q_INT1 = 1, Q_VEC = 2, Q_FP = 3 };

// fl32(1e-12): the clamp(min=1e-12) of every quantizer (mxtorch.py:1444,1458,1497,1748).
#define MXK_AMIN 9.99999996e-13f

// IEEE division a/b given y = RN(1/b), by Markstein's correction
// (q0 = RN(a*y); r = a - b*q0 exactly by FMA; q1 = RN(q0 + r*y)).  The
// residual is exact and the result correctly rounded when |a| >= 2^-96 and
// b, a/b are normal; below that the hardware divide sequence is used.
__device__ __forceinline__ float div_rn(float a, float b, float y) {
  if (__builtin_expect(__builtin_fabsf(a) < 0x1p-96f, 0)) return a / b;
  float q0 = a * y;
  float r = __builtin_fmaf(-q0, b, a);
  return __builtin_fmaf(r, y, q0);
}

// The same quotient without the per-element check, for callers that have
// already established that no lane of the wave holds a nonzero |a| < 2^-96
// (div_rn_all): a per-element branch costs more than the division itself.
// For b > 0 the quotient has the sign of a, zeros included, and the final
// copysign restores it where the last FMA would turn -0 into +0.
__device__ __forceinline__ float div_rn_nochk(float a, float b, float y) {
  float q0 = a * y;
  float r = __builtin_fmaf(-q0, b, a);
  return __builtin_copysignf(__builtin_fmaf(r, y, q0), a);
}

// v[i] = RN(v[i] / b) for E values and b > 0: one wave-wide vote on the
// smallest nonzero magnitude picks the Markstein path for the whole wave, or
// the hardware divide when any lane holds a nonzero value below 2^-96.
// (bits << 1) - 1 orders the nonzero magnitudes and sends both zeros to
// 0xFFFFFFFF, so its minimum is below 2 * bits(2^-96) - 1 exactly when some
// value has 0 < |v| < 2^-96; true when any lane of the wave holds one.
template <int E>
__device__ __forceinline__ bool any_tiny(const float (&v)[E]) {
  uint32_t mnb = 0xFFFFFFFFu;
#pragma unroll
  for (int i = 0; i < E; ++i) mnb = min(mnb, (__float_as_uint(v[i]) << 1) - 1u);
  return __ballot(mnb < 2u * 0x0F800000u - 1u) != 0ull;
}

template <int E>
__device__ __forceinline__ void div_rn_all(float (&v)[E], float b, float y) {
  if (__builtin_expect(any_tiny<E>(v), 0)) {
#pragma unroll
    for (int i = 0; i < E; ++i) v[i] = v[i] / b;
  } else {
#pragma unroll
    for (int i = 0; i < E; ++i) v[i] = div_rn_nochk(v[i], b, y);
  }
}

__device__ __forceinline__ float rne(float v) { return __builtin_rintf(v); }

// Lane-group max over `G` consecutive lanes (G a power of two <= 64); every
// lane of the group ends with the group maximum.
template <int G>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (G >= 2)
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true)));
  if constexpr (G >= 4)
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true)));
  if constexpr (G >= 8)  // row_half_mirror: lane i <-> 7-i within 8
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true)));
  if constexpr (G >= 16)  // row_mirror: lane i <-> 15-i within 16
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true)));
  if constexpr (G >= 32)  // swap 16-lane halves of each 32
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F)));
  if constexpr (G >= 64) v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

// NaN-propagating block maxima.  torch's amax returns NaN for a block that
// holds a NaN and clamp(min=1e-12) keeps it (mxtorch.py:1456-1457, 1497,
// 1748), so that block's scale is NaN.  Magnitudes compared as unsigned
// integers order like floats, and every NaN (sign cleared) sorts above
// +inf, so an integer maximum over the magnitude bits propagates it.
__device__ __forceinline__ uint32_t mag_bits(float v) { return __float_as_uint(v) & 0x7FFFFFFFu; }

template <int G>
__device__ __forceinline__ uint32_t group_max_u(uint32_t v) {
  if constexpr (G >= 2) v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true));
  if constexpr (G >= 4) v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, true));
  if constexpr (G >= 8) v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, true));
  if constexpr (G >= 16) v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, true));
  if constexpr (G >= 32) v = max(v, (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x401F));
  if constexpr (G >= 64) v = max(v, (uint32_t)__shfl_xor((int)v, 32));
  return v;
}

// max(a, fl32(1e-12)) of a magnitude given by its bits, keeping a NaN
__device__ __forceinline__ float amax_clamped(uint32_t m) {
  return __uint_as_float(max(m, __float_as_uint(MXK_AMIN)));
}

// ---------------------------------------------------------------- element loads
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4v __attribute__((ext_vector_type(4)));
template <typename T> struct ElemT;
template <> struct ElemT<float> {
  static __device__ __forceinline__ float cvt(float v) { return v; }
};
template <> struct ElemT<__half> {
  static __device__ __forceinline__ float cvt(__half v) { return __half2float(v); }
};
template <> struct ElemT<hip_bfloat16> {
  static __device__ __forceinline__ float cvt(hip_bfloat16 v) {
    return __uint_as_float(static_cast<uint32_t>(reinterpret_cast<const uint16_t&>(v)) << 16);
  }
};

// Load E consecutive elements starting at `idx` as float; elements at or
// beyond n read as +0.0 (the reference zero-pads the last block).  A full
// in-range group uses 16-byte loads (the caller guarantees alignment).
template <typename T, int E>
__device__ __forceinline__ void load_elems(const T* __restrict__ x, int64_t idx, int64_t n,
                                           float (&v)[E]) {
  constexpr int PER16 = 16 / sizeof(T);
  static_assert(E % PER16 == 0, "E must cover whole 16-byte vectors");
  if (idx + E <= n) {
    const u32x4* p = reinterpret_cast<const u32x4*>(x + idx);
#pragma unroll
    for (int q = 0; q < E / PER16; ++q) {
      u32x4 w = __builtin_nontemporal_load(p + q);
      const T* t = reinterpret_cast<const T*>(&w);
#pragma unroll
      for (int i = 0; i < PER16; ++i) v[q * PER16 + i] = ElemT<T>::cvt(t[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < E; ++i) v[i] = (idx + i < n) ? ElemT<T>::cvt(x[idx + i]) : 0.0f;
  }
}

// Raw buffer resource over [p, p + bytes): loads past the end return 0
// (hardware range check), offsets are 32-bit (one per lane + one scalar).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint32_t buf_load_b32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0);
}
__device__ __forceinline__ u32x4 buf_load_b128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}
// Non-temporal loads (cache policy nt) for streams read exactly once, such
// as a decode's weights and scales: they then do not displace the lines
// that other workgroups re-read (x, partials) in L2.  Config 2 decode:
// 12.98 -> 12.5 us per step.
__device__ __forceinline__ uint32_t buf_load_b32_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 2);
}
__device__ __forceinline__ u32x4 buf_load_b128_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 2));
}

// Store `NB` bytes from `w` at dst+off when they fit below `limit`; bytes at
// or past `limit` are dropped (tail of a packed buffer).
template <int NB>
__device__ __forceinline__ void store_bytes(uint8_t* __restrict__ dst, int64_t off, int64_t limit,
                                            const uint32_t* w) {
  if (off + NB <= limit) {
    if constexpr (NB == 1) dst[off] = static_cast<uint8_t>(w[0]);
    else if constexpr (NB == 2) *reinterpret_cast<uint16_t*>(dst + off) = static_cast<uint16_t>(w[0]);
    else if constexpr (NB == 4) *reinterpret_cast<uint32_t*>(dst + off) = w[0];
    else if constexpr (NB == 8) *reinterpret_cast<u32x2*>(dst + off) = u32x2{w[0], w[1]};
    else if constexpr (NB == 16)
      *reinterpret_cast<u32x4*>(dst + off) = u32x4{w[0], w[1], w[2], w[3]};
    else if constexpr (NB == 32) {
      *reinterpret_cast<u32x4*>(dst + off) = u32x4{w[0], w[1], w[2], w[3]};
      *reinterpret_cast<u32x4*>(dst + off + 16) = u32x4{w[4], w[5], w[6], w[7]};
    }
  } else {
    for (int b = 0; b < NB; ++b)
      if (off + b < limit) dst[off + b] = static_cast<uint8_t>(w[b >> 2] >> ((b & 3) * 8));
  }
}

// Zeroes the fields of codes at positions >= lim (lim may be <= 0) in a
// lane's NW words of BITS-bit fields (code i at bit i * BITS): the codes a
// quantizer writes past n_store.  Called only for the lanes that reach the
// end, so the other lanes skip a per-code comparison.
template <int NW, int BITS>
__device__ __forceinline__ void clear_tail(uint32_t (&w)[NW], int64_t lim) {
#pragma unroll
  for (int k = 0; k < NW; ++k) {
    const int64_t keep = lim * BITS - 32 * k;
    w[k] &= keep >= 32 ? 0xFFFFFFFFu : (keep <= 0 ? 0u : ((1u << keep) - 1u));
  }
}

// ---------------------------------------------------------------- float grids
// Positive grid magnitude of code c (c < 2^(bits-1)), in units of the
// format's largest value, exactly as _get_minifloat_grid builds it
// (mxtorch.py:1023-1054): FP4 E2M1 values /6, FP8 E4M3 values (exponent 15
// is a normal binade, max 480) /480, each an IEEE float32 division.
__host__ __device__ inline float fmt_value(int bits, int c) {
  if (bits == 4) {
    int e = c >> 1, m = c & 1;
    return e == 0 ? 0.5f * (float)m : ldexpf((float)(2 + m), e - 2);
  }
  int e = c >> 3, m = c & 7;
  return e == 0 ? ldexpf((float)m, -9) : ldexpf((float)(8 + m), e - 10);
}
__host__ __device__ inline float fmt_max(int bits) { return bits == 4 ? 6.0f : 480.0f; }

// LDS tables for a float format with H = 2^(bits-1):
//   P[0] = -inf, P[j] = RN(RN(g[j-1]+g[j])*0.5) for j in [1,H), P[H] = +inf
//   G[0..2H): the sorted grid; G[H-1] = -0.0, G[H] = +0.0 (torch.sort's order).
template <int BITS>
__device__ void build_tables(float* P, float* G) {
  constexpr int H = 1 << (BITS - 1);
  __shared__ float g[H];
  for (int c = threadIdx.x; c < H; c += blockDim.x) g[c] = fmt_value(BITS, c) / fmt_max(BITS);
  __syncthreads();
  for (int j = threadIdx.x; j <= H; j += blockDim.x) {
    if (P) P[j] = j == 0 ? -INFINITY : (j == H ? INFINITY : (g[j - 1] + g[j]) * 0.5f);
  }
  if (G)
    for (int c = threadIdx.x; c < H; c += blockDim.x) {
      G[H + c] = g[c];
      G[H - 1 - c] = -g[c];
    }
  __syncthreads();
}

// Value of sorted-grid index f of the 8-bit float format without a table
// (G[f] of build_tables<8>): codes 0..127 are the negative half, in
// decreasing magnitude, so the magnitude index is c = f ^ 0x7F there and
// f - 128 above.  With e = c >> 3 and mantissa m = c & 7 (plus 8 when e > 0),
// fmt_value(c) / 480 = (m / 15) * 2^(max(e,1) - 15); the power of two scales
// exactly (the smallest nonzero value, 2^-14 / 15, is normal), so the value
// is RN(m / 15) scaled, and RN(m / 15) is the exactly rounded quotient of two
// small integers.  Index 127 gives -0.0, as in the table.
__device__ __forceinline__ float fp8_grid_value(uint32_t f) {
  const uint32_t neg = ((f >> 7) & 1u) ^ 1u;
  const uint32_t c = (f ^ (neg * 0x7Fu)) & 0x7Fu;
  const uint32_t e = c >> 3;
  const float m = (float)((c & 7u) | (e != 0u ? 8u : 0u));
  const float q = div_rn_nochk(m, 15.0f, 0x1.111112p-4f);  // RN(1/15)
  const float g = __builtin_ldexpf(q, (int)(e != 0u ? e : 1u) - 15);
  return neg ? -g : g;
}

// Index of y in the sorted grid: #{mids < y} (torch.bucketize, right=False).
// By the grid's symmetry this is H + #{P_j < |y|} for y > 0 and
// H-1 - #{P_j <= |y|} otherwise.  The count comes from rounding |y| to the
// nearest format value (a candidate at most one off) and one comparison
// with each neighbouring midpoint.
template <int BITS>
__device__ __forceinline__ int bucket(float y, const float* __restrict__ P) {
  constexpr int H = 1 << (BITS - 1);
  float a = __builtin_fabsf(y);
  int c0;
  if constexpr (BITS == 8) {
    float t = a * 480.0f;
    c0 = t < 0x1p-6f ? (int)__builtin_rintf(t * 512.0f) : (int)((__float_as_uint(t) + 0x80000u) >> 20) - 960;
  } else {
    float t = a * 6.0f;
    c0 = t < 1.0f ? (int)__builtin_rintf(t * 2.0f) : (int)((__float_as_uint(t) + 0x200000u) >> 22) - 252;
  }
  c0 = min(max(c0, 0), H - 1);
  float lo = P[c0], hi = P[c0 + 1];
  if (y > 0.0f) return H + c0 + (hi < a ? 1 : 0) - (lo >= a ? 1 : 0);
  return (H - 1) - (c0 + (hi <= a ? 1 : 0) - (lo > a ? 1 : 0));
}

// ---------------------------------------------------------------- per-block params
struct BlockParams {
  float s;    // stored scale
  float mul;  // Q_INT: inv ; Q_VEC/Q_FP: RN(1/s)
};

template <int MODE>
__device__ __forceinline__ BlockParams block_params(float ap, float qf) {
  BlockParams bp;
  if constexpr (MODE == Q_INT) {
    float r = 1.0f / ap;
    bp.mul = r * qf;
    bp.s = 1.0f / bp.mul;
  } else if constexpr (MODE == Q_VEC) {
    bp.s = ap / qf;
    bp.mul = 1.0f / bp.s;
  } else {  // Q_INT1, Q_FP
    bp.s = ap;
    bp.mul = 1.0f / ap;
  }
  // a NaN scale is stored as the reference's host makes it: 0x7FC00000
  if (!(bp.s == bp.s)) bp.s = __uint_as_float(0x7FC00000u);
  return bp;
}

// The positive mids of the normalized E2M1 grid: RN((g[j-1] + g[j]) * 0.5)
// with g[c] = RN(v_c / 6) in float32, the values build_tables computes.
namespace fp4c {
constexpr float g1 = 0.5f / 6.0f, g2 = 1.0f / 6.0f, g3 = 1.5f / 6.0f, g4 = 2.0f / 6.0f, g5 = 3.0f / 6.0f,
                g6 = 4.0f / 6.0f, g7 = 6.0f / 6.0f;
constexpr float P1 = (0.0f + g1) * 0.5f, P2 = (g1 + g2) * 0.5f, P3 = (g2 + g3) * 0.5f, P4 = (g3 + g4) * 0.5f,
                P5 = (g4 + g5) * 0.5f, P6 = (g5 + g6) * 0.5f, P7 = (g6 + g7) * 0.5f;
}  // namespace fp4c

// bucket<4> without the table: #{mids < a} comes from a binary search over
// the constant mids (three comparisons, selects, no LDS); for y <= 0 the
// count of mids <= |y| is the count of mids < nextup(|y|).  Equal to
// bucket<4> for every finite y (checked exhaustively over all float32
// patterns); a NaN takes the last index, as torch.bucketize gives it.
__device__ __forceinline__ int bucket_fp4(float y) {
  using namespace fp4c;
  const float a0 = __builtin_fabsf(y);
  const bool pos = !(y <= 0.0f);
  const float a = pos ? a0 : __uint_as_float(__float_as_uint(a0) + 1u);
  // !(a <= P) is a > P for numbers and true for a NaN
  int c = !(a <= P4) ? 4 : 0;
  c += !(a <= (c ? P6 : P2)) ? 2 : 0;
  c += !(a <= (c == 6 ? P7 : (c == 4 ? P5 : (c == 2 ? P3 : P1)))) ? 1 : 0;
  return pos ? 8 + c : 7 - c;
}

// bucket<BITS> through an LDS table keyed by the top bits of the
// magnitude.  FP4: key k = clamp((bits >> 21) - 488, 0, 31), a quarter
// binade from 2^-5 on ([0, 1.25 * 2^-5) for k = 0, [7, inf] and NaN for
// k = 31).  FP8: k = clamp((bits >> 19) - 1728, 0, 304), a sixteenth of a
// binade from 2^-19 on (below the smallest mid, 2^-9 / 960) up to [1, inf]
// and NaN.  Each key's interval holds at most one mid (consecutive mids are
// more than one key apart), so #{mids < a} = T[k].x + (a > T[k].y) with
// T[k] = (#mids below the interval, the mid inside it or +inf).  For y <= 0
// it counts the mids below nextup(|y|), and H + c / H - 1 - c are c ^ H /
// c ^ (H - 1).  One LDS read and ~10 VALU per element against ~15 (FP4
// search over constant mids) or ~18 (FP8 candidate and two mids); float4d
// quantize at 2^28: 265 -> 228 us.  Equal to torch.bucketize over the mids
// for every float32 pattern, NaN included (last index), checked exhaustively.
template <int BITS> struct FpKeys;
template <> struct FpKeys<4> { static constexpr int N = 32, SHIFT = 21, BASE = 488; };
template <> struct FpKeys<8> { static constexpr int N = 305, SHIFT = 19, BASE = 1728; };

// P: the positive mids at P[1..H-1] (build_tables<8>'s table; FP4 uses its
// constants and ignores P)
template <int BITS>
__device__ __forceinline__ void build_fp_keys(int2* T, const float* P) {
  constexpr int H = 1 << (BITS - 1);
  using K = FpKeys<BITS>;
  for (int k = threadIdx.x; k < K::N; k += blockDim.x) {
    const float lo = k == 0 ? 0.0f : __uint_as_float((uint32_t)(k + K::BASE) << K::SHIFT);
    const float hi = k == K::N - 1 ? __builtin_inff() : __uint_as_float((uint32_t)(k + K::BASE + 1) << K::SHIFT);
    int cnt = 0;
    float mid = __builtin_inff();
    if constexpr (BITS == 4) {
      using namespace fp4c;
      const float Q[7] = {P1, P2, P3, P4, P5, P6, P7};
#pragma unroll
      for (int j = 0; j < 7; ++j) {
        if (Q[j] < lo) ++cnt;
        else if (Q[j] < hi) mid = Q[j];
      }
    } else {
      // cnt = #{P[1..H-1] < lo} by bisection over the sorted mids
      int a = 0, b = H - 1;
      while (a < b) {
        const int m = (a + b + 1) >> 1;
        if (P[m] < lo) a = m;
        else b = m - 1;
      }
      cnt = a;
      if (cnt + 1 <= H - 1 && P[cnt + 1] < hi) mid = P[cnt + 1];
    }
    T[k] = make_int2(cnt, __float_as_int(mid));
  }
  __syncthreads();
}

template <int BITS>
__device__ __forceinline__ int bucket_keyed(float y, const int2* __restrict__ T) {
  constexpr int H = 1 << (BITS - 1);
  using K = FpKeys<BITS>;
  const bool pos = !(y <= 0.0f);
  const uint32_t ab = (__float_as_uint(y) & 0x7FFFFFFFu) + (pos ? 0u : 1u);
  // the key clamped before the base is taken off (one v_med3_u32; the
  // subtraction folds into the table address)
  const uint32_t kc = min(max(ab >> K::SHIFT, (uint32_t)K::BASE), (uint32_t)(K::BASE + K::N - 1));
  const int2 e = T[kc - (uint32_t)K::BASE];
  const int c = e.x + (__uint_as_float(ab) > __int_as_float(e.y) ? 1 : 0);
  return c ^ (pos ? H : H - 1);
}

template <int MODE, int BITS>
__device__ __forceinline__ int encode(float v, const BlockParams& bp, float qf, const float* P) {
  if constexpr (MODE == Q_INT) {
    // rne of the clamped product by the float adder: t + 1.5 * 2^23 (|t| <=
    // q <= 2^15) is rounded to an integer with ties to even and leaves
    // 2^22 + 2^23 + rne(t) in the significand, so the integer is the bit
    // pattern minus that of 1.5 * 2^23 (one add and one subtract in place
    // of a round and a conversion; callers that mask the low bits lose the
    // subtract)
    const float t = __builtin_amdgcn_fmed3f(v * bp.mul, -qf, qf);  // the clamp, one instruction
    return (int)(__float_as_uint(t + 12582912.0f) - 0x4B400000u);
  } else if constexpr (MODE == Q_INT1) {
    return v >= 0.0f ? 0 : 1;
  } else if constexpr (MODE == Q_VEC) {
    return (int)rne(fminf(fmaxf(div_rn(v, bp.s, bp.mul), -qf), qf));
  } else if constexpr (BITS == 4) {
    return bucket_fp4(div_rn(v, bp.s, bp.mul));
  } else {
    return bucket<BITS>(div_rn(v, bp.s, bp.mul), P);
  }
}

// Codes of a block whose scale is not finite (a NaN in the block makes it
// NaN, an infinity makes it +inf), as the reference's CPU path computes
// them: the quotient by a true division (the multiplier of Q_INT is then
// NaN or 0); a NaN quotient converts to INT_MIN on the reference's host,
// whose stored field is 0, and a float code is bucketize's last index for
// it; int1 codes take the sign rule as always.  Out of the hot loops:
// kernels branch here per block.
template <int MODE, int BITS>
__device__ __forceinline__ int encode_nonfinite(float v, const BlockParams& bp, float qf, const float* P) {
  if constexpr (MODE == Q_INT1) {
    return v >= 0.0f ? 0 : 1;
  } else if constexpr (MODE == Q_FP) {
    const float y = v / bp.s;
    if (!(y == y)) return (1 << BITS) - 1;
    if constexpr (BITS == 4) return bucket_fp4(y);
    else return bucket<BITS>(y, P);
  } else {
    const float y = MODE == Q_INT ? v * bp.mul : v / bp.s;
    if (!(y == y)) return 0;
    return (int)rne(fminf(fmaxf(y, -qf), qf));
  }
}
__device__ __forceinline__ bool finite_scale(float s) { return __builtin_fabsf(s) < __builtin_inff(); }

// encode<> with float codes through the key table of build_fp_keys (T
// unused for the other formats)
template <int MODE, int BITS>
__device__ __forceinline__ int encode_keyed(float v, const BlockParams& bp, float qf, const float* P, const int2* T) {
  if constexpr (MODE == Q_FP) return bucket_keyed<BITS>(div_rn(v, bp.s, bp.mul), T);
  else return encode<MODE, BITS>(v, bp, qf, P);
}

// LDS entries of a kernel's key table (1 when it encodes no float codes)
template <int MODE, int BITS>
constexpr int fp_keys_n() {
  if constexpr (MODE == Q_FP) return FpKeys<BITS>::N;
  else return 1;
}

// The 'v' rule over E values of a block at once: the quotients RN(v / s)
// with one wave-wide vote for the division path (div_rn_all), then
// encode_vec_q encodes a quotient exactly as encode<Q_VEC> encodes the value.
__device__ __forceinline__ int encode_vec_q(float u, float qf) {
  const float t = __builtin_amdgcn_fmed3f(u, -qf, qf);
  return (int)(__float_as_uint(t + 12582912.0f) - 0x4B400000u);
}

// ---------------------------------------------------------------- decode
// Value of the field at bit `sh` of `word` for scale s (sG: the sorted grid
// of a 4-bit float format; the 8-bit format decodes arithmetically).
template <int MODE, int BITS>
__device__ __forceinline__ float decode_field(uint32_t word, int sh, float s, const float* sG) {
  if constexpr (MODE == Q_INT1) {
    return ((word >> sh) & 1u) == 0u ? s : -s;
  } else if constexpr (MODE == Q_FP && BITS == 8) {
    return fp8_grid_value((word >> sh) & 0xFFu) * s;
  } else if constexpr (MODE == Q_FP) {
    return sG[(word >> sh) & ((1u << BITS) - 1u)] * s;
  } else {
    const int32_t c = (int32_t)(word << (32 - BITS - sh)) >> (32 - BITS);
    return (float)c * s;
  }
}

// vector_quantize per row (mxtorch.py:2946-2987: the 'v' rule with block =
// row, int32 codes unpacked): launches the long-block row quantizer with
// 32-bit fields when the shape suits it (16-byte aligned x and codes, rows
// of 264..8192 elements, a multiple of 8); returns false otherwise.
bool vec_rows_i32(const void* x, int x_type, int64_t rows, int64_t cols, int bits, int32_t* codes, float* scales,
                  hipStream_t st);

// MFMA weight-only linear (mxk_linear_mfma.hip) for int4/int8 weights with
// blocks of 128 and N a multiple of 128: [K][N] weights (mx_linear) and
// [N][K] weights (K a multiple of 128).  Workspace bytes (0 when the shape is
// not taken; the first 64 KiB are left untouched), and the products, which
// return MXK_EUNSUPPORTED with nothing launched for shapes they do not take.
size_t linear_mfma_workspace(int64_t M, int64_t K, int64_t N, int bits, int block, bool nk);
int linear_mfma_kn(const void* x, int x_type, int64_t M, int64_t K, const void* w_packed, const float* w_scales,
                   const float* w_scales_t, int64_t N, int kind, int bits, int block, const float* bias, float* out,
                   void* workspace, size_t workspace_nbytes, hipStream_t st);
// [K][N] int4 weight in the tiled layout of mxk_linear_prepack_weight (K % 32 == 0)
int linear_mfma_kn_tiled(const void* x, int x_type, int64_t M, int64_t K, const void* w_tiled,
                         const float* w_scales_t, int64_t N, const float* bias, float* out, void* workspace,
                         size_t workspace_nbytes, hipStream_t st);
int linear_mfma_nk(const void* x, int x_type, int64_t M, int64_t K, const void* w_packed, const float* w_scales,
                   const float* w_scales_t, int64_t N, int kind, int bits, int block, const float* bias, float* out,
                   void* workspace, size_t workspace_nbytes, hipStream_t st);
// [N][K] int4 weights as their tiled copy (k_tile_w4t's layout) with
// K-block-major scales [K/128][N]: the MFMA path of mxk_linear_wq_nt_tiled
int linear_mfma_nk_tiled(const void* x, int x_type, int64_t M, int64_t K, const void* w_tiled,
                         const float* w_scales_t, int64_t N, const float* bias, float* out, void* workspace,
                         size_t workspace_nbytes, hipStream_t st);

// 'v'-rule requantization of a float32 buffer (GEMM outputs), mxtorch.py:1372-1385.
int requant_vec_f32(const float* x, int64_t n, int bits, int block, void* packed, int64_t packed_nbytes,
                    float* scales, int64_t n_store, void* ws, size_t ws_bytes, hipStream_t st);

}  // namespace mxk
