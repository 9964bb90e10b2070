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

// Unsigned 32-bit division by an invariant d >= 1 (Granlund and Montgomery,
// "Division by Invariant Integers using Multiplication", PLDI 1994, fig.
// 4.1): with l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1, sh1 =
// min(l, 1), sh2 = max(l - 1, 0), t = mulhi(m, n):
// n / d = (t + ((n - t) >> sh1)) >> sh2 for every 0 <= n < 2^32.  Five VALU
// in place of a 64-bit division (~66 VALU and ~67 SALU).
struct DivU32 {
  uint32_t m;
  int sh1, sh2;
};
inline DivU32 make_divu32(uint32_t d) {
  int l = 0;
  while (l < 32 && (1ull << l) < (uint64_t)d) ++l;
  DivU32 r;
  r.m = (uint32_t)((((1ull << l) - (uint64_t)d) << 32) / (uint64_t)d + 1ull);
  r.sh1 = l < 1 ? l : 1;
  r.sh2 = l - 1 > 0 ? l - 1 : 0;
  return r;
}
__device__ __forceinline__ uint32_t divu32(uint32_t n, const DivU32& d) {
  const uint32_t t = __umulhi(d.m, n);
  return (t + ((n - t) >> d.sh1)) >> d.sh2;
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
// E in-range elements at p (16-byte aligned) as float, no range check
template <typename T, int E>
__device__ __forceinline__ void load_whole(const T* __restrict__ p, float (&v)[E]) {
  constexpr int PER16 = 16 / sizeof(T);
  static_assert(E % PER16 == 0, "E must cover whole 16-byte vectors");
  const u32x4* p4 = reinterpret_cast<const u32x4*>(p);
#pragma unroll
  for (int q = 0; q < E / PER16; ++q) {
    u32x4 w = __builtin_nontemporal_load(p4 + q);
    const T* t = reinterpret_cast<const T*>(&w);
#pragma unroll
    for (int i = 0; i < PER16; ++i) v[q * PER16 + i] = ElemT<T>::cvt(t[i]);
  }
}

template <typename T, int E>
__device__ __forceinline__ void load_elems(const T* __restrict__ x, int64_t idx, int64_t n,
                                           float (&v)[E]) {
  if (idx + E <= n) {
    load_whole<T, E>(x + idx, v);
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
__device__ __forceinline__ uint32_t buf_load_b8_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, (int)voff, (int)soff, 2);
}
__device__ __forceinline__ uint32_t buf_load_b16_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, 2);
}
__device__ __forceinline__ uint2 buf_load_b64_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 2);
  return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ u32x4 buf_load_b128_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 2));
}

// Store `NB` bytes from `w` at byte voff of a buffer resource (aligned to NB)
template <int NB>
__device__ __forceinline__ void buf_store(__amdgpu_buffer_rsrc_t r, uint32_t voff, const uint32_t* w) {
  if constexpr (NB == 1) __builtin_amdgcn_raw_buffer_store_b8((uint8_t)w[0], r, (int)voff, 0, 0);
  else if constexpr (NB == 2) __builtin_amdgcn_raw_buffer_store_b16((uint16_t)w[0], r, (int)voff, 0, 0);
  else if constexpr (NB == 4) __builtin_amdgcn_raw_buffer_store_b32(w[0], r, (int)voff, 0, 0);
  else if constexpr (NB == 8) __builtin_amdgcn_raw_buffer_store_b64(u32x2{w[0], w[1]}, r, (int)voff, 0, 0);
  else if constexpr (NB == 16)
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{w[0], w[1], w[2], w[3]}, r, (int)voff, 0, 0);
  else if constexpr (NB == 32) {
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{w[0], w[1], w[2], w[3]}, r, (int)voff, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{w[4], w[5], w[6], w[7]}, r, (int)voff + 16, 0, 0);
  }
}

// E elements at byte voff of a buffer resource (16-byte aligned) as float,
// non-temporal
template <typename T, int E>
__device__ __forceinline__ void buf_load_elems(__amdgpu_buffer_rsrc_t r, uint32_t voff, float (&v)[E]) {
  constexpr int PER16 = 16 / sizeof(T);
  static_assert(E % PER16 == 0, "E must cover whole 16-byte vectors");
#pragma unroll
  for (int q = 0; q < E / PER16; ++q) {
    u32x4 w = buf_load_b128_nt(r, voff + 16 * q, 0);
    const T* t = reinterpret_cast<const T*>(&w);
#pragma unroll
    for (int i = 0; i < PER16; ++i) v[q * PER16 + i] = ElemT<T>::cvt(t[i]);
  }
}

// Store `NB` bytes from `w` at dst (aligned to NB), no range check
template <int NB>
__device__ __forceinline__ void store_whole(uint8_t* __restrict__ dst, const uint32_t* w) {
  if constexpr (NB == 1) *dst = static_cast<uint8_t>(w[0]);
  else if constexpr (NB == 2) *reinterpret_cast<uint16_t*>(dst) = static_cast<uint16_t>(w[0]);
  else if constexpr (NB == 4) *reinterpret_cast<uint32_t*>(dst) = w[0];
  else if constexpr (NB == 8) *reinterpret_cast<u32x2*>(dst) = u32x2{w[0], w[1]};
  else if constexpr (NB == 16) *reinterpret_cast<u32x4*>(dst) = u32x4{w[0], w[1], w[2], w[3]};
  else if constexpr (NB == 32) {
    *reinterpret_cast<u32x4*>(dst) = u32x4{w[0], w[1], w[2], w[3]};
    *reinterpret_cast<u32x4*>(dst + 16) = u32x4{w[4], w[5], w[6], w[7]};
  }
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
// small integers.  Index 127 gives -0.0, as in the table.  RN(m / 15) for
// the 16 numerators is fma(m, A, RN(m * B)) with A = RN(1/15) and B =
// RN(1/15 - A) (checked against the division for every m; 2 VALU where the
// Markstein quotient took 4), both scaled by 2^-15 here (exact).
__device__ __forceinline__ float fp8_grid_value(uint32_t f) {
  const uint32_t c = (f ^ ((f >> 7) - 1u)) & 0x7Fu;  // f ^ 0x7F below 128, f - 128 above
  const uint32_t e = c >> 3;
  const float m = (float)((c & 7u) | (min(e, 1u) << 3));
  const float q = __builtin_fmaf(m, 0x1.111112p-19f, m * -0x1.dddddep-44f);  // RN(m / 15) * 2^-15
  const float g = __builtin_ldexpf(q, (int)max(e, 1u));
  return f < 128u ? -g : g;
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

// bucket<BITS> of a finite y through an LDS table keyed by the sign and
// the top bits of the clamped magnitude.  Magnitude key k = (bits(c) >>
// SHIFT) - BASE of c = clamp(|y|, LO, HI): FP4 a quarter binade from 2^-5
// on (N 32, SHIFT 21, BASE 488; key 0 = [0, 1.25 * 2^-5), key 31 = [7,
// inf)), FP8 a sixteenth of a binade from 2^-19 on (N 305, SHIFT 19, BASE
// 1728; key 304 = [1, inf)).  Each key's interval holds at most one
// positive mid m_k (consecutive mids are more than one key apart) and key
// 0 none (it ends below the smallest mid); c_k counts the mids below the
// interval.  With torch.bucketize's count of mids < y:
//   y > 0:   H + c_k + (y > m_k)
//   y <= 0:  H - 1 - #{mids <= |y|} = (H - 2 - c_k) + (y > -m_k)
// so every (sign, key) entry is a base and a threshold, code = base +
// (y > thr): positive (H + c_k, m_k), negative (H - 2 - c_k, -m_k), a key
// without a mid (H + c_k, +inf) / (H - 1 - c_k, +inf), and positive key 0
// (H - 1, +0) so that +0 takes the code of -0.  The sign selects a half of
// the table: FP4 as bit 10 of the key itself (bits(c) with y's sign bit,
// shifted), the table indexed by that key unreduced (entries from BASE on,
// the negative half 1024 entries further, 12 KB of LDS) so that the address
// is two VALU; FP8 by selecting the half's base address (305 entries on).  ~7 VALU and one LDS
// read per element against ~11 for the unsigned key (count, nextup of |y|
// for y <= 0, then c ^ H or c ^ (H - 1)).  Equal to torch.bucketize over
// the mids for every finite float32 and +-inf (checked over every pattern
// near a mid or a key boundary and a stride through all of them).
template <int BITS> struct FpKeys;
// OFF: the index of positive key 0's entry; NEG: the negative half's
// distance from the positive one
template <> struct FpKeys<4> { static constexpr int N = 32, SHIFT = 21, BASE = 488, NEG = 1 << 10, OFF = 488; };
template <> struct FpKeys<8> { static constexpr int N = 305, SHIFT = 19, BASE = 1728, NEG = 305, OFF = 0; };

// The tables are made by the compiler (constant evaluation is IEEE float32
// arithmetic, rounded to nearest, the operations build_tables performs at
// run time) and live in device memory; a workgroup copies the 2 * N key
// entries into LDS (load_fp_keys) instead of building them: float8d
// quantize spent ~100 VALU per wave on the build (a division per grid value,
// a bisection per key) against ~2.7 steps of ~220.
namespace fpt {
constexpr float pow2(int e) {
  float r = 1.0f;
  for (int i = 0; i < e; ++i) r *= 2.0f;
  for (int i = 0; i < -e; ++i) r *= 0.5f;
  return r;
}
// fmt_value(bits, c) / fmt_max(bits)
constexpr float grid(int bits, int c) {
  if (bits == 4) {
    const int e = c >> 1, m = c & 1;
    return (e == 0 ? 0.5f * (float)m : (float)(2 + m) * pow2(e - 2)) / 6.0f;
  }
  const int e = c >> 3, m = c & 7;
  return (e == 0 ? (float)m * pow2(-9) : (float)(8 + m) * pow2(e - 10)) / 480.0f;
}
template <int BITS>
struct Tables {
  static constexpr int H = 1 << (BITS - 1), N = FpKeys<BITS>::N;
  float P[H + 1];     // build_tables' P: -inf, the positive mids, +inf
  float G[2 * H];     // build_tables' G: the sorted grid (G[H - 1] = -0.0)
  int key[2 * N][2];  // positive keys 0..N-1, then negative keys 0..N-1
};
template <int BITS>
constexpr Tables<BITS> make_tables() {
  using K = FpKeys<BITS>;
  constexpr int H = 1 << (BITS - 1);
  Tables<BITS> t{};
  t.P[0] = -__builtin_inff();
  t.P[H] = __builtin_inff();
  for (int j = 1; j < H; ++j) t.P[j] = (grid(BITS, j - 1) + grid(BITS, j)) * 0.5f;
  for (int c = 0; c < H; ++c) {
    t.G[H + c] = grid(BITS, c);
    t.G[H - 1 - c] = -grid(BITS, c);
  }
  for (int k = 0; k < K::N; ++k) {
    const float lo = k == 0 ? 0.0f : __builtin_bit_cast(float, (uint32_t)(k + K::BASE) << K::SHIFT);
    const float hi =
        k == K::N - 1 ? __builtin_inff() : __builtin_bit_cast(float, (uint32_t)(k + K::BASE + 1) << K::SHIFT);
    int cnt = 0;
    float mid = __builtin_inff();
    for (int j = 1; j < H; ++j) {
      if (t.P[j] < lo) ++cnt;
      else if (t.P[j] < hi && mid == __builtin_inff()) mid = t.P[j];
    }
    const bool has = mid < __builtin_inff();
    t.key[k][0] = k == 0 ? H - 1 : H + cnt;
    t.key[k][1] = __builtin_bit_cast(int, k == 0 ? 0.0f : mid);
    t.key[K::N + k][0] = has ? H - 2 - cnt : H - 1 - cnt;
    t.key[K::N + k][1] = __builtin_bit_cast(int, has ? -mid : mid);
  }
  return t;
}
}  // namespace fpt

template <int BITS> struct FpTables;
template <> struct FpTables<4> { static __device__ const fpt::Tables<4> t; };
template <> struct FpTables<8> { static __device__ const fpt::Tables<8> t; };
inline __device__ const fpt::Tables<4> FpTables<4>::t = fpt::make_tables<4>();
inline __device__ const fpt::Tables<8> FpTables<8>::t = fpt::make_tables<8>();

// build_tables<BITS>' P (FP4's is its constants), in device memory
template <int BITS>
__device__ __forceinline__ const float* fp_mids() { return FpTables<BITS>::t.P; }

// Copies the sorted grid (2H floats) into G and waits for the workgroup.
template <int BITS>
__device__ __forceinline__ void load_fp_grid(float* G) {
  constexpr int H = 1 << (BITS - 1);
  for (int t = threadIdx.x; t < 2 * H; t += blockDim.x) G[t] = FpTables<BITS>::t.G[t];
  __syncthreads();
}

// Copies the 2 * N key entries into T's layout (FP4 leaves the entries below
// OFF and between the halves unwritten) and waits for the workgroup.
template <int BITS>
__device__ __forceinline__ void load_fp_keys(int2* T) {
  using K = FpKeys<BITS>;
  const int2* src = reinterpret_cast<const int2*>(FpTables<BITS>::t.key);
  for (int t = threadIdx.x; t < 2 * K::N; t += blockDim.x)
    T[K::OFF + (t < K::N ? t : K::NEG + t - K::N)] = src[t];
  __syncthreads();
}

// The code of a finite y (or +-inf) in [0, 2H - 1]; T is load_fp_keys'
// table.
template <int BITS>
__device__ __forceinline__ int bucket_signed(float y, const int2* __restrict__ T) {
  using K = FpKeys<BITS>;
  const float c = __builtin_amdgcn_fmed3f(__builtin_fabsf(y), __uint_as_float((uint32_t)K::BASE << K::SHIFT),
                                          __uint_as_float((uint32_t)(K::BASE + K::N - 1) << K::SHIFT));
  int2 e;
  if constexpr (K::NEG == (1 << (31 - K::SHIFT))) {
    static_assert(K::OFF == K::BASE, "the key indexes the table unreduced");
    const uint32_t u = __float_as_uint(c) | (__float_as_uint(y) & 0x80000000u);
    e = T[u >> K::SHIFT];
  } else {
    const int2* Th = (int)__float_as_uint(y) < 0 ? T + K::OFF + K::NEG : T + K::OFF;
    e = Th[(__float_as_uint(c) >> K::SHIFT) - (uint32_t)K::BASE];
  }
  return e.x + (y > __int_as_float(e.y) ? 1 : 0);
}

// LDS entries of load_fp_keys' table
template <int BITS>
constexpr int fp_keys_size() { return FpKeys<BITS>::OFF + FpKeys<BITS>::NEG + FpKeys<BITS>::N; }

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

// encode<> with float codes through the key table of load_fp_keys (T
// unused for the other formats)
template <int MODE, int BITS>
__device__ __forceinline__ int encode_keyed(float v, const BlockParams& bp, float qf, const float* P, const int2* T) {
  if constexpr (MODE == Q_FP) return bucket_signed<BITS>(div_rn(v, bp.s, bp.mul), T);
  else return encode<MODE, BITS>(v, bp, qf, P);
}

// LDS entries of a kernel's key table (1 when it encodes no float codes)
template <int MODE, int BITS>
constexpr int fp_keys_n() {
  if constexpr (MODE == Q_FP) return fp_keys_size<BITS>();
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
                         const float* w_scales_t, int64_t N, int kind, const float* bias, float* out,
                         void* workspace, size_t workspace_nbytes, hipStream_t st);
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

// ---------------------------------------------------------------- float codes as f16 B operands
// Two float codes (indices into the sorted grid of 2^B values: B = 4 FP4
// E2M1, B = 8 FP8 E4M3 with exponent 15 a normal binade) as the f16 pair of
// their grid values times vmax · 2^-P (vmax 6 or 480, P = 14 or 8): the
// format's own values v, scaled by a power of two, exact in f16 (subnormal
// for the smallest: the MFMA takes f16 subnormals).  FP4 codes sit at bits
// 0-3 and 16-19 of d (the bits above each code ignored), FP8 codes at bits
// 8-15 and 24-31 (the callers' byte permutes put them there; the bits below
// ignored).  c ^ 2^(B-1) is the B-bit one's complement of +-m, m the bit
// pattern of |v| (the grid is symmetric and sorted); at the top of a 16-bit
// half, xor-ed with its sign mask and shifted to f16's mantissa position, m
// is the f16 of |v| * 2^-P.
template <int B>
__device__ __forceinline__ uint32_t fp_code_pair_f16(uint32_t d) {
  typedef short s2v __attribute__((ext_vector_type(2)));
  // code at the top of each half, its top bit flipped
  const uint32_t x = (B == 4 ? d << 12 : d) ^ 0x80008000u;
  const uint32_t sm = __builtin_bit_cast(uint32_t, __builtin_bit_cast(s2v, x) >> (short)15);
  const uint32_t y = x ^ sm;
  const uint32_t m = (y >> (B == 4 ? 3 : 1)) & (B == 4 ? 0x0E000E00u : 0x3F803F80u);
  return (sm & 0x80008000u) | m;
}

}  // namespace mxk
