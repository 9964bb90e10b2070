// Dynamic (runtime) activation quantization, dynamic_quantize
// (mxtorch.py:2665-2731), for gfx950.
//
// Every granularity uses the same per-element rule with max_int =
// 2^(bits-1)-1 of the dtype's width (for float dtypes too, mxtorch.py:2705):
//   s = RN(max(absmax, 1e-12) / max_int),  code = rne(clamp(RN(x / s), +-max_int))
// and packs the codes with pack_auto (mxtorch.py:976-985).  They differ in
// what one scale covers:
//   per_token    one scale per row of the last dimension: the 'v' rule with
//                block = row length, run by mxk_quantize (mxtorch.py:2708-2714);
//   per_channel  one scale per column of x.reshape(shape[0], -1)
//                (mxtorch.py:2716-2722);
//   per_tensor   one scale for the whole tensor (mxtorch.py:2724-2729).
// The absmax of a column or of the tensor is reduced with atomicMax on the
// bit patterns of non-negative floats, which order like the floats: the
// result is exact and independent of the order of arrival.
#include "mxk_internal.h"

#include <algorithm>
#include <type_traits>

namespace mxk {

__global__ __launch_bounds__(256) void k_fill_u32(uint32_t* __restrict__ p, int64_t n, uint32_t v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

// amax[c] = max over rows of |x[r][c]|; blockIdx.y takes `rows_per` rows.
template <typename T>
__global__ __launch_bounds__(256) void k_absmax_cols(const T* __restrict__ x, int64_t R, int64_t C, int64_t rows_per,
                                                     uint32_t* __restrict__ amax) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  const int64_t r0 = (int64_t)blockIdx.y * rows_per;
  const int64_t r1 = std::min<int64_t>(R, r0 + rows_per);
  float m = 0.0f;
  for (int64_t r = r0; r < r1; ++r) m = fmaxf(m, __builtin_fabsf(ElemT<T>::cvt(x[r * C + c])));
  atomicMax(amax + c, __float_as_uint(m));
}

// amax[0] = max over all n of |x|: grid-stride, wave maximum, one atomic per wave.
template <typename T>
__global__ __launch_bounds__(256) void k_absmax_all(const T* __restrict__ x, int64_t n, uint32_t* __restrict__ amax) {
  float m = 0.0f;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    m = fmaxf(m, __builtin_fabsf(ElemT<T>::cvt(x[i])));
  m = group_max<64>(m);
  if ((threadIdx.x & 63) == 0) atomicMax(amax, __float_as_uint(m));
}

// scales[i] = RN(max(amax[i], fl32(1e-12)) / max_int)
__global__ __launch_bounds__(256) void k_dyn_scales(const uint32_t* __restrict__ amax, int64_t cnt, float q,
                                                    float* __restrict__ scales) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < cnt; i += (int64_t)gridDim.x * blockDim.x)
    scales[i] = fmaxf(__uint_as_float(amax[i]), MXK_AMIN) / q;
}

// One packed byte per thread: the 8/BITS codes of elements u*per .. u*per+per-1,
// each divided by its scale (scales[j % C], or scales[0] when C == 0).
template <typename T, int BITS>
__global__ __launch_bounds__(256) void k_dyn_encode(const T* __restrict__ x, int64_t n, int64_t C,
                                                    const float* __restrict__ scales, float q,
                                                    uint8_t* __restrict__ packed, int64_t nbytes) {
  constexpr int PER = 8 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < nbytes; u += (int64_t)gridDim.x * blockDim.x) {
    uint32_t w = 0u;
#pragma unroll
    for (int f = 0; f < PER; ++f) {
      const int64_t j = u * PER + f;
      if (j >= n) break;
      const float s = scales[C ? j % C : 0];
      const float y = ElemT<T>::cvt(x[j]) / s;
      const int code = (int)rne(fminf(fmaxf(y, -q), q));
      w |= ((uint32_t)code & MASK) << (f * BITS);
    }
    packed[u] = (uint8_t)w;
  }
}

// workspace of the vector path: scales' reciprocals (cnt words, padded to
// 64), then the absmax parts: DYN_PARTS maxima per tensor, or DYN_COL_PARTS
// rows of cols maxima per channel
#define DYN_PARTS 1024
#define DYN_COL_PARTS 128
static int64_t dyn_pad(int64_t c) { return (c + 63) & ~(int64_t)63; }

// ---- vector paths (x 16-byte aligned; see dyn_run for the shapes).  A
// wave's load q covers 64 * EPL consecutive elements (lane l: EPL at
// EPL * l), so every load instruction reads whole lines.
template <typename T>
__device__ __forceinline__ void load16(const T* __restrict__ p, float (&v)[16 / sizeof(T)]) {
  constexpr int EPL = 16 / (int)sizeof(T);
  const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  const T* t = reinterpret_cast<const T*>(&w);
#pragma unroll
  for (int e = 0; e < EPL; ++e) v[e] = ElemT<T>::cvt(t[e]);
}

// part[blockIdx.x] = max |x| over the workgroup's share of x (n % 16 == 0):
// four wave loads in flight, wave maximum, then across the 4 waves in LDS.
template <typename T>
__global__ __launch_bounds__(256) void k_absmax_all_v(const T* __restrict__ x, int64_t n, float* __restrict__ part) {
  constexpr int EPL = 16 / (int)sizeof(T), U = 4, WCH = 64 * EPL;
  __shared__ float sm[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t stride = (int64_t)gridDim.x * 4 * WCH * U;
  float m = 0.0f;
  for (int64_t b0 = ((int64_t)blockIdx.x * 4 + wave) * WCH * U; b0 < n; b0 += stride) {
    float v[U][EPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = b0 + (int64_t)u * WCH + EPL * lane;
      if (i < n) {
        load16<T>(x + i, v[u]);
      } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) v[u][e] = 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int e = 0; e < EPL; ++e) m = fmaxf(m, __builtin_fabsf(v[u][e]));
  }
  m = group_max<64>(m);
  if (lane == 0) sm[wave] = m;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
}

// part[blockIdx.y][c] = max over the workgroup's rows of |x[r][c]| (C a
// multiple of 16 / sizeof(T)): thread t takes the EPL columns at
// EPL * (blockIdx.x * 256 + t), one 16-byte load per row, eight rows in flight.
template <typename T>
__global__ __launch_bounds__(256) void k_absmax_cols_v(const T* __restrict__ x, int64_t R, int64_t C,
                                                       int64_t rows_per, float* __restrict__ part) {
  constexpr int EPL = 16 / (int)sizeof(T), U = 8;
  const int64_t c0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * EPL;
  if (c0 >= C) return;
  const int64_t r0 = (int64_t)blockIdx.y * rows_per;
  const int64_t r1 = std::min<int64_t>(R, r0 + rows_per);
  float m[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) m[e] = 0.0f;
  for (int64_t r = r0; r < r1; r += U) {
    float v[U][EPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (r + u < r1) {
        load16<T>(x + (r + u) * C + c0, v[u]);
      } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) v[u][e] = 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int e = 0; e < EPL; ++e) m[e] = fmaxf(m[e], __builtin_fabsf(v[u][e]));
  }
  float* dst = part + (int64_t)blockIdx.y * C + c0;
#pragma unroll
  for (int e = 0; e < EPL; e += 4) *reinterpret_cast<f32x4v*>(dst + e) = f32x4v{m[e], m[e + 1], m[e + 2], m[e + 3]};
}

// scales[i] = RN(max(amax_i, fl32(1e-12)) / max_int), rcp[i] = RN(1 / scales[i]),
// amax_i the maximum of part[k * cnt + i] over k < parts.
__global__ __launch_bounds__(256) void k_dyn_scales_parts(const float* __restrict__ part, int64_t parts, int64_t cnt,
                                                          float q, float* __restrict__ scales,
                                                          float* __restrict__ rcp) {
  if (cnt == 1) {  // one workgroup: the maximum over all parts
    __shared__ float sm[4];
    float m = 0.0f;
    for (int64_t k = threadIdx.x; k < parts; k += 256) m = fmaxf(m, part[k]);
    m = group_max<64>(m);
    if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0 && blockIdx.x == 0) {
      const float sc = fmaxf(fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3])), MXK_AMIN) / q;
      scales[0] = sc;
      if (rcp) rcp[0] = 1.0f / sc;
    }
    return;
  }
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < cnt; i += (int64_t)gridDim.x * blockDim.x) {
    float m = 0.0f;
    for (int64_t k0 = 0; k0 < parts; k0 += 8) {
      float t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) t[u] = k0 + u < parts ? part[(k0 + u) * cnt + i] : 0.0f;
#pragma unroll
      for (int u = 0; u < 8; ++u) m = fmaxf(m, t[u]);
    }
    const float sc = fmaxf(m, MXK_AMIN) / q;
    scales[i] = sc;
    if (rcp) rcp[i] = 1.0f / sc;
  }
}

// int32 codes of vector_quantize per column (C % 1024 == 0): the load layout
// of k_dyn_encode_v, RN(x / s) by the hardware divide, clamp, round to
// nearest even; each load's EPL codes in one or two 16-byte stores.
template <typename T, bool FIXED>
__global__ __launch_bounds__(256) void k_vec_encode_cols_v(const T* __restrict__ x, int64_t n, int64_t C,
                                                           const float* __restrict__ scales, float q,
                                                           int32_t* __restrict__ codes) {
  constexpr int EPL = 16 / (int)sizeof(T), QL = 16 / EPL, WCH = 64 * EPL, STEP = 1024;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t stride = (int64_t)gridDim.x * 4 * STEP;
  float sf[QL][EPL];
  if constexpr (FIXED) {
    const int64_t cb = (((int64_t)blockIdx.x * 4 + wave) * STEP) % C;
#pragma unroll
    for (int ql = 0; ql < QL; ++ql)
#pragma unroll
      for (int e = 0; e < EPL; e += 4) {
        const f32x4v a = *reinterpret_cast<const f32x4v*>(scales + cb + (int64_t)ql * WCH + EPL * lane + e);
#pragma unroll
        for (int k = 0; k < 4; ++k) sf[ql][e + k] = a[k];
      }
  }
  for (int64_t b0 = ((int64_t)blockIdx.x * 4 + wave) * STEP; b0 < n; b0 += stride) {
    float v[QL][EPL];
#pragma unroll
    for (int ql = 0; ql < QL; ++ql) {
      const int64_t i = b0 + (int64_t)ql * WCH + EPL * lane;
      if (i < n) {
        load16<T>(x + i, v[ql]);
      } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) v[ql][e] = 0.0f;
      }
    }
    float sv[QL][EPL];
    if constexpr (FIXED) {
#pragma unroll
      for (int ql = 0; ql < QL; ++ql)
#pragma unroll
        for (int e = 0; e < EPL; ++e) sv[ql][e] = sf[ql][e];
    } else {
      const int64_t cb = b0 % C;  // wave-uniform
#pragma unroll
      for (int ql = 0; ql < QL; ++ql)
#pragma unroll
        for (int e = 0; e < EPL; e += 4) {
          const f32x4v a = *reinterpret_cast<const f32x4v*>(scales + cb + (int64_t)ql * WCH + EPL * lane + e);
#pragma unroll
          for (int k = 0; k < 4; ++k) sv[ql][e + k] = a[k];
        }
    }
#pragma unroll
    for (int ql = 0; ql < QL; ++ql) {
      const int64_t i = b0 + (int64_t)ql * WCH + EPL * lane;
      uint32_t c[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float t = __builtin_amdgcn_fmed3f(v[ql][e] / sv[ql][e], -q, q);
        c[e] = __float_as_uint(t + 12582912.0f) - 0x4B400000u;  // rne(t) as an int32 (|t| <= q < 2^22)
      }
      if (i < n) {
#pragma unroll
        for (int e = 0; e < EPL; e += 4)
          *reinterpret_cast<u32x4*>(codes + i + e) = u32x4{c[e], c[e + 1], c[e + 2], c[e + 3]};
      }
    }
  }
}

// Encode, a wave taking 1024 consecutive elements per step (n % 16 == 0;
// per channel C % 1024 == 0, so a step stays in one row): load q of lane l
// is the EPL elements at 64 * EPL * q + EPL * l.  RN(x / s) by Markstein's
// correction with y = RN(1 / s), or the hardware divide for a lane holding
// a nonzero |x| below 2^-96; clamp, round to nearest even, and each load's
// EPL codes stored together (one store instruction of the wave covers
// 64 * EPL * BITS / 8 contiguous bytes).
template <typename T, int BITS, bool PER_CHANNEL, bool FIXED>
__global__ __launch_bounds__(256) void k_dyn_encode_v(const T* __restrict__ x, int64_t n, int64_t C,
                                                      const float* __restrict__ scales, const float* __restrict__ rcp,
                                                      float q, uint8_t* __restrict__ packed) {
  constexpr int EPL = 16 / (int)sizeof(T), QL = 16 / EPL, WCH = 64 * EPL, STEP = 1024;
  constexpr int GB = EPL * BITS / 8;  // packed bytes of one load's codes
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t stride = (int64_t)gridDim.x * 4 * STEP;
  const float s_all = PER_CHANNEL ? 0.0f : scales[0], y_all = PER_CHANNEL ? 0.0f : rcp[0];
  // FIXED (the grid's stride a multiple of C): a wave's columns are the same
  // at every step, so its scales are loaded once
  float sf[QL][EPL], yf[QL][EPL];
  if constexpr (PER_CHANNEL && FIXED) {
    const int64_t cb = (((int64_t)blockIdx.x * 4 + wave) * STEP) % C;
#pragma unroll
    for (int ql = 0; ql < QL; ++ql)
#pragma unroll
      for (int e = 0; e < EPL; e += 4) {
        const int64_t c = cb + (int64_t)ql * WCH + EPL * lane + e;
        const f32x4v a = *reinterpret_cast<const f32x4v*>(scales + c);
        const f32x4v b = *reinterpret_cast<const f32x4v*>(rcp + c);
#pragma unroll
        for (int k = 0; k < 4; ++k) { sf[ql][e + k] = a[k]; yf[ql][e + k] = b[k]; }
      }
  }
  for (int64_t b0 = ((int64_t)blockIdx.x * 4 + wave) * STEP; b0 < n; b0 += stride) {
    float v[QL][EPL];
#pragma unroll
    for (int ql = 0; ql < QL; ++ql) {
      const int64_t i = b0 + (int64_t)ql * WCH + EPL * lane;
      if (i < n) {
        load16<T>(x + i, v[ql]);
      } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) v[ql][e] = 0.0f;
      }
    }
    float sv[QL][EPL], yv[QL][EPL];
    if constexpr (PER_CHANNEL && FIXED) {
#pragma unroll
      for (int ql = 0; ql < QL; ++ql)
#pragma unroll
        for (int e = 0; e < EPL; ++e) { sv[ql][e] = sf[ql][e]; yv[ql][e] = yf[ql][e]; }
    } else if constexpr (PER_CHANNEL) {
      const int64_t cb = b0 % C;  // wave-uniform
#pragma unroll
      for (int ql = 0; ql < QL; ++ql)
#pragma unroll
        for (int e = 0; e < EPL; e += 4) {
          const int64_t c = cb + (int64_t)ql * WCH + EPL * lane + e;
          const f32x4v a = *reinterpret_cast<const f32x4v*>(scales + c);
          const f32x4v b = *reinterpret_cast<const f32x4v*>(rcp + c);
#pragma unroll
          for (int k = 0; k < 4; ++k) { sv[ql][e + k] = a[k]; yv[ql][e + k] = b[k]; }
        }
    } else {
#pragma unroll
      for (int ql = 0; ql < QL; ++ql)
#pragma unroll
        for (int e = 0; e < EPL; ++e) { sv[ql][e] = s_all; yv[ql][e] = y_all; }
    }
    uint32_t mnb = 0xFFFFFFFFu;  // (bits << 1) - 1: both zeros map to the maximum
#pragma unroll
    for (int ql = 0; ql < QL; ++ql)
#pragma unroll
      for (int e = 0; e < EPL; ++e) mnb = min(mnb, (__float_as_uint(v[ql][e]) << 1) - 1u);
    if (__builtin_expect(mnb < 2u * 0x0F800000u - 1u, 0)) {
#pragma unroll
      for (int ql = 0; ql < QL; ++ql)
#pragma unroll
        for (int e = 0; e < EPL; ++e) v[ql][e] = v[ql][e] / sv[ql][e];
    } else {
#pragma unroll
      for (int ql = 0; ql < QL; ++ql)
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          const float q0 = v[ql][e] * yv[ql][e];
          v[ql][e] = __builtin_fmaf(__builtin_fmaf(-q0, sv[ql][e], v[ql][e]), yv[ql][e], q0);
        }
    }
#pragma unroll
    for (int ql = 0; ql < QL; ++ql) {
      const int64_t i = b0 + (int64_t)ql * WCH + EPL * lane;
      uint32_t w[(GB + 3) / 4];
#pragma unroll
      for (int k = 0; k < (GB + 3) / 4; ++k) w[k] = 0u;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        // rne of the clamped quotient by the float adder (|t| <= q < 2^22)
        const float t = __builtin_amdgcn_fmed3f(v[ql][e], -q, q);
        const uint32_t code = __float_as_uint(t + 12582912.0f) & MASK;
        w[(e * BITS) >> 5] |= code << ((e * BITS) & 31);
      }
      if (i < n) {
        uint8_t* dst = packed + i * BITS / 8;
        if constexpr (GB == 8) *reinterpret_cast<u32x2*>(dst) = u32x2{w[0], w[1]};
        else if constexpr (GB == 4) *reinterpret_cast<uint32_t*>(dst) = w[0];
        else if constexpr (GB == 2) *reinterpret_cast<uint16_t*>(dst) = (uint16_t)w[0];
        else *dst = (uint8_t)w[0];
      }
    }
  }
}

// amax[r] = max over row r of |x[r][:]|, as float bits: one workgroup per
// row (grid-stride over the rows), a wave maximum, then across the 4 waves.
template <typename T>
__global__ __launch_bounds__(256) void k_absmax_rows(const T* __restrict__ x, int64_t R, int64_t C,
                                                     uint32_t* __restrict__ amax) {
  __shared__ float sm[4];
  for (int64_t r = blockIdx.x; r < R; r += gridDim.x) {
    float m = 0.0f;
    for (int64_t c = threadIdx.x; c < C; c += 256) m = fmaxf(m, __builtin_fabsf(ElemT<T>::cvt(x[r * C + c])));
    m = group_max<64>(m);
    if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) amax[r] = __float_as_uint(fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3])));
    __syncthreads();
  }
}

// int32 codes of vector_quantize: rne(clamp(RN(x / s), +-max_int)) with s the
// element's row scale (PER_ROW) or column scale.
template <typename T, bool PER_ROW>
__global__ __launch_bounds__(256) void k_vec_encode(const T* __restrict__ x, int64_t n, int64_t C,
                                                    const float* __restrict__ scales, float q,
                                                    int32_t* __restrict__ codes) {
  for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += (int64_t)gridDim.x * blockDim.x) {
    const float s = scales[PER_ROW ? j / C : j % C];
    codes[j] = (int32_t)rne(fminf(fmaxf(ElemT<T>::cvt(x[j]) / s, -q), q));
  }
}

// vector_dequantize: out = RN(code * s), s per row or per column.
template <bool PER_ROW>
__global__ __launch_bounds__(256) void k_vec_decode(const int32_t* __restrict__ codes, int64_t n, int64_t C,
                                                    const float* __restrict__ scales, float* __restrict__ out) {
  for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += (int64_t)gridDim.x * blockDim.x)
    out[j] = (float)codes[j] * scales[PER_ROW ? j / C : j % C];
}

// vector_dequantize with cols % 4 == 0 and 16-byte aligned buffers: a wave
// takes 1024 consecutive codes per step (load q of lane l: the 4 codes at
// 256 q + 4 l, so each load and store instruction covers whole lines); the
// 4 codes of a load share a row and lie in consecutive columns.
template <bool PER_ROW>
__global__ __launch_bounds__(256) void k_vec_decode_v(const int32_t* __restrict__ codes, int64_t n, int64_t C,
                                                      const float* __restrict__ scales, float* __restrict__ out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t stride = (int64_t)gridDim.x * 4 * 1024;
  for (int64_t b0 = ((int64_t)blockIdx.x * 4 + wave) * 1024; b0 < n; b0 += stride) {
    u32x4 cv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t i = b0 + 256 * q + 4 * lane;
      cv[q] = i < n ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(codes + i)) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t i = b0 + 256 * q + 4 * lane;
      if (i >= n) continue;
      const int64_t r = i / C, c = i - r * C;
      f32x4v sv;
      if constexpr (PER_ROW) {
        const float sc = scales[r];
        sv = f32x4v{sc, sc, sc, sc};
      } else {
        sv = *reinterpret_cast<const f32x4v*>(scales + c);
      }
      const f32x4v o = {(float)(int32_t)cv[q][0] * sv[0], (float)(int32_t)cv[q][1] * sv[1],
                        (float)(int32_t)cv[q][2] * sv[2], (float)(int32_t)cv[q][3] * sv[3]};
      __builtin_nontemporal_store(o, reinterpret_cast<f32x4v*>(out + i));
    }
  }
}

template <typename T>
static int vec_run(const T* x, int64_t rows, int64_t cols, int axis, int bits, int32_t* codes, float* scales,
                   hipStream_t st) {
  const int64_t n = rows * cols;
  const float q = (float)((1u << (bits - 1)) - 1u);
  const int cap = num_cus() * 8;
  constexpr int x_type = sizeof(T) == 4 ? MXK_IN_F32 : (std::is_same<T, __half>::value ? MXK_IN_F16 : MXK_IN_BF16);
  // per row: the long-block row quantizer, one pass over x
  if (axis == 1 && vec_rows_i32(x, x_type, rows, cols, bits, codes, scales, st)) return check_launch("vector_quantize");
  // per column, whole 1024-column steps: column maxima in parts (held in
  // the codes buffer, which the encode overwrites afterwards), then a
  // vector encode
  if (axis == 0 && aligned16(x) && cols % 1024 == 0 && (reinterpret_cast<uintptr_t>(codes) & 15u) == 0) {
    constexpr int EPL = 16 / (int)sizeof(T);
    const int64_t cus = num_cus();
    float* part = reinterpret_cast<float*>(codes);
    const int64_t col_blocks = ceil_div(cols / EPL, 256);
    const int64_t chunks = std::max<int64_t>(
        1, std::min<int64_t>({(int64_t)DYN_COL_PARTS, ceil_div(rows, 8), ceil_div(cus * 8, col_blocks)}));
    const int64_t rows_per = ceil_div(rows, chunks);
    const int64_t parts = ceil_div(rows, rows_per);
    hipLaunchKernelGGL((k_absmax_cols_v<T>), dim3((unsigned)col_blocks, (unsigned)parts), dim3(256), 0, st, x, rows,
                       cols, rows_per, part);
    hipLaunchKernelGGL(k_dyn_scales_parts, dim3((unsigned)std::min<int64_t>(ceil_div(cols, 256), cus * 8)), dim3(256),
                       0, st, part, parts, cols, q, scales, nullptr);
    int64_t g = std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, 4 * 1024), cus * 16));
    const int64_t c1 = cols / 1024, m = c1 / std::__gcd<int64_t>(c1, 4);
    if (m <= cus * 64) {
      g = std::max<int64_t>(m, (g / m) * m);
      hipLaunchKernelGGL((k_vec_encode_cols_v<T, true>), dim3((unsigned)g), dim3(256), 0, st, x, n, cols, scales, q,
                         codes);
    } else {
      hipLaunchKernelGGL((k_vec_encode_cols_v<T, false>), dim3((unsigned)g), dim3(256), 0, st, x, n, cols, scales, q,
                         codes);
    }
    return check_launch("vector_quantize");
  }
  // the absmax bits accumulate in the scales buffer, which k_dyn_scales then
  // turns into the scales in place
  uint32_t* amax = reinterpret_cast<uint32_t*>(scales);
  const int64_t cnt = axis == 1 ? rows : cols;
  if (axis == 1) {
    hipLaunchKernelGGL((k_absmax_rows<T>), dim3((unsigned)std::min<int64_t>(rows, (int64_t)cap * 2)), dim3(256), 0, st,
                       x, rows, cols, amax);
  } else {
    hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)std::min<int64_t>(ceil_div(cnt, 256), cap)), dim3(256), 0, st, amax,
                       cnt, 0u);
    const int64_t col_blocks = ceil_div(cols, 256);
    const int64_t chunks = std::max<int64_t>(1, std::min<int64_t>(rows, ceil_div((int64_t)num_cus() * 4, col_blocks)));
    const int64_t rows_per = ceil_div(rows, chunks);
    hipLaunchKernelGGL((k_absmax_cols<T>), dim3((unsigned)col_blocks, (unsigned)ceil_div(rows, rows_per)), dim3(256),
                       0, st, x, rows, cols, rows_per, amax);
  }
  hipLaunchKernelGGL(k_dyn_scales, dim3((unsigned)std::min<int64_t>(ceil_div(cnt, 256), cap)), dim3(256), 0, st, amax,
                     cnt, q, scales);
  const dim3 g((unsigned)std::min<int64_t>(ceil_div(n, 256), (int64_t)cap * 4));
  if (axis == 1)
    hipLaunchKernelGGL((k_vec_encode<T, true>), g, dim3(256), 0, st, x, n, cols, scales, q, codes);
  else
    hipLaunchKernelGGL((k_vec_encode<T, false>), g, dim3(256), 0, st, x, n, cols, scales, q, codes);
  return check_launch("vector_quantize");
}

// The vector kernels take 16-byte aligned x, n % 16 == 0 and, per channel,
// cols % 1024 == 0; other shapes run the element-wise kernels.
template <typename T>
static bool dyn_vector_ok(const T* x, int64_t rows, int64_t cols, int granularity, const uint8_t* packed, int bits) {
  const int64_t n = rows * cols;
  if (!aligned16(x) || n % 16 != 0) return false;
  constexpr int EPL = 16 / (int)sizeof(T);
  if ((reinterpret_cast<uintptr_t>(packed) % (uintptr_t)std::max(1, EPL * bits / 8)) != 0) return false;
  return granularity != MXK_DYN_PER_CHANNEL || cols % 1024 == 0;
}


template <typename T>
static int dyn_run_vector(const T* x, int64_t rows, int64_t cols, int granularity, int bits, uint8_t* packed,
                          float* scales, float* ws, hipStream_t st) {
  constexpr int EPL = 16 / (int)sizeof(T);
  const int64_t n = rows * cols;
  const float q = (float)((1u << (bits - 1)) - 1u);
  const int64_t cus = num_cus();
  const bool pc = granularity == MXK_DYN_PER_CHANNEL;
  const int64_t cnt = pc ? cols : 1;
  float* rcp = ws;
  float* part = ws + dyn_pad(cnt);
  int64_t parts;
  if (pc) {
    const int64_t col_blocks = ceil_div(cols / EPL, 256);
    const int64_t chunks = std::max<int64_t>(
        1, std::min<int64_t>({(int64_t)DYN_COL_PARTS, ceil_div(rows, 8), ceil_div(cus * 8, col_blocks)}));
    const int64_t rows_per = ceil_div(rows, chunks);
    parts = ceil_div(rows, rows_per);
    hipLaunchKernelGGL((k_absmax_cols_v<T>), dim3((unsigned)col_blocks, (unsigned)parts), dim3(256), 0, st, x, rows,
                       cols, rows_per, part);
  } else {
    parts = std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, 4 * 64 * EPL * 4), (int64_t)DYN_PARTS));
    hipLaunchKernelGGL((k_absmax_all_v<T>), dim3((unsigned)parts), dim3(256), 0, st, x, n, part);
  }
  hipLaunchKernelGGL(k_dyn_scales_parts, dim3(pc ? (unsigned)std::min<int64_t>(ceil_div(cnt, 256), cus * 8) : 1u),
                     dim3(256), 0, st, part, parts, cnt, q, scales, rcp);
  int64_t g = std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, 4 * 1024), cus * 16));
  // per channel, a grid whose stride (4096 elements per workgroup) is a
  // multiple of cols keeps every wave on the same columns
  bool fixed = false;
  if (pc) {
    const int64_t c1 = cols / 1024, m = c1 / std::__gcd<int64_t>(c1, 4);
    if (m <= cus * 64) {
      g = std::max<int64_t>(m, (g / m) * m);
      fixed = true;
    }
  }
#define MXK_DYNV(BITS)                                                                                             \
  if (pc && fixed)                                                                                                 \
    hipLaunchKernelGGL((k_dyn_encode_v<T, BITS, true, true>), dim3((unsigned)g), dim3(256), 0, st, x, n, cols,     \
                       scales, rcp, q, packed);                                                                    \
  else if (pc)                                                                                                     \
    hipLaunchKernelGGL((k_dyn_encode_v<T, BITS, true, false>), dim3((unsigned)g), dim3(256), 0, st, x, n, cols,    \
                       scales, rcp, q, packed);                                                                    \
  else                                                                                                             \
    hipLaunchKernelGGL((k_dyn_encode_v<T, BITS, false, false>), dim3((unsigned)g), dim3(256), 0, st, x, n, cols,   \
                       scales, rcp, q, packed)
  switch (bits) {
    case 2: MXK_DYNV(2); break;
    case 4: MXK_DYNV(4); break;
    default: MXK_DYNV(8); break;
  }
#undef MXK_DYNV
  return check_launch("dynamic_quantize");
}

template <typename T>
static int dyn_run(const T* x, int64_t rows, int64_t cols, int granularity, int bits, uint8_t* packed,
                   int64_t pbytes, float* scales, uint32_t* amax, hipStream_t st) {
  if (dyn_vector_ok(x, rows, cols, granularity, packed, bits))
    return dyn_run_vector(x, rows, cols, granularity, bits, packed, scales, reinterpret_cast<float*>(amax), st);
  const int64_t n = rows * cols;
  const float q = (float)((1u << (bits - 1)) - 1u);
  const int cap = num_cus() * 8;
  const int64_t cnt = granularity == MXK_DYN_PER_CHANNEL ? cols : 1;
  hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)std::min<int64_t>(ceil_div(cnt, 256), cap)), dim3(256), 0, st, amax,
                     cnt, 0u);
  if (granularity == MXK_DYN_PER_CHANNEL) {
    // enough row chunks that the grid fills the chip; each chunk reads whole rows
    const int64_t col_blocks = ceil_div(cols, 256);
    const int64_t chunks = std::max<int64_t>(1, std::min<int64_t>(rows, ceil_div((int64_t)num_cus() * 4, col_blocks)));
    const int64_t rows_per = ceil_div(rows, chunks);
    hipLaunchKernelGGL((k_absmax_cols<T>), dim3((unsigned)col_blocks, (unsigned)ceil_div(rows, rows_per)), dim3(256),
                       0, st, x, rows, cols, rows_per, amax);
  } else {
    hipLaunchKernelGGL((k_absmax_all<T>), dim3((unsigned)std::min<int64_t>(ceil_div(n, 256), cap)), dim3(256), 0, st,
                       x, n, amax);
  }
  hipLaunchKernelGGL(k_dyn_scales, dim3((unsigned)std::min<int64_t>(ceil_div(cnt, 256), cap)), dim3(256), 0, st, amax,
                     cnt, q, scales);
  const int64_t C = granularity == MXK_DYN_PER_CHANNEL ? cols : 0;
  const dim3 g((unsigned)std::min<int64_t>(ceil_div(pbytes, 256), cap));
  switch (bits) {
    case 2: hipLaunchKernelGGL((k_dyn_encode<T, 2>), g, dim3(256), 0, st, x, n, C, scales, q, packed, pbytes); break;
    case 4: hipLaunchKernelGGL((k_dyn_encode<T, 4>), g, dim3(256), 0, st, x, n, C, scales, q, packed, pbytes); break;
    default: hipLaunchKernelGGL((k_dyn_encode<T, 8>), g, dim3(256), 0, st, x, n, C, scales, q, packed, pbytes); break;
  }
  return check_launch("dynamic_quantize");
}

}  // namespace mxk

using namespace mxk;

extern "C" {

size_t mxk_dynamic_quantize_workspace(int64_t rows, int64_t cols, int granularity, int bits) {
  if (rows <= 0 || cols <= 0) return 0;
  if (granularity == MXK_DYN_PER_TOKEN)
    return mxk_quantize_workspace(rows * cols, MXK_KIND_INT, bits, MXK_VAR_VECTOR, (int)cols, 0);
  // the element-wise path: absmax bits (cnt words); the vector path:
  // reciprocal scales (cnt words, padded to 64), then the absmax parts
  const bool pc = granularity == MXK_DYN_PER_CHANNEL;
  const int64_t cnt = pc ? cols : 1;
  const int64_t words = std::max<int64_t>(cnt, dyn_pad(cnt) + (pc ? (int64_t)DYN_COL_PARTS * cols : DYN_PARTS));
  return (size_t)((words * 4 + 255) & ~(int64_t)255);
}

int mxk_dynamic_quantize(const void* x, int x_type, int64_t rows, int64_t cols, int granularity, int bits,
                         void* packed, int64_t packed_nbytes, float* scales, void* workspace,
                         size_t workspace_nbytes, void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (rows <= 0 || cols <= 0) return fail(MXK_EINVAL, "dynamic_quantize: rows and cols must be positive");
  if (!x || !packed || !scales) return fail(MXK_EINVAL, "dynamic_quantize: null buffer");
  if (x_type != MXK_IN_F32 && x_type != MXK_IN_F16 && x_type != MXK_IN_BF16)
    return fail(MXK_EINVAL, "dynamic_quantize: x_type must be f32, f16 or bf16");
  if (granularity < MXK_DYN_PER_TOKEN || granularity > MXK_DYN_PER_TENSOR)
    return fail(MXK_EINVAL, "dynamic_quantize: unknown granularity");
  const int64_t n = rows * cols;
  if (granularity == MXK_DYN_PER_TOKEN) {
    // the 'v' rule with one block per row and max_int of the width
    if (!(bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 7 || bits == 8 || bits == 16))
      return fail(MXK_EUNSUPPORTED, "dynamic_quantize(per_token): widths 2..8 and 16 are implemented");
    if (cols > INT32_MAX) return fail(MXK_EINVAL, "dynamic_quantize(per_token): row too long");
    return mxk_quantize(x, x_type, n, MXK_KIND_INT, bits, MXK_VAR_VECTOR, (int)cols, nullptr, 0, packed,
                        packed_nbytes, scales, n, workspace, workspace_nbytes, stream);
  }
  if (!(bits == 2 || bits == 4 || bits == 8))
    return fail(MXK_EUNSUPPORTED, "dynamic_quantize(per_channel/per_tensor): widths 2, 4 and 8 are implemented");
  if (packed_nbytes != mxk_packed_nbytes(bits, n))
    return fail(MXK_EINVAL, "dynamic_quantize: packed buffer must hold exactly pack_auto's bytes");
  if (!workspace || workspace_nbytes < mxk_dynamic_quantize_workspace(rows, cols, granularity, bits))
    return fail(MXK_EINVAL, "dynamic_quantize: workspace too small");
  uint32_t* amax = reinterpret_cast<uint32_t*>(workspace);
  uint8_t* pk = reinterpret_cast<uint8_t*>(packed);
  switch (x_type) {
    case MXK_IN_F32:
      return dyn_run(reinterpret_cast<const float*>(x), rows, cols, granularity, bits, pk, packed_nbytes, scales, amax, st);
    case MXK_IN_F16:
      return dyn_run(reinterpret_cast<const __half*>(x), rows, cols, granularity, bits, pk, packed_nbytes, scales, amax, st);
    default:
      return dyn_run(reinterpret_cast<const hip_bfloat16*>(x), rows, cols, granularity, bits, pk, packed_nbytes, scales,
                     amax, st);
  }
}

int mxk_vector_quantize(const void* x, int x_type, int64_t rows, int64_t cols, int axis, int bits, int32_t* codes,
                        float* scales, void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (rows <= 0 || cols <= 0) return fail(MXK_EINVAL, "vector_quantize: rows and cols must be positive");
  if (!x || !codes || !scales) return fail(MXK_EINVAL, "vector_quantize: null buffer");
  if (axis != 0 && axis != 1) return fail(MXK_EINVAL, "vector_quantize: axis must be 0 or 1");
  if (bits < 2 || bits > 16) return fail(MXK_EUNSUPPORTED, "vector_quantize: widths 2..16 are implemented");
  switch (x_type) {
    case MXK_IN_F32: return vec_run(reinterpret_cast<const float*>(x), rows, cols, axis, bits, codes, scales, st);
    case MXK_IN_F16: return vec_run(reinterpret_cast<const __half*>(x), rows, cols, axis, bits, codes, scales, st);
    case MXK_IN_BF16:
      return vec_run(reinterpret_cast<const hip_bfloat16*>(x), rows, cols, axis, bits, codes, scales, st);
    default: return fail(MXK_EINVAL, "vector_quantize: x_type must be f32, f16 or bf16");
  }
}

int mxk_vector_dequantize(const int32_t* codes, const float* scales, int64_t rows, int64_t cols, int axis, float* out,
                          void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (rows <= 0 || cols <= 0) return fail(MXK_EINVAL, "vector_dequantize: rows and cols must be positive");
  if (!codes || !scales || !out) return fail(MXK_EINVAL, "vector_dequantize: null buffer");
  if (axis != 0 && axis != 1) return fail(MXK_EINVAL, "vector_dequantize: axis must be 0 or 1");
  const int64_t n = rows * cols;
  if (cols % 4 == 0 && aligned16(codes) && aligned16(out) && aligned16(scales)) {
    const dim3 gv((unsigned)std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, 4 * 1024), (int64_t)num_cus() * 16)));
    if (axis == 1) hipLaunchKernelGGL(k_vec_decode_v<true>, gv, dim3(256), 0, st, codes, n, cols, scales, out);
    else hipLaunchKernelGGL(k_vec_decode_v<false>, gv, dim3(256), 0, st, codes, n, cols, scales, out);
    return check_launch("vector_dequantize");
  }
  const dim3 g((unsigned)std::min<int64_t>(ceil_div(n, 256), (int64_t)num_cus() * 32));
  if (axis == 1) hipLaunchKernelGGL(k_vec_decode<true>, g, dim3(256), 0, st, codes, n, cols, scales, out);
  else hipLaunchKernelGGL(k_vec_decode<false>, g, dim3(256), 0, st, codes, n, cols, scales, out);
  return check_launch("vector_dequantize");
}

}  // extern "C"
