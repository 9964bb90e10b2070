// Weight-only quantized linear for gfx950: y = x.float() @ dequant(W) (+ bias)
// with W stored as quantize(weight.t()) -> [K=in, N=out] row-major, blocks of
// `block` consecutive flat elements (mx_linear.from_linear / forward,
// mxtorch.py:7439-7473).  The dequantized weight is the reference's
// RN(code * s) (mxtorch.py:1573-1575) and never touches memory.
//
// Generic kernel: 64x64 output tiles, K steps of 16, weights decoded into
// LDS, fp32 FMA accumulation.  Any M, K, N, width and block size.
#include "mxk_internal.h"

#include <algorithm>

namespace mxk {

// decode element `flat` of a packed weight (int, int1 or float grid codes)
template <int MODE, int BITS>
__device__ __forceinline__ float decode_weight(const uint8_t* __restrict__ packed, int64_t pbytes,
                                               const float* __restrict__ scales, int64_t flat, int block,
                                               const float* __restrict__ G) {
  constexpr bool WORDS = !(BITS == 1 || BITS == 2 || BITS == 4 || BITS == 8);
  constexpr int PER = WORDS ? 32 / BITS : 8 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  const int64_t unit = flat / PER;
  const int sh = (int)(flat % PER) * BITS;
  uint32_t f = 0u;
  if (WORDS) {
    if (unit * 4 + 3 < pbytes) f = (reinterpret_cast<const uint32_t*>(packed)[unit] >> sh) & MASK;
  } else {
    if (unit < pbytes) f = ((uint32_t)packed[unit] >> sh) & MASK;
  }
  const float s = scales[flat / block];
  if constexpr (MODE == Q_INT1) {
    return f == 0u ? s : -s;
  } else if constexpr (MODE == Q_FP) {
    return G[f] * s;
  } else {
    int32_t c = (int32_t)(f << (32 - BITS)) >> (32 - BITS);
    return (float)c * s;
  }
}

template <typename T, int MODE, int BITS>
__global__ __launch_bounds__(256) void k_linear_generic(const T* __restrict__ x, int64_t M, int64_t K, int64_t N,
                                                        const uint8_t* __restrict__ packed, int64_t pbytes,
                                                        const float* __restrict__ scales, int block,
                                                        const float* __restrict__ bias, float* __restrict__ out) {
  constexpr int BM = 64, BN = 64, BK = 16;
  constexpr int H = MODE == Q_FP ? (1 << (BITS - 1)) : 1;
  __shared__ float sG[2 * H];
  __shared__ float sx[BK][BM + 4];
  __shared__ float sw[BK][BN + 4];
  if constexpr (MODE == Q_FP) build_tables<BITS>(nullptr, sG);
  const int tid = threadIdx.x;
  const int tm = tid / 16, tn = tid % 16;  // 16x16 threads, 4x4 outputs each
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
  for (int64_t k0 = 0; k0 < K; k0 += BK) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int e = tid + 256 * r;  // 1024 elements per tile
      // x tile: [BM][BK] -> sx[k][m]
      {
        const int mm = e / BK, kk = e % BK;
        const int64_t gm = m0 + mm, gk = k0 + kk;
        sx[kk][mm] = (gm < M && gk < K) ? ElemT<T>::cvt(x[gm * K + gk]) : 0.0f;
      }
      // w tile: [BK][BN]
      {
        const int kk = e / BN, nn = e % BN;
        const int64_t gk = k0 + kk, gn = n0 + nn;
        sw[kk][nn] = (gk < K && gn < N) ? decode_weight<MODE, BITS>(packed, pbytes, scales, gk * N + gn, block, sG) : 0.0f;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BK; ++kk) {
      float xv[4], wv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) xv[i] = sx[kk][tm * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) wv[j] = sw[kk][tn * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(xv[i], wv[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t gm = m0 + tm * 4 + i;
    if (gm >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t gn = n0 + tn * 4 + j;
      if (gn < N) out[gm * N + gn] = bias ? acc[i][j] + bias[gn] : acc[i][j];
    }
  }
}

template <typename T, int MODE, int BITS>
static int launch_linear(const T* x, int64_t M, int64_t K, int64_t N, const uint8_t* packed, int64_t pbytes,
                         const float* scales, int block, const float* bias, float* out, hipStream_t st) {
  dim3 grid((unsigned)ceil_div(N, 64), (unsigned)ceil_div(M, 64));
  hipLaunchKernelGGL((k_linear_generic<T, MODE, BITS>), grid, dim3(256), 0, st, x, M, K, N, packed, pbytes, scales,
                     block, bias, out);
  return check_launch("linear_wq");
}

template <typename T>
static int linear_t(const T* x, int64_t M, int64_t K, int64_t N, const uint8_t* packed, int64_t pbytes,
                    const float* scales, int kind, int bits, int block, const float* bias, float* out,
                    hipStream_t st) {
#define MXK_L(MODE, BITS) \
  if (mode == MODE && bits == BITS) return launch_linear<T, MODE, BITS>(x, M, K, N, packed, pbytes, scales, block, bias, out, st);
  const int mode = kind == MXK_KIND_FLOAT ? Q_FP : (bits == 1 ? Q_INT1 : Q_INT);
  MXK_L(Q_INT1, 1)
  MXK_L(Q_INT, 2)
  MXK_L(Q_INT, 3)
  MXK_L(Q_INT, 4)
  MXK_L(Q_INT, 5)
  MXK_L(Q_INT, 6)
  MXK_L(Q_INT, 7)
  MXK_L(Q_INT, 8)
  MXK_L(Q_INT, 16)
  MXK_L(Q_FP, 4)
  MXK_L(Q_FP, 8)
#undef MXK_L
  return fail(MXK_EUNSUPPORTED, "linear_wq: unsupported weight kind/bits");
}

}  // namespace mxk

using namespace mxk;

extern "C" {

size_t mxk_linear_workspace(int64_t M, int64_t K, int64_t N, int bits, int block) {
  (void)M;
  (void)K;
  (void)N;
  (void)bits;
  (void)block;
  return 0;
}

int mxk_linear_wq(const void* x, int x_type, int64_t M, int64_t K, const void* w_packed, const float* w_scales,
                  int64_t N, int kind, int bits, int block, const float* bias, float* out, void* workspace,
                  size_t workspace_nbytes, void* stream) {
  (void)workspace;
  (void)workspace_nbytes;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (M <= 0 || K <= 0 || N <= 0 || block <= 0) return fail(MXK_EINVAL, "linear_wq: sizes must be positive");
  if (!x || !w_packed || !w_scales || !out) return fail(MXK_EINVAL, "linear_wq: null pointer");
  const int64_t nb = ceil_div(K * N, block);
  const int64_t pbytes = mxk_packed_nbytes(bits, nb * block);
  const uint8_t* pk = reinterpret_cast<const uint8_t*>(w_packed);
  if (x_type == MXK_IN_F32)
    return linear_t<float>((const float*)x, M, K, N, pk, pbytes, w_scales, kind, bits, block, bias, out, st);
  if (x_type == MXK_IN_F16)
    return linear_t<__half>((const __half*)x, M, K, N, pk, pbytes, w_scales, kind, bits, block, bias, out, st);
  if (x_type == MXK_IN_BF16)
    return linear_t<hip_bfloat16>((const hip_bfloat16*)x, M, K, N, pk, pbytes, w_scales, kind, bits, block, bias,
                                  out, st);
  return fail(MXK_EINVAL, "linear_wq: bad input type");
}

}  // extern "C"
