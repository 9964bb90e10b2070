// Packed block-scaled GEMM for gfx950: the CPU semantics of _dispatch_qgemm
// (mxtorch.py:5497-5573) and _qscale_matmul (mxtorch.py:1299-1385).
//
//   codes   A [M,K], B [K,N], both unpacked with a's width (mxtorch.py:5564-5565)
//   SA[m,kb] = a_scales[m*KB+kb]  (ones when a_nscales != M*KB)      mxtorch.py:1352-1353
//   SB[kb,n] = b_scales[kb*N+n]   (ones when b_nscales != KB*N)      mxtorch.py:1354-1355
//   for kb ascending:  P = sum_{k in kb} a*b   (exact integer)
//                      C = RN(C + RN(RN(P*SA)*SB))                   mxtorch.py:1357-1370
//   requantize C per `block` flat elements with the 'v' rule           mxtorch.py:1372-1385
//
// Structure: a pre-pass unpacks the sub-byte codes of A and the columns of
// B into k-contiguous int8 rows, each K block zero-padded to a multiple of
// 64 (one v_mfma_i32_16x16x64_i8 K step).  The main kernel computes a
// 128x128 tile per 256-thread workgroup (2x2 waves of 64x64, 4x4 MFMA
// tiles each), one fresh int32 accumulator per K block, and applies the
// fp32 epilogue in the reference's order (compiled without FMA contraction).
#include "mxk_internal.h"

#include <algorithm>

namespace mxk {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// dst[r][kb*BP + j] = code(r, kb*block + j) for j < block (0 beyond K or
// beyond block), rows r < R are read, rows up to Rpad are zero.  The code
// of (r, k) sits at flat index r*sr + k*sk of a bits-packed buffer.
__global__ __launch_bounds__(256) void k_unpack_rows(const uint8_t* __restrict__ src, int64_t src_nbytes, int bits,
                                                     int64_t R, int64_t Rpad, int64_t K, int64_t sr, int64_t sk,
                                                     int block, int BP, int KB, int8_t* __restrict__ dst) {
  const int64_t KBP = (int64_t)KB * BP;
  const int64_t chunks_per_row = KBP / 16;
  const int64_t total = Rpad * chunks_per_row;
  const int per = 8 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    // consecutive threads take consecutive rows so that B's column reads coalesce
    const int64_t r = t % Rpad, ch = t / Rpad;
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    if (r < R) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int64_t kk = ch * 16 + j;
        const int64_t kb = kk / BP, jj = kk % BP;
        const int64_t k = kb * block + jj;
        int32_t c = 0;
        if (jj < block && k < K) {
          const int64_t flat = r * sr + k * sk;
          const int64_t byte = flat / per;
          if (byte < src_nbytes) {
            uint32_t f = ((uint32_t)src[byte] >> ((flat % per) * bits)) & mask;
            c = (int32_t)(f << (32 - bits)) >> (32 - bits);
          }
        }
        w[j >> 2] |= ((uint32_t)c & 0xFFu) << ((j & 3) * 8);
      }
    }
    *reinterpret_cast<u32x4*>(dst + r * KBP + ch * 16) = u32x4{w[0], w[1], w[2], w[3]};
  }
}

#define QG_BM 128
#define QG_BN 128
#define QG_LDS_STRIDE 80  // 64 bytes of K + 16 bytes of skew per row

template <bool WRITE_ACC, bool WRITE_C>
__global__ __launch_bounds__(256) void k_qgemm_i8(const int8_t* __restrict__ A8, int64_t lda, int64_t Arows,
                                                  const int8_t* __restrict__ B8, int64_t ldb, int64_t Brows,
                                                  const float* __restrict__ a_scales, int a_ok,
                                                  const float* __restrict__ b_scales, int b_ok, int64_t M, int64_t N,
                                                  int KB, int BP, float* __restrict__ C, int32_t* __restrict__ acc_out) {
  __shared__ __attribute__((aligned(16))) int8_t sA[QG_BM * QG_LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) int8_t sB[QG_BN * QG_LDS_STRIDE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.y * QG_BM, n0 = (int64_t)blockIdx.x * QG_BN;
  const int lr = lane & 15, lg = lane >> 4;

  float c[4][4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) c[a][b][i] = 0.0f;

  const int steps = BP / 64;
  for (int kb = 0; kb < KB; ++kb) {
    i32x4 p[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) p[a][b] = i32x4{0, 0, 0, 0};
    for (int s = 0; s < steps; ++s) {
      const int64_t k0 = (int64_t)kb * BP + s * 64;
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int cidx = tid + 256 * it;
        const int row = cidx >> 2, col = (cidx & 3) * 16;
        const int64_t ga = std::min<int64_t>(m0 + row, Arows - 1);
        const int64_t gb = std::min<int64_t>(n0 + row, Brows - 1);
        *reinterpret_cast<u32x4*>(sA + row * QG_LDS_STRIDE + col) =
            *reinterpret_cast<const u32x4*>(A8 + ga * lda + k0 + col);
        *reinterpret_cast<u32x4*>(sB + row * QG_LDS_STRIDE + col) =
            *reinterpret_cast<const u32x4*>(B8 + gb * ldb + k0 + col);
      }
      __syncthreads();
      i32x4 af[4], bf[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        af[t] = *reinterpret_cast<const i32x4*>(sA + (wm * 64 + t * 16 + lr) * QG_LDS_STRIDE + lg * 16);
        bf[t] = *reinterpret_cast<const i32x4*>(sB + (wn * 64 + t * 16 + lr) * QG_LDS_STRIDE + lg * 16);
      }
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) p[a][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[a], bf[b], p[a][b], 0, 0, 0);
      __syncthreads();
    }
    // epilogue of this K block: C = RN(C + RN(RN(P*SA)*SB))
#pragma unroll
    for (int a = 0; a < 4; ++a) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t row = m0 + wm * 64 + a * 16 + lg * 4 + i;
        const float sa = (a_ok && row < M) ? a_scales[row * KB + kb] : 1.0f;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int64_t col = n0 + wn * 64 + b * 16 + lr;
          const float sb = (b_ok && col < N) ? b_scales[(int64_t)kb * N + col] : 1.0f;
          const float t = ((float)p[a][b][i] * sa) * sb;
          c[a][b][i] = c[a][b][i] + t;
          if (WRITE_ACC && row < M && col < N) acc_out[((int64_t)kb * M + row) * N + col] = p[a][b][i];
        }
      }
    }
  }
  if (WRITE_C) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t row = m0 + wm * 64 + a * 16 + lg * 4 + i;
        if (row >= M) continue;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int64_t col = n0 + wn * 64 + b * 16 + lr;
          if (col < N) C[row * N + col] = c[a][b][i];
        }
      }
  }
}

struct GemmPlan {
  int KB, BP;
  int64_t KBP, Mpad, Npad;
  bool direct_a;
  size_t a_bytes, b_bytes, c_bytes, q_bytes;
};

static GemmPlan plan_gemm(int64_t M, int64_t K, int64_t N, int bits, int block, int out_bits) {
  GemmPlan p;
  p.KB = (int)ceil_div(K, block);
  p.BP = (int)(ceil_div(block, 64) * 64);
  p.KBP = (int64_t)p.KB * p.BP;
  p.Mpad = ceil_div(M, QG_BM) * QG_BM;
  p.Npad = ceil_div(N, QG_BN) * QG_BN;
  p.direct_a = (bits == 8 && block % 64 == 0 && K % block == 0);
  auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
  p.a_bytes = p.direct_a ? 0 : up((size_t)p.Mpad * (size_t)p.KBP);
  p.b_bytes = up((size_t)p.Npad * (size_t)p.KBP);
  p.c_bytes = out_bits > 0 ? up((size_t)M * (size_t)N * sizeof(float)) : 0;
  p.q_bytes = out_bits > 0 ? up((size_t)ceil_div(M * N, block) * sizeof(float2)) : 0;
  return p;
}

}  // namespace mxk

using namespace mxk;

extern "C" {

size_t mxk_qgemm_workspace(int64_t M, int64_t K, int64_t N, int bits, int block, int out_bits) {
  if (M <= 0 || K <= 0 || N <= 0 || block <= 0) return 0;
  GemmPlan p = plan_gemm(M, K, N, bits, block, out_bits);
  return p.a_bytes + p.b_bytes + p.c_bytes + p.q_bytes + 1024;
}

int mxk_qgemm(const void* a_packed, const float* a_scales, int64_t a_nscales, const void* b_packed,
              const float* b_scales, int64_t b_nscales, int64_t M, int64_t K, int64_t N, int bits, int block,
              int out_bits, void* c_packed, int64_t c_packed_nbytes, float* c_scales, float* c_f32, int32_t* acc_i32,
              void* workspace, size_t workspace_nbytes, void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (M <= 0 || K <= 0 || N <= 0 || block <= 0) return fail(MXK_EINVAL, "qgemm: sizes must be positive");
  if (!(bits == 1 || bits == 2 || bits == 4 || bits == 8))
    return fail(MXK_EUNSUPPORTED, "qgemm: operand widths 1, 2, 4 and 8 are implemented");
  if (!a_packed || !b_packed || !a_scales || !b_scales) return fail(MXK_EINVAL, "qgemm: null operand");
  if (out_bits > 0 && (!c_packed || !c_scales)) return fail(MXK_EINVAL, "qgemm: packed output needs buffers");
  if (out_bits > 0 && !((out_bits >= 2 && out_bits <= 8) || out_bits == 16))
    return fail(MXK_EUNSUPPORTED, "qgemm: output width must be 2..8 or 16");
  if (out_bits > 0 && c_packed_nbytes < mxk_packed_nbytes(out_bits, M * N))
    return fail(MXK_EINVAL, "qgemm: packed output too small");
  GemmPlan p = plan_gemm(M, K, N, bits, block, out_bits);
  const size_t need = p.a_bytes + p.b_bytes + p.c_bytes + p.q_bytes;
  if (!workspace || workspace_nbytes < need) return fail(MXK_EINVAL, "qgemm: workspace too small");
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  int8_t* A8 = p.direct_a ? (int8_t*)a_packed : reinterpret_cast<int8_t*>(ws);
  int8_t* B8 = reinterpret_cast<int8_t*>(ws + p.a_bytes);
  float* Cbuf = c_f32 ? c_f32 : (p.c_bytes ? reinterpret_cast<float*>(ws + p.a_bytes + p.b_bytes) : nullptr);
  void* qws = ws + p.a_bytes + p.b_bytes + p.c_bytes;
  const int64_t a_bytes_src = mxk_packed_nbytes(bits, M * K);
  const int64_t b_bytes_src = mxk_packed_nbytes(bits, K * N);
  const int cap = num_cus() * 8;
  if (!p.direct_a) {
    const int64_t total = p.Mpad * (p.KBP / 16);
    hipLaunchKernelGGL(k_unpack_rows, dim3((int)std::min<int64_t>(ceil_div(total, 256), cap)), dim3(256), 0, st,
                       (const uint8_t*)a_packed, a_bytes_src, bits, M, p.Mpad, K, K, 1, block, p.BP, p.KB, A8);
  }
  {
    const int64_t total = p.Npad * (p.KBP / 16);
    hipLaunchKernelGGL(k_unpack_rows, dim3((int)std::min<int64_t>(ceil_div(total, 256), cap)), dim3(256), 0, st,
                       (const uint8_t*)b_packed, b_bytes_src, bits, N, p.Npad, K, 1, N, block, p.BP, p.KB, B8);
  }
  const int a_ok = a_nscales == M * p.KB;
  const int b_ok = b_nscales == (int64_t)p.KB * N;
  dim3 grid((unsigned)ceil_div(N, QG_BN), (unsigned)ceil_div(M, QG_BM));
  const int64_t lda = p.direct_a ? K : p.KBP;
  const int64_t arows = p.direct_a ? M : p.Mpad;
  const bool wc = Cbuf != nullptr;
  if (acc_i32 && wc)
    hipLaunchKernelGGL((k_qgemm_i8<true, true>), grid, dim3(256), 0, st, A8, lda, arows, B8, p.KBP, p.Npad, a_scales,
                       a_ok, b_scales, b_ok, M, N, p.KB, p.BP, Cbuf, acc_i32);
  else if (acc_i32)
    hipLaunchKernelGGL((k_qgemm_i8<true, false>), grid, dim3(256), 0, st, A8, lda, arows, B8, p.KBP, p.Npad,
                       a_scales, a_ok, b_scales, b_ok, M, N, p.KB, p.BP, Cbuf, acc_i32);
  else if (wc)
    hipLaunchKernelGGL((k_qgemm_i8<false, true>), grid, dim3(256), 0, st, A8, lda, arows, B8, p.KBP, p.Npad,
                       a_scales, a_ok, b_scales, b_ok, M, N, p.KB, p.BP, Cbuf, acc_i32);
  else
    return fail(MXK_EINVAL, "qgemm: no output requested");
  int rc = check_launch("qgemm");
  if (rc != MXK_OK) return rc;
  if (out_bits > 0)
    return requant_vec_f32(Cbuf, M * N, out_bits, block, c_packed, c_packed_nbytes, c_scales, M * N, qws,
                                     p.q_bytes, st);
  return MXK_OK;
}

}  // extern "C"
