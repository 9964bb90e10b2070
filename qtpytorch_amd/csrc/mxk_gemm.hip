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

// int8 B [K][N] (row-major, N % 16 == 0) to k-contiguous rows
// B8[n][k] (n < Npad, k < KBP) when the padded block equals the block
// (block % 64 == 0): a 64x64 byte tile per workgroup through LDS, 16-byte
// loads along n and 16-byte stores along k; zeros past K and past N.
__global__ __launch_bounds__(256) void k_transpose_b8(const int8_t* __restrict__ B, int64_t K, int64_t N,
                                                      int64_t Npad, int64_t KBP, int8_t* __restrict__ B8) {
  __shared__ uint8_t tile[64][64 + 4];
  const int t = threadIdx.x;
  const int64_t n0 = (int64_t)blockIdx.x * 64, k0 = (int64_t)blockIdx.y * 64;
  {
    const int kr = t >> 2, nc = (t & 3) * 16;
    const int64_t k = k0 + kr, n = n0 + nc;
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (k < K && n < N) v = *reinterpret_cast<const u32x4*>(B + k * N + n);
    const uint8_t* vb = reinterpret_cast<const uint8_t*>(&v);
#pragma unroll
    for (int i = 0; i < 16; ++i) tile[kr][nc + i] = vb[i];
  }
  __syncthreads();
  {
    const int nr = t >> 2, kc = (t & 3) * 16;
    const int64_t n = n0 + nr, k = k0 + kc;
    if (n < Npad && k < KBP) {
      uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int i = 0; i < 16; ++i) w[i >> 2] |= (uint32_t)tile[kc + i][nr] << ((i & 3) * 8);
      *reinterpret_cast<u32x4*>(B8 + n * KBP + k) = u32x4{w[0], w[1], w[2], w[3]};
    }
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
                                                  int KB, int BP, float* __restrict__ C, int32_t* __restrict__ acc_out,
                                                  const float* __restrict__ bias) {
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
          if (col < N) C[row * N + col] = bias ? c[a][b][i] + bias[col] : c[a][b][i];
        }
      }
  }
}

// v2 for blocks of 65..128 (one 128-byte padded K block, BP = 128): the
// same 128x128 tile and MFMA layout, one K block per pipeline stage, two
// LDS buffers.  The next stage's A/B tiles go straight from global memory to
// LDS (global_load_lds_dwordx4: lane L of a wave instruction fills bytes
// 16L..16L+15 of a 1 KiB window) while the MFMAs and the fp32 epilogue of
// the current stage run; one barrier per K block.  Rows are 128 bytes with
// no padding; the 16-byte chunk c of row r sits in slot c ^ ((r >> 1) & 7),
// which makes the 16-row fragment reads of a wave bank-conflict free.  SA
// comes pre-transposed ([KB][M]), SB is a row of b_scales; both go through
// registers into LDS.
__device__ __forceinline__ int qg2_slot(int r, int c) { return c ^ ((r >> 1) & 7); }

template <bool WRITE_ACC, bool WRITE_C>
__global__ __launch_bounds__(256, 2) void k_qgemm_i8_v2(const int8_t* __restrict__ A8, int64_t lda, int64_t Arows,
                                                        const int8_t* __restrict__ B8, int64_t ldb, int64_t Brows,
                                                        const float* __restrict__ sa_t, int a_ok,
                                                        const float* __restrict__ b_scales, int b_ok, int64_t M,
                                                        int64_t N, int KB, float* __restrict__ C,
                                                        int32_t* __restrict__ acc_out, int grouped,
                                                        const float* __restrict__ bias) {
  __shared__ __attribute__((aligned(1024))) int8_t sA[2][QG_BM * 128];
  __shared__ __attribute__((aligned(1024))) int8_t sB[2][QG_BN * 128];
  __shared__ __attribute__((aligned(16))) float sSA[2][QG_BM];
  __shared__ __attribute__((aligned(16))) float sSB[2][QG_BN];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  // tile order: with `grouped`, the workgroups on one XCD (b % 8) take 8x8
  // blocks of tiles in turn, so that the 64 tiles an XCD runs at once share
  // 8 A row panels and 8 B column panels in its L2; otherwise row-major
  // (the host enables it only when the tile counts are multiples of 8 and
  // the tile total a multiple of 512, so that every XCD owns whole blocks)
  int tm, tn;
  {
    const int b = (int)blockIdx.x;
    const int tiles_n = (int)((N + QG_BN - 1) / QG_BN);
    if (grouped) {
      const int xcd = b & 7, local = b >> 3;
      const int gidx = (local >> 6) * 8 + xcd, within = local & 63;
      const int groups_n = tiles_n >> 3;
      tm = (gidx / groups_n) * 8 + (within >> 3);
      tn = (gidx % groups_n) * 8 + (within & 7);
    } else {
      tm = b / tiles_n;
      tn = b % tiles_n;
    }
  }
  const int64_t m0 = (int64_t)tm * QG_BM, n0 = (int64_t)tn * QG_BN;
  const int lr = lane & 15, lg = lane >> 4;

  // wave w fills rows 32w .. 32w+31 of each tile, 8 rows per instruction:
  // lane L -> row 32w + 8q + (L >> 3), slot L & 7, holding chunk slot ^ ((row >> 1) & 7)
  const int8_t* ga[4];
  const int8_t* gb[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = 32 * wave + 8 * q + (lane >> 3);
    const int cch = qg2_slot(r, lane & 7);
    ga[q] = A8 + std::min<int64_t>(m0 + r, Arows - 1) * lda + cch * 16;
    gb[q] = B8 + std::min<int64_t>(n0 + r, Brows - 1) * ldb + cch * 16;
  }
  auto load_tiles = [&](int kb, int buf) {
    const int64_t k0 = (int64_t)kb * 128;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(ga[q] + k0),
                                       (__attribute__((address_space(3))) void*)(&sA[buf][(32 * wave + 8 * q) * 128]),
                                       16, 0, 0);
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(gb[q] + k0),
                                       (__attribute__((address_space(3))) void*)(&sB[buf][(32 * wave + 8 * q) * 128]),
                                       16, 0, 0);
    }
  };
  auto load_scale = [&](int kb) -> float {
    if (tid < 128) {
      const int64_t row = m0 + tid;
      return (a_ok && row < M) ? sa_t[(int64_t)kb * M + row] : 1.0f;
    }
    const int64_t col = n0 + tid - 128;
    return (b_ok && col < N) ? b_scales[(int64_t)kb * N + col] : 1.0f;
  };
  auto store_scale = [&](int buf, float v) {
    if (tid < 128) sSA[buf][tid] = v;
    else sSB[buf][tid - 128] = v;
  };

  float c[4][4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) c[a][b][i] = 0.0f;

  load_tiles(0, 0);
  store_scale(0, load_scale(0));
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int kb = 0; kb < KB; ++kb) {
    const int cur = kb & 1;
    float rs = 1.0f;
    if (kb + 1 < KB) {
      load_tiles(kb + 1, cur ^ 1);
      rs = load_scale(kb + 1);
    }
    i32x4 p[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) p[a][b] = i32x4{0, 0, 0, 0};
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      i32x4 bf[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int r = wn * 64 + t * 16 + lr;
        bf[t] = *reinterpret_cast<const i32x4*>(&sB[cur][r * 128 + qg2_slot(r, sub * 4 + lg) * 16]);
      }
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int r = wm * 64 + a * 16 + lr;
        const i32x4 af = *reinterpret_cast<const i32x4*>(&sA[cur][r * 128 + qg2_slot(r, sub * 4 + lg) * 16]);
#pragma unroll
        for (int b = 0; b < 4; ++b) p[a][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf[b], p[a][b], 0, 0, 0);
      }
    }
    // epilogue of this K block: C = RN(C + RN(RN(P*SA)*SB))
    float sb[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) sb[b] = sSB[cur][wn * 64 + b * 16 + lr];
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const f32x4v sa4 = *reinterpret_cast<const f32x4v*>(&sSA[cur][wm * 64 + a * 16 + lg * 4]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const float t = ((float)p[a][b][i] * sa4[i]) * sb[b];
          c[a][b][i] = c[a][b][i] + t;
          if (WRITE_ACC) {
            const int64_t row = m0 + wm * 64 + a * 16 + lg * 4 + i;
            const int64_t col = n0 + wn * 64 + b * 16 + lr;
            if (row < M && col < N) acc_out[((int64_t)kb * M + row) * N + col] = p[a][b][i];
          }
        }
      }
    }
    if (kb + 1 < KB) store_scale(cur ^ 1, rs);
    __builtin_amdgcn_s_waitcnt(0);  // this thread's tile loads have landed in LDS
    __syncthreads();
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
          if (col < N) C[row * N + col] = bias ? c[a][b][i] + bias[col] : c[a][b][i];
        }
      }
  }
}

// v3 for large problems, blocks of 65..128: 512 threads (8 waves, 2 per
// SIMD) on a 256x128 tile, each wave 64x64 as in v2 (4 slices of 16 rows x
// 4 column fragments); three LDS stages of one K block each (A 32 KiB, B
// 16 KiB, scales 2 KiB), filled two stages ahead by buffer loads straight to
// LDS (tiles 16 B per lane, scales 4 B per lane).  Every thread issues the
// same 7 loads per stage, spread over the slices of the K block two stages
// earlier, so that one vmcnt value waits for a stage and the LDS writes do
// not pile onto the fragment reads that follow each barrier.  One barrier
// per K block, before the loads that refill the stage every wave has just
// finished.  sa_t is [KB][M] and sb_src [KB][N] (both all ones when the
// reference would use ones).  The host takes this path only when A8, B8
// and both scale arrays stay below 2^31 bytes (32-bit buffer offsets).
#define QG3_BM 256
#define QG3_BN 128
#define QG3_NS 3

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | 0x0F70 | ((N >> 4) << 14));
}

// Barrier without a memory fence: the LDS data a stage reads arrives by
// buffer loads to LDS, whose completion each thread waits for with vmcnt
// before the barrier; a fence here would make the compiler wait for every
// load in flight, including the stages still being prefetched.
__device__ __forceinline__ void qg3_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Fragment reads as inline-asm ds_read_b128 (base VGPR + immediate offset),
// each followed (before first use) by an lgkmcnt wait tied to its result.
// The compiler does not see these as LDS reads, so it does not add vmcnt
// waits for the buffer-load traffic still filling the other stages; every
// LDS op completes in order, so the explicit lgkmcnt counts stay valid.
// Every read must be waited for while its result is still live: the data
// lands in the register asynchronously, and a register the compiler
// considers free could already hold another value.
template <uint32_t OFF>
__device__ __forceinline__ i32x4 qg3_ds_read(uint32_t base) {
  static_assert(OFF < 65536, "ds_read offset field");
  i32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(base), "n"(OFF) : "memory");
  return v;
}
template <int N>
__device__ __forceinline__ void qg3_lgkm_wait(i32x4& v) {
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(v) : "n"(N));
}

typedef int32_t i32x2 __attribute__((ext_vector_type(2)));

// Transposed 8-byte LDS read (ds_read_b64_tr_b8).  Within each group of 16
// lanes, lane i receives byte i % 8 of the 8-byte rows addressed by lanes
// i / 8 + 2j, j = 0..7, as its bytes j.  When lanes 2j and 2j + 1 address
// the two halves of a 16-column segment of K row kappa_j of an N-contiguous
// tile, lane i receives B[kappa_0..7][column i]: eight K values of the i8
// MFMA B operand of column i.  Same waiting rules as qg3_ds_read.
template <uint32_t OFF>
__device__ __forceinline__ i32x2 qg3_ds_read_tr(uint32_t base) {
  static_assert(OFF < 65536, "ds_read offset field");
  i32x2 v;
  asm volatile("ds_read_b64_tr_b8 %0, %1 offset:%2" : "=v"(v) : "v"(base), "n"(OFF) : "memory");
  return v;
}
template <int N>
__device__ __forceinline__ void qg3_lgkm_wait(i32x2& v) {
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(v) : "n"(N));
}

// 16-byte LDS store as inline asm, so that the compiler does not order it
// after the buffer loads to LDS still filling other stages.  The data
// registers are read when the store issues; the store's completion is
// waited for (lgkmcnt 0) before the barrier that publishes the stage.
template <uint32_t OFF>
__device__ __forceinline__ void qg3_ds_write(uint32_t addr, u32x4 v) {
  static_assert(OFF < 65536, "ds_write offset field");
  asm volatile("ds_write_b128 %0, %1 offset:%2" : : "v"(addr), "v"(v), "n"(OFF) : "memory");
}

// Slot (16-byte unit) of chunk c in K row r of an N-contiguous B stage:
// rows r and r + 2 differ in the low two bits of the XOR and rows r and r +
// 16 in the third, so the 32 rows one transposed read touches (8 rows in
// each of 4 lane groups, 16 rows apart) spread over every slot.
__device__ __forceinline__ int qg3_bslot(int r, int c) { return c ^ (((r >> 1) & 3) | ((r >> 2) & 4)); }

// Column (within 16) held at LDS column position l of a B fragment: the
// int4 stages unpack the nibble pairs of every 8 columns as 0,2,4,6,1,3,5,7;
// the same map orders K within the int4 A rows and the rows the B reads take.
template <int MODE>
__device__ __forceinline__ int qg3_lcol(int l) {
  return MODE == 2 ? ((l & 8) | ((l & 3) << 1) | ((l >> 2) & 1)) : l;
}

// Nibbles of 8 int4 codes (w: code 2j in the low nibble of byte j) as 8
// int8 bytes 16 * code: [even codes | odd codes]
__device__ __forceinline__ u32x4 qg3_unpack16(uint32_t w0, uint32_t w1) {
  return u32x4{(w0 << 4) & 0xF0F0F0F0u, w0 & 0xF0F0F0F0u, (w1 << 4) & 0xF0F0F0F0u, w1 & 0xF0F0F0F0u};
}

#define QG3_LDS_BYTES (QG3_NS * (32768 + 16384 + 2048))

// Operand modes of the v3 tile loop:
//   0  A8 [Arows][lda] and B8 [Brows][ldb] int8, both K-contiguous (B8 holds
//      B's columns as rows); fragments by ds_read_b128.
//   1  A8 as in mode 0; B8 is B as stored, [K][ldb = N] int8, N-contiguous:
//      its stages are copied as they are and read with transposed LDS reads,
//      so no pass transposes B.
//   2  int4 codes as stored: A [Arows][lda = K/2 bytes] packed along K, B
//      [K][ldb = N/2 bytes] packed along N.  Each thread loads its share of
//      a stage into VGPRs one K block ahead and unpacks it into the int8 LDS
//      layouts of mode 0 (A) and mode 1 (B).  Code c becomes the byte 16c
//      (its nibble moved to the top of the byte: two instructions per four
//      codes, no sign extension), so the MFMA sums P = sum (16a)(16b), 256
//      times the code product.  sa_t then holds SA * 2^-8, and
//      RN(float(P) * SA * 2^-8) = RN(P/256 * SA) when SA * 2^-8 is exact; with
//      EXACT (some scale is too small for that) sa_t holds SA and P is
//      scaled by 2^-8 first (exact: an integer below 2^24).
//
// REQ (16 or 8): the requantization of C to REQ-bit codes by the 'v' rule
// (mxtorch.py:1372-1385) runs in the epilogue, for N a multiple of 128:
// every 128-element block of the flat C is then one row of a tile, whose
// two 64-column halves belong to waves (wm, 0) and (wm, 1).  The row's
// maximum meets in LDS, s = RN(max(a, 1e-12) / q) and the codes
// rne(clamp(RN(C / s))) use the same functions as the two-pass kernel
// (requant_vec_f32), and the codes go out through an LDS tile as whole
// packed rows.  No fp32 C reaches memory unless WRITE_C asks for it.
template <int MODE, bool WRITE_ACC, bool WRITE_C, bool ROWSCALE, bool EXACT, int REQ = 0>
__device__ __forceinline__ void qg3_run(int8_t* lds, const int8_t* __restrict__ A8, int64_t lda, int64_t Arows,
                                        const int8_t* __restrict__ B8, int64_t ldb, int64_t Brows,
                                        const float* __restrict__ sa_t, const float* __restrict__ sb_src, int64_t M,
                                        int64_t N, int KB, float* __restrict__ C, int32_t* __restrict__ acc_out,
                                        int grouped, const float* __restrict__ bias, uint8_t* __restrict__ cq = nullptr,
                                        float* __restrict__ cq_scales = nullptr) {
  static_assert(MODE == 0 || !ROWSCALE, "row scales are a mode-0 epilogue");
  // [A stages 0..2, 32 KiB each][B stages 0..2, 16 KiB each][scale stages 0..2, 2 KiB each]:
  // a stage's scales hold SA rows at floats 0..255 and SB columns at 256..383
  constexpr uint32_t LA = 0, LB = QG3_NS * 32768, LS = QG3_NS * (32768 + 16384);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  int tm, tn;
  {
    const int b = (int)blockIdx.x;
    const int tiles_n = (int)((N + QG3_BN - 1) / QG3_BN);
    if (grouped) {
      const int xcd = b & 7, local = b >> 3;
      const int gidx = (local >> 6) * 8 + xcd, within = local & 63;
      const int groups_n = tiles_n >> 3;
      tm = (gidx / groups_n) * 8 + (within >> 3);
      tn = (gidx % groups_n) * 8 + (within & 7);
    } else {
      tm = b / tiles_n;
      tn = b % tiles_n;
    }
  }
  const int64_t m0 = (int64_t)tm * QG3_BM, n0 = (int64_t)tn * QG3_BN;
  const int lr = lane & 15, lg = lane >> 4;

  // Per-lane byte offsets of the stage loads; the K block goes into the
  // scalar offset.  A rows 32w + 8q + (L >> 3), B rows 16w + 8q + (L >> 3),
  // chunk = slot ^ ((row >> 1) & 7) as in v2 (mode 1: B K rows, chunk =
  // qg3_bslot(row, slot)); scale float 64w + L.  Mode 2: 16 packed bytes
  // (32 codes) per thread of A rows tid/4 and 128 + tid/4 and of B K row
  // tid/4, at byte 16 (tid % 4) of the K block (A) or of the tile's columns (B).
  uint32_t oa[4], ob[2];
  if constexpr (MODE == 2) {
    const int r = tid >> 2, pc = tid & 3;
    oa[0] = (uint32_t)(std::min<int64_t>(m0 + r, Arows - 1) * lda + pc * 16);
    oa[1] = (uint32_t)(std::min<int64_t>(m0 + 128 + r, Arows - 1) * lda + pc * 16);
    oa[2] = oa[3] = 0;
    ob[0] = (uint32_t)(r * ldb + n0 / 2 + pc * 16);
    ob[1] = 0;
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = 32 * wave + 8 * q + (lane >> 3);
      oa[q] = (uint32_t)(std::min<int64_t>(m0 + r, Arows - 1) * lda + qg2_slot(r, lane & 7) * 16);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int r = 16 * wave + 8 * q + (lane >> 3);
      ob[q] = MODE == 0 ? (uint32_t)(std::min<int64_t>(n0 + r, Brows - 1) * ldb + qg2_slot(r, lane & 7) * 16)
                        : (uint32_t)(r * ldb + n0 + qg3_bslot(r, lane & 7) * 16);
    }
  }
  const int f = 64 * wave + lane;
  // waves 0-3: SA rows, 4-5: SB columns, 6-7: a harmless load of SA row 0
  const bool is_b = wave == 4 || wave == 5;
  const float* gsb = is_b ? sb_src : sa_t;
  const int64_t gstride = is_b ? N : M;
  // SB is stored lane-major: float 256 + 64*wn + 4*lr + t holds column
  // n0 + 64*wn + 16t + qg3_lcol(lr), so a lane's four SB values are one 16-byte read
  const int fb = f - 256;  // 0..127 on waves 4-5
  const uint32_t os =
      (uint32_t)(4 * (f < 256 ? std::min<int64_t>(m0 + f, M - 1)
                              : (f < 384 ? std::min<int64_t>(n0 + (fb & ~63) + (fb & 3) * 16 +
                                                                 qg3_lcol<MODE>((fb & 63) >> 2),
                                                             N - 1)
                                         : 0)));
  const __amdgpu_buffer_rsrc_t rA = make_rsrc(A8, (uint32_t)(Arows * lda));
  const __amdgpu_buffer_rsrc_t rB = make_rsrc(B8, (uint32_t)(Brows * ldb));
  const __amdgpu_buffer_rsrc_t rS = make_rsrc(gsb, (uint32_t)((int64_t)KB * gstride * 4));
  typedef __attribute__((address_space(3))) void* lds_ptr;
  // the 7 loads of a stage in 4 parts: A rows of q 0-1, A rows of q 2-3, B, scales
  auto load_part = [&](int kb, int buf, int part) {
    if (part < 2) {
#pragma unroll
      for (int q = 2 * part; q < 2 * part + 2; ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_ptr)(&lds[LA + buf * 32768 + (32 * wave + 8 * q) * 128]), 16,
                                                 (int)oa[q], kb * 128, 0, 0);
    } else if (part == 2) {
      // mode 1: the K block is 128 rows of ldb bytes (K * N < 2^31, checked by the host)
      const int kboff = MODE == 0 ? kb * 128 : kb * 128 * (int)ldb;
#pragma unroll
      for (int q = 0; q < 2; ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (lds_ptr)(&lds[LB + buf * 16384 + (16 * wave + 8 * q) * 128]), 16,
                                                 (int)ob[q], kboff, 0, 0);
    } else {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rS, (lds_ptr)(&lds[LS + buf * 2048 + 256 * wave]), 4, (int)os,
                                               (int)((int64_t)kb * gstride * 4), 0, 0);
    }
  };

  // LDS byte addresses of this lane's fragments in stage 0: row r = base +
  // 16a + lr keeps (r >> 1) & 7 = (lr >> 1) & 7 for every slice a, so slice
  // a adds a * 2048 (an immediate); a stage adds its size to the bases.
  const int sw = (lr >> 1) & 7;
  const uint32_t l0 = (uint32_t)(uintptr_t)(&lds[0]);
  const uint32_t bA0 = l0 + LA + (wm * 64 + lr) * 128 + ((lg ^ sw) * 16);
  const uint32_t bA1 = l0 + LA + (wm * 64 + lr) * 128 + (((4 + lg) ^ sw) * 16);
  const uint32_t bB0 = l0 + LB + (wn * 64 + lr) * 128 + ((lg ^ sw) * 16);
  const uint32_t bB1 = l0 + LB + (wn * 64 + lr) * 128 + (((4 + lg) ^ sw) * 16);
  const uint32_t bSB = l0 + LS + 4u * (256 + wn * 64 + 4 * lr);
  const uint32_t bSA = l0 + LS + 4u * (wm * 64 + lg * 4);
  // Modes 1 and 2, transposed B reads: lane (lr, lg) addresses K row 16 lg +
  // map(lr / 2) (+ 64 per K half, + 8 for the second read: immediates) at the
  // 8-byte half lr % 2 of column segment 4 wn + t, so that its bytes hold the
  // K values its A fragment holds, in the same order.  The row's slot XOR
  // depends only on lr / 2 and lg, not on the half or the read.
  uint32_t bT[4] = {0u, 0u, 0u, 0u};
  if constexpr (MODE != 0) {
    const int kl = 16 * lg + qg3_lcol<MODE>(lr >> 1);
#pragma unroll
    for (int t = 0; t < 4; ++t) bT[t] = l0 + LB + kl * 128 + qg3_bslot(kl, 4 * wn + t) * 16 + 8 * (lr & 1);
  }
  // Mode 2: the packed codes of one stage in VGPRs, loaded one K block before
  // they are unpacked; the LDS addresses of the unpacked chunks (A rows r and
  // r + 128 share a swizzle, 16 KiB apart)
  u32x4 ra0 = {0u, 0u, 0u, 0u}, ra1 = {0u, 0u, 0u, 0u}, rb = {0u, 0u, 0u, 0u};
  uint32_t wA0 = 0, wA1 = 0, wB0 = 0, wB1 = 0;
  if constexpr (MODE == 2) {
    const int r = tid >> 2, pc = tid & 3;
    wA0 = l0 + LA + r * 128 + qg2_slot(r, 2 * pc) * 16;
    wA1 = l0 + LA + r * 128 + qg2_slot(r, 2 * pc + 1) * 16;
    wB0 = l0 + LB + r * 128 + qg3_bslot(r, 2 * pc) * 16;
    wB1 = l0 + LB + r * 128 + qg3_bslot(r, 2 * pc + 1) * 16;
  }
  auto load4 = [&](int kb) {
    ra0 = buf_load_b128(rA, oa[0], (uint32_t)kb * 64u);
    ra1 = buf_load_b128(rA, oa[1], (uint32_t)kb * 64u);
    rb = buf_load_b128(rB, ob[0], (uint32_t)kb * 128u * (uint32_t)ldb);
  };
  auto write4 = [&](int buf) {
    const uint32_t da = (uint32_t)buf * 32768u, db = (uint32_t)buf * 16384u;
    qg3_ds_write<0>(wA0 + da, qg3_unpack16(ra0[0], ra0[1]));
    qg3_ds_write<0>(wA1 + da, qg3_unpack16(ra0[2], ra0[3]));
    qg3_ds_write<16384>(wA0 + da, qg3_unpack16(ra1[0], ra1[1]));
    qg3_ds_write<16384>(wA1 + da, qg3_unpack16(ra1[2], ra1[3]));
    qg3_ds_write<0>(wB0 + db, qg3_unpack16(rb[0], rb[1]));
    qg3_ds_write<0>(wB1 + db, qg3_unpack16(rb[2], rb[3]));
  };
  const int lcol = qg3_lcol<MODE>(lr);

  float c[4][4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) c[a][b][i] = 0.0f;
  // slice 3 of the previous K block, applied during slice 0 of the next one
  // (zeros before the first block: C + RN(RN(0*0)*0) = C for C = +0)
  i32x4 p3[4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
  i32x4 sa3 = {0, 0, 0, 0}, sb3 = {0, 0, 0, 0};

  // C = RN(C + RN(RN(P*SA)*SB)) for output (slice a, row i, fragment t) of K block kbw;
  // ROWSCALE (SA the same in every K block of a row): C = fma(P, SB, C), times SA at the end
  auto epi_elem = [&](int a, int i, int t, const i32x4 (&p)[4], const i32x4& sav, const i32x4& sbvv, int kbw) {
    if constexpr (ROWSCALE) {
      c[a][t][i] = __builtin_fmaf((float)p[t][i], __int_as_float(sbvv[t]), c[a][t][i]);
    } else {
      float pf = (float)p[t][i];
      if constexpr (MODE == 2 && EXACT) pf = pf * 0.00390625f;
      const float v = (pf * __int_as_float(sav[i])) * __int_as_float(sbvv[t]);
      c[a][t][i] = c[a][t][i] + v;
    }
    if (WRITE_ACC) {
      const int64_t row = m0 + wm * 64 + a * 16 + lg * 4 + i;
      const int64_t col = n0 + wn * 64 + t * 16 + lcol;
      if (kbw >= 0 && row < M && col < N)
        acc_out[((int64_t)kbw * M + row) * N + col] = MODE == 2 ? (p[t][i] >> 8) : p[t][i];
    }
  };

  auto body = [&](int kb, int cur) {
    // stage bases for this K block; fragment offsets are immediates
    const uint32_t b0 = bA0 + (uint32_t)cur * 32768u, b1 = bA1 + (uint32_t)cur * 32768u;
    const uint32_t bb0 = bB0 + (uint32_t)cur * 16384u, bb1 = bB1 + (uint32_t)cur * 16384u;
    const uint32_t bsa = bSA + (uint32_t)cur * 2048u, bsb = bSB + (uint32_t)cur * 2048u;
    uint32_t bt[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) bt[t] = bT[t] + (uint32_t)cur * 16384u;
    // stage kb has landed once at most the next stage's loads are pending
    // (modes 0/1: its 7 loads; mode 2: the 3 packed loads and the scale load
    // of stage kb+1); mode 2 also waits for its own LDS stores of stage kb
    if constexpr (MODE == 2) {
      if (kb + 1 < KB) wait_vmcnt<4>();
      else wait_vmcnt<0>();
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    } else {
      if (kb + 1 < KB) wait_vmcnt<7>();
      else wait_vmcnt<0>();
    }
    qg3_barrier();  // stage kb visible; every wave is done with stage kb-1
    const bool ld = kb + 2 < KB;
    const int lbuf = cur == 0 ? 2 : cur - 1;
    // reads in need order, at most 15 in flight (the lgkmcnt limit): A
    // slice 0, B column fragments 0..3, SB, SA0, A slice 1, SA1
    i32x4 af[4][2], bf[2][4], sa[4], sbv;
    // modes 1/2: B fragment (h, t) is two transposed reads (K rows 0-7 and 8-15 of its lane group)
    i32x2 btr[4][4];
    auto issue_b = [&](int t) {
      btr[t][0] = qg3_ds_read_tr<0>(bt[t]);
      btr[t][1] = qg3_ds_read_tr<1024>(bt[t]);
      btr[t][2] = qg3_ds_read_tr<8192>(bt[t]);
      btr[t][3] = qg3_ds_read_tr<8192 + 1024>(bt[t]);
    };
    af[0][0] = qg3_ds_read<0>(b0);
    af[0][1] = qg3_ds_read<0>(b1);
    if constexpr (MODE == 0) {
      bf[0][0] = qg3_ds_read<0 * 2048>(bb0);
      bf[1][0] = qg3_ds_read<0 * 2048>(bb1);
      bf[0][1] = qg3_ds_read<1 * 2048>(bb0);
      bf[1][1] = qg3_ds_read<1 * 2048>(bb1);
      bf[0][2] = qg3_ds_read<2 * 2048>(bb0);
      bf[1][2] = qg3_ds_read<2 * 2048>(bb1);
      bf[0][3] = qg3_ds_read<3 * 2048>(bb0);
      bf[1][3] = qg3_ds_read<3 * 2048>(bb1);
      sbv = qg3_ds_read<0>(bsb);
      sa[0] = qg3_ds_read<0>(bsa);
      af[1][0] = qg3_ds_read<2048>(b0);
      af[1][1] = qg3_ds_read<2048>(b1);
      sa[1] = qg3_ds_read<64>(bsa);
    } else {
      // 2 + 12 reads; column fragment 3, the scales and A slice 1 follow
      // once the first pairs have been waited for
      issue_b(0);
      issue_b(1);
      issue_b(2);
    }
    __builtin_amdgcn_sched_barrier(0);
    auto slice_mfma = [&](int a, i32x4 (&p)[4]) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        p[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[a][0], bf[0][t], i32x4{0, 0, 0, 0}, 0, 0, 0);
        p[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[a][1], bf[1][t], p[t], 0, 0, 0);
      }
    };
    auto slice_epilogue = [&](int a, const i32x4 (&p)[4], const i32x4& sav) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int t = 0; t < 4; ++t) epi_elem(a, i, t, p, sav, sbv, kb);
    };
    // The MFMAs of slice a+1 go one by one between the epilogue VALU ops of
    // slice a (8 MFMAs, 64 VALU ops), so the matrix core runs while the same
    // wave issues the epilogue.
#define QG3_INTERLEAVE()                                 \
    for (int ii = 0; ii < 8; ++ii) {                     \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); \
      __builtin_amdgcn_sched_group_barrier(0x002, 8, 0); \
    }
    i32x4 p0[4], p1[4];
    // Slice 0: MFMA pair t waits only for its own fragments (A0 and B
    // column fragment t: the first 4 + 2t reads); the carried slice-3
    // epilogue of the previous K block fills the gaps, 2 outputs (8 VALU
    // ops) per chunk.
    auto chunk = [&](int j) {
      epi_elem(3, (2 * j) >> 2, (2 * j) & 3, p3, sa3, sb3, kb - 1);
      epi_elem(3, (2 * j + 1) >> 2, (2 * j + 1) & 3, p3, sa3, sb3, kb - 1);
    };
#define QG3_SLICE0_PAIR(T, WAITN)                                                                   \
    chunk(2 * T);                                                                                   \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    qg3_lgkm_wait<WAITN>(af[0][0]);                                                                 \
    qg3_lgkm_wait<WAITN>(af[0][1]);                                                                 \
    qg3_lgkm_wait<WAITN>(bf[0][T]);                                                                 \
    qg3_lgkm_wait<WAITN>(bf[1][T]);                                                                 \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    p0[T] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[0][0], bf[0][T], i32x4{0, 0, 0, 0}, 0, 0, 0); \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    chunk(2 * T + 1);                                                                               \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    p0[T] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[0][1], bf[1][T], p0[T], 0, 0, 0);             \
    __builtin_amdgcn_sched_barrier(0);
// modes 1/2: the pair's B fragments are its 4 transposed reads
#define QG3_SLICE0_PAIRT(T, WAITN)                                                                  \
    chunk(2 * T);                                                                                   \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    qg3_lgkm_wait<WAITN>(af[0][0]);                                                                 \
    qg3_lgkm_wait<WAITN>(af[0][1]);                                                                 \
    qg3_lgkm_wait<WAITN>(btr[T][0]);                                                                \
    qg3_lgkm_wait<WAITN>(btr[T][1]);                                                                \
    qg3_lgkm_wait<WAITN>(btr[T][2]);                                                                \
    qg3_lgkm_wait<WAITN>(btr[T][3]);                                                                \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    bf[0][T] = i32x4{btr[T][0][0], btr[T][0][1], btr[T][1][0], btr[T][1][1]};                       \
    bf[1][T] = i32x4{btr[T][2][0], btr[T][2][1], btr[T][3][0], btr[T][3][1]};                       \
    p0[T] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[0][0], bf[0][T], i32x4{0, 0, 0, 0}, 0, 0, 0); \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    chunk(2 * T + 1);                                                                               \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    p0[T] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[0][1], bf[1][T], p0[T], 0, 0, 0);             \
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (MODE == 0) {
      QG3_SLICE0_PAIR(0, 11)
      QG3_SLICE0_PAIR(1, 9)
      QG3_SLICE0_PAIR(2, 7)
      QG3_SLICE0_PAIR(3, 5)
    } else {
      // in flight: A0 (2), fragments 0-2 (12); pair t needs A0 and fragment t
      QG3_SLICE0_PAIRT(0, 8)
      issue_b(3);  // fragments 1-3: 12 in flight
      QG3_SLICE0_PAIRT(1, 8)
      sbv = qg3_ds_read<0>(bsb);
      sa[0] = qg3_ds_read<0>(bsa);
      af[1][0] = qg3_ds_read<2048>(b0);
      af[1][1] = qg3_ds_read<2048>(b1);
      sa[1] = qg3_ds_read<64>(bsa);  // fragments 2-3 and these 5: 13 in flight
      __builtin_amdgcn_sched_barrier(0);
      QG3_SLICE0_PAIRT(2, 9)
      QG3_SLICE0_PAIRT(3, 5)
    }
#undef QG3_SLICE0_PAIR
#undef QG3_SLICE0_PAIRT
    qg3_lgkm_wait<0>(sbv);
    qg3_lgkm_wait<0>(sa[0]);
    qg3_lgkm_wait<0>(af[1][0]);
    qg3_lgkm_wait<0>(af[1][1]);
    qg3_lgkm_wait<0>(sa[1]);
    af[2][0] = qg3_ds_read<2 * 2048>(b0);
    af[2][1] = qg3_ds_read<2 * 2048>(b1);
    sa[2] = qg3_ds_read<128>(bsa);
    af[3][0] = qg3_ds_read<3 * 2048>(b0);
    af[3][1] = qg3_ds_read<3 * 2048>(b1);
    sa[3] = qg3_ds_read<192>(bsa);
    if (MODE != 2 && ld) load_part(kb + 2, lbuf, 0);
    __builtin_amdgcn_sched_barrier(0);
    slice_mfma(1, p1);
    slice_epilogue(0, p0, sa[0]);
    QG3_INTERLEAVE();
    __builtin_amdgcn_sched_barrier(0);
    qg3_lgkm_wait<3>(af[2][0]);
    qg3_lgkm_wait<3>(af[2][1]);
    qg3_lgkm_wait<3>(sa[2]);
    if (MODE != 2 && ld) load_part(kb + 2, lbuf, 1);
    __builtin_amdgcn_sched_barrier(0);
    slice_mfma(2, p0);
    slice_epilogue(1, p1, sa[1]);
    QG3_INTERLEAVE();
    __builtin_amdgcn_sched_barrier(0);
    qg3_lgkm_wait<0>(af[3][0]);
    qg3_lgkm_wait<0>(af[3][1]);
    qg3_lgkm_wait<0>(sa[3]);
    if constexpr (MODE == 2) {
      // every read of this stage has returned: unpack stage kb+1 (loaded
      // during kb-1) into its buffer, then load stage kb+2 into the VGPRs
      // and its scales into the stage every wave finished before this
      // block's barrier
      if (kb + 1 < KB) write4(cur == 2 ? 0 : cur + 1);
      if (ld) {
        load4(kb + 2);
        load_part(kb + 2, lbuf, 3);
      }
    } else if (ld) {
      load_part(kb + 2, lbuf, 2);
      load_part(kb + 2, lbuf, 3);
    }
    __builtin_amdgcn_sched_barrier(0);
    slice_mfma(3, p3);
    slice_epilogue(2, p0, sa[2]);
    QG3_INTERLEAVE();
    __builtin_amdgcn_sched_barrier(0);
#undef QG3_INTERLEAVE
    sa3 = sa[3];
    sb3 = sbv;
  };

  if constexpr (MODE == 2) {
    // stage 0 unpacked into LDS, stage 1 in flight (packed codes in VGPRs)
    load4(0);
    load_part(0, 0, 3);
    write4(0);
    if (KB > 1) {
      load4(1);
      load_part(1, 1, 3);
    }
  } else {
    load_part(0, 0, 0);
    load_part(0, 0, 1);
    load_part(0, 0, 2);
    load_part(0, 0, 3);
    if (KB > 1) {
      load_part(1, 1, 0);
      load_part(1, 1, 1);
      load_part(1, 1, 2);
      load_part(1, 1, 3);
    }
  }
  int cur = 0;
  for (int kb = 0; kb < KB; ++kb) {
    body(kb, cur);
    cur = cur == 2 ? 0 : cur + 1;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int t = 0; t < 4; ++t) epi_elem(3, i, t, p3, sa3, sb3, KB - 1);
  if (WRITE_C) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t row = m0 + wm * 64 + a * 16 + lg * 4 + i;
        if (row >= M) continue;
        const float rs = ROWSCALE ? sa_t[row] : 1.0f;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int64_t col = n0 + wn * 64 + b * 16 + lcol;
          const float v = ROWSCALE ? c[a][b][i] * rs : c[a][b][i];
          if (col < N) C[row * N + col] = bias ? v + bias[col] : v;
        }
      }
  }
  if constexpr (REQ > 0) {
    constexpr int RB = 128 * REQ / 8;  // bytes of one packed row of the tile
    static_assert(2048 + 256 * RB <= QG3_LDS_BYTES, "requant tile");
    __syncthreads();  // every wave is done with the stage buffers
    uint32_t* smax = reinterpret_cast<uint32_t*>(lds);  // [wn][256 rows] maxima (magnitude bits)
    uint8_t* tile = reinterpret_cast<uint8_t*>(lds) + 2048;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t m = 0u;
#pragma unroll
        for (int b = 0; b < 4; ++b) m = max(m, mag_bits(c[a][b][i]));
        m = group_max_u<16>(m);  // the 16 lanes of lane group lg hold the wave's 64 columns of the row
        if (lr == 0) smax[wn * 256 + wm * 64 + a * 16 + lg * 4 + i] = m;
      }
    __syncthreads();
    constexpr float qf = (float)((1 << (REQ - 1)) - 1);
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rl = wm * 64 + a * 16 + lg * 4 + i;
        const BlockParams bp = block_params<Q_VEC>(amax_clamped(max(smax[rl], smax[256 + rl])), qf);
        const bool nf = !finite_scale(bp.s);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int cl = wn * 64 + b * 16 + lcol;
          const int code = nf ? encode_nonfinite<Q_VEC, REQ>(c[a][b][i], bp, qf, nullptr)
                              : encode<Q_VEC, REQ>(c[a][b][i], bp, qf, nullptr);
          if constexpr (REQ == 16) reinterpret_cast<int16_t*>(tile + rl * RB)[cl] = (int16_t)code;
          else tile[rl * RB + cl] = (uint8_t)code;
        }
        const int64_t row = m0 + rl;
        if (wn == 0 && lr == 0 && row < M) cq_scales[row * (N / 128) + n0 / 128] = bp.s;
      }
    __syncthreads();
    for (int idx = tid; idx < 256 * RB / 16; idx += 512) {
      const int rl = idx / (RB / 16), ch = idx % (RB / 16);
      const int64_t row = m0 + rl;
      if (row < M)
        *reinterpret_cast<u32x4*>(cq + (row * N + n0) * REQ / 8 + ch * 16) =
            *reinterpret_cast<const u32x4*>(tile + rl * RB + ch * 16);
    }
  }
}

template <bool WRITE_ACC, bool WRITE_C, bool ROWSCALE = false>
__global__ __launch_bounds__(512, 1) void k_qgemm_i8_v3(const int8_t* __restrict__ A8, int64_t lda, int64_t Arows,
                                                        const int8_t* __restrict__ B8, int64_t ldb, int64_t Brows,
                                                        const float* __restrict__ sa_t,
                                                        const float* __restrict__ sb_src, int64_t M, int64_t N,
                                                        int KB, float* __restrict__ C, int32_t* __restrict__ acc_out,
                                                        int grouped, const float* __restrict__ bias) {
  __shared__ __attribute__((aligned(1024))) int8_t lds[QG3_LDS_BYTES];
  qg3_run<0, WRITE_ACC, WRITE_C, ROWSCALE, false>(lds, A8, lda, Arows, B8, ldb, Brows, sa_t, sb_src, M, N, KB, C,
                                                  acc_out, grouped, bias);
}

// The packed GEMM on operands as the caller stores them: mode 1 (int8; B
// [K][N]) or mode 2 (int4; A [M][K/2], B [K][N/2]), see qg3_run.  Mode 2
// reads `exact` (written by k_prep_sa4) once: 0 takes sa_s = SA * 2^-8, 1
// the exact epilogue on sa_u = SA.
template <int MODE, bool WRITE_ACC, bool WRITE_C, int REQ = 0>
__global__ __launch_bounds__(512, 1) void k_qgemm_kn(const int8_t* __restrict__ A, int64_t lda, int64_t Arows,
                                                     const int8_t* __restrict__ B, int64_t ldb, int64_t Brows,
                                                     const float* __restrict__ sa_s, const float* __restrict__ sa_u,
                                                     const int* __restrict__ exact, const float* __restrict__ sb_src,
                                                     int64_t M, int64_t N, int KB, float* __restrict__ C,
                                                     int32_t* __restrict__ acc_out, int grouped,
                                                     uint8_t* __restrict__ cq, float* __restrict__ cq_scales) {
  __shared__ __attribute__((aligned(1024))) int8_t lds[QG3_LDS_BYTES];
  if (MODE == 2 && __builtin_amdgcn_readfirstlane(*exact) != 0)
    qg3_run<MODE, WRITE_ACC, WRITE_C, false, true, REQ>(lds, A, lda, Arows, B, ldb, Brows, sa_u, sb_src, M, N, KB, C,
                                                        acc_out, grouped, nullptr, cq, cq_scales);
  else
    qg3_run<MODE, WRITE_ACC, WRITE_C, false, false, REQ>(lds, A, lda, Arows, B, ldb, Brows, sa_s, sb_src, M, N, KB,
                                                         C, acc_out, grouped, nullptr, cq, cq_scales);
}

// ---------------------------------------------------------------- small GEMMs
// int8 codes, block BLK = 128 or 64, operands and scales as stored, for
// shapes whose 256x128 tiles do not give every CU a workgroup (config 1:
// 512^3), in one launch.  One 32x32 output tile per workgroup of 4 waves;
// the K blocks go round-robin to the waves (wave w: blocks w, w + 4, ...).
// For its block a wave
//  - loads its A operands straight from A (rows m0 + 16i + lr, bytes
//    16 lg .. 16 lg + 15 of each 64-wide half of the block; one half for
//    BLK = 64),
//  - copies the block's BLK x 32 slab of B (as stored, N-contiguous) into
//    its own LDS slot and takes the B operands out with ds_read_b64_tr_b8 (K
//    rows 16 lg + 8 rd + lr / 2, half lr % 2 of each 16-column segment:
//    lane lr then holds 8 K values of column lr),
//  - runs 4 v_mfma_i32_16x16x64_i8 per 64-wide half and forms
//    v = RN(RN(P*SA)*SB) for its 16 outputs per lane (v does not depend on C).
// The waves' v meet in LDS, where each thread adds those of its 4 outputs
// to C in K-block order, C = RN(C + v) for kb ascending from C = +0, the
// reference's sum (mxtorch.py:1357-1370).  The B slot is the wave's own, and
// LDS runs one wave's accesses in order: no barrier between the copy and
// the transposed reads.
#define QGS_TILE 32
template <bool WRITE_ACC, bool WRITE_C, int BLK>
__global__ __launch_bounds__(256) void k_qgemm_small(const int8_t* __restrict__ A, const int8_t* __restrict__ B,
                                                     const float* __restrict__ sa, const float* __restrict__ sb,
                                                     int sa_ok, int sb_ok, int64_t M, int64_t K, int64_t N, int KB,
                                                     float* __restrict__ C, int32_t* __restrict__ acc_out) {
  static_assert(BLK == 64 || BLK == 128, "K blocks of one or two MFMA depths");
  constexpr int H = BLK / 64;         // 64-wide halves of a K block
  constexpr int NQ = BLK * QGS_TILE / 16 / 64;  // 16-byte pieces of the B slab per lane
  __shared__ __attribute__((aligned(16))) int8_t sB[4 * BLK * QGS_TILE];
  __shared__ __attribute__((aligned(16))) float sV[4 * 64 * 16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int64_t m0 = (int64_t)blockIdx.y * QGS_TILE, n0 = (int64_t)blockIdx.x * QGS_TILE;
  const __amdgpu_buffer_rsrc_t rA = make_rsrc(A, (uint32_t)(M * K));
  const __amdgpu_buffer_rsrc_t rB = make_rsrc(B, (uint32_t)(K * N));
  const __amdgpu_buffer_rsrc_t rSA = make_rsrc(sa, sa_ok ? (uint32_t)(M * KB * 4) : 0u);
  const __amdgpu_buffer_rsrc_t rSB = make_rsrc(sb, sb_ok ? (uint32_t)((int64_t)KB * N * 4) : 0u);
  constexpr uint32_t OOB = 0x80000000u;  // past every range: the load returns zeros
  // per-lane offsets that do not depend on the K block
  uint32_t oa[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int64_t m = m0 + 16 * i + lr;
    oa[i] = m < M ? (uint32_t)(m * K + 16 * lg) : OOB;
  }
  uint32_t ob[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int c = lane + 64 * q, rr = c >> 1, hh = c & 1;
    ob[q] = n0 + 16 * hh < N ? (uint32_t)(rr * N + n0 + 16 * hh) : OOB;
  }
  int8_t* slot = sB + wave * BLK * QGS_TILE;
  const uint32_t tr_base = (uint32_t)(uintptr_t)slot + (uint32_t)((16 * lg + (lr >> 1)) * QGS_TILE + 8 * (lr & 1));
  float cacc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int own = tid >> 6;  // this thread's (row tile, column tile) of lane `lane` in the sums

  for (int kb0 = 0; kb0 < KB; kb0 += 4) {
    const int kb = kb0 + wave;
    if (kb < KB) {
      u32x4 af[2][H], bl[NQ];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int h = 0; h < H; ++h)
          af[i][h] = buf_load_b128(rA, oa[i] == OOB ? OOB : oa[i] + 64u * h, (uint32_t)kb * (uint32_t)BLK);
#pragma unroll
      for (int q = 0; q < NQ; ++q)
        bl[q] = buf_load_b128(rB, ob[q] == OOB ? OOB : ob[q], (uint32_t)((int64_t)kb * BLK * N));
      float sav[2][4], sbv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t m = m0 + 16 * i + 4 * lg + r;
          sav[i][r] = sa_ok ? __uint_as_float(buf_load_b32(rSA, m < M ? (uint32_t)((m * KB + kb) * 4) : OOB, 0u))
                            : 1.0f;
        }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int64_t n = n0 + 16 * t + lr;
        sbv[t] = sb_ok ? __uint_as_float(buf_load_b32(rSB, n < N ? (uint32_t)(((int64_t)kb * N + n) * 4) : OOB, 0u))
                       : 1.0f;
      }
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int c = lane + 64 * q;
        *reinterpret_cast<u32x4*>(slot + (c >> 1) * QGS_TILE + 16 * (c & 1)) = bl[q];
      }
      // B operands: column tile t, K half h, K rows 16 lg + 8 rd + 0..7
      i32x2 btr[2][H][2];
      btr[0][0][0] = qg3_ds_read_tr<0>(tr_base);
      btr[0][0][1] = qg3_ds_read_tr<8 * QGS_TILE>(tr_base);
      btr[1][0][0] = qg3_ds_read_tr<16>(tr_base);
      btr[1][0][1] = qg3_ds_read_tr<8 * QGS_TILE + 16>(tr_base);
      if constexpr (H == 2) {
        btr[0][H - 1][0] = qg3_ds_read_tr<64 * QGS_TILE>(tr_base);
        btr[0][H - 1][1] = qg3_ds_read_tr<72 * QGS_TILE>(tr_base);
        btr[1][H - 1][0] = qg3_ds_read_tr<64 * QGS_TILE + 16>(tr_base);
        btr[1][H - 1][1] = qg3_ds_read_tr<72 * QGS_TILE + 16>(tr_base);
      }
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int h = 0; h < H; ++h)
#pragma unroll
          for (int rd = 0; rd < 2; ++rd) qg3_lgkm_wait<0>(btr[t][h][rd]);
      i32x4 bf[2][H];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int h = 0; h < H; ++h)
          bf[t][h] = i32x4{btr[t][h][0][0], btr[t][h][0][1], btr[t][h][1][0], btr[t][h][1][1]};
      f32x4v* vout = reinterpret_cast<f32x4v*>(sV + (wave * 64 + lane) * 16);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          i32x4 p = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, af[i][0]), bf[t][0],
                                                          i32x4{0, 0, 0, 0}, 0, 0, 0);
          if constexpr (H == 2)
            p = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, af[i][H - 1]), bf[t][H - 1], p, 0, 0,
                                                      0);
          f32x4v v;
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = ((float)p[r] * sav[i][r]) * sbv[t];
          vout[i * 2 + t] = v;
          if constexpr (WRITE_ACC) {
            const int64_t n = n0 + 16 * t + lr;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int64_t m = m0 + 16 * i + 4 * lg + r;
              if (m < M && n < N) acc_out[((int64_t)kb * M + m) * N + n] = p[r];
            }
          }
        }
    }
    __syncthreads();
    const int nk = KB - kb0 < 4 ? KB - kb0 : 4;
    for (int u = 0; u < nk; ++u) {
      const f32x4v v = *reinterpret_cast<const f32x4v*>(sV + (u * 64 + lane) * 16 + own * 4);
#pragma unroll
      for (int r = 0; r < 4; ++r) cacc[r] = cacc[r] + v[r];
    }
    __syncthreads();
  }
  if constexpr (WRITE_C) {
    const int i = own >> 1, t = own & 1;
    const int64_t n = n0 + 16 * t + lr;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t m = m0 + 16 * i + 4 * lg + r;
      if (m < M && n < N) C[m * N + n] = cacc[r];
    }
  }
}

__global__ __launch_bounds__(256) void k_fill_ones(float* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 1.0f;
}

// sa_t[kb][m] = a_scales[m * KB + kb]: A's scales in K-block-major order
__global__ __launch_bounds__(256) void k_transpose_sa(const float* __restrict__ s, int64_t M, int64_t KB,
                                                      float* __restrict__ t) {
  __shared__ float tile[32][33];
  const int64_t k0 = (int64_t)blockIdx.x * 32, m0 = (int64_t)blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int i = ty; i < 32; i += 8) {
    const int64_t m = m0 + i, k = k0 + tx;
    tile[i][tx] = (m < M && k < KB) ? s[m * KB + k] : 0.0f;
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    const int64_t k = k0 + i, m = m0 + tx;
    if (k < KB && m < M) t[k * M + m] = tile[tx][i];
  }
}

// The int4 loop's A scales: ts[kb][m] = SA * 2^-8 and tu[kb][m] = SA for SA
// = s[m * KB + kb] (1 when s is null); *exact becomes 1 when some SA * 2^-8
// is inexact (an SA below 2^-118 with low bits that the shift drops), which
// selects the loop's exact epilogue.  *exact is zeroed by k_zero_flag first.
__global__ __launch_bounds__(256) void k_prep_sa4(const float* __restrict__ s, int64_t M, int64_t KB,
                                                  float* __restrict__ ts, float* __restrict__ tu,
                                                  int* __restrict__ exact) {
  __shared__ float tile[32][33];
  const int64_t k0 = (int64_t)blockIdx.x * 32, m0 = (int64_t)blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int i = ty; i < 32; i += 8) {
    const int64_t m = m0 + i, k = k0 + tx;
    tile[i][tx] = (m < M && k < KB) ? (s ? s[m * KB + k] : 1.0f) : 0.0f;
  }
  __syncthreads();
  bool lost = false;
  for (int i = ty; i < 32; i += 8) {
    const int64_t k = k0 + i, m = m0 + tx;
    if (k < KB && m < M) {
      const float v = tile[tx][i];
      const float vs = v * 0.00390625f;
      ts[k * M + m] = vs;
      tu[k * M + m] = v;
      lost = lost || (vs * 256.0f != v && v == v);
    }
  }
  if (lost) atomicOr(exact, 1);
}

__global__ void k_zero_flag(int* __restrict__ p) { *p = 0; }

// t[kb][r] (kb_major) or t[r][kb] = s[(r*K + kb*kblk) / B]: the scale of
// the kblk-wide K chunk kb of row r of a [R][K] operand whose flat blocks
// of B elements each carry one scale (0 past the ns scales given).
__global__ __launch_bounds__(256) void k_gather_scales(const float* __restrict__ s, int64_t ns, int64_t R, int64_t K,
                                                       int64_t B, int kblk, int KB, int kb_major,
                                                       float* __restrict__ t) {
  const int64_t total = R * (int64_t)KB;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = kb_major ? i % R : i / KB;
    const int64_t kb = kb_major ? i / R : i % KB;
    const int64_t j = (r * K + kb * kblk) / B;
    t[i] = j < ns ? s[j] : 0.0f;
  }
}

struct GemmPlan {
  int KB, BP;
  int64_t KBP, Mpad, Npad;
  bool direct_a, v2, v3;
  bool small = false;  // k_qgemm_small: int8, block 128 or 64, grids of 256x128 tiles below the CU count
  int kn;  // 1: int8 with B read as stored, 2: int4 A and B read as stored (k_qgemm_kn), 0: unpacking pre-pass
  int req;  // output width requantized in the GEMM's epilogue (kn, N % 128 == 0), 0: a second pass
  size_t a_bytes, b_bytes, c_bytes, q_bytes, sa_bytes, sb_bytes, su_bytes;
};

// `aligned`: both packed operands start on 16 bytes (the as-stored loops
// load 16-byte pieces of them)
static GemmPlan plan_gemm(int64_t M, int64_t K, int64_t N, int bits, int block, int out_bits, bool aligned = true) {
  GemmPlan p;
  p.KB = (int)ceil_div(K, block);
  p.BP = (int)(ceil_div(block, 64) * 64);
  p.KBP = (int64_t)p.KB * p.BP;
  p.Mpad = ceil_div(M, QG_BM) * QG_BM;
  p.Npad = ceil_div(N, QG_BN) * QG_BN;
  auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
  p.c_bytes = out_bits > 0 ? up((size_t)M * (size_t)N * sizeof(float)) : 0;
  p.q_bytes = out_bits > 0 ? up((size_t)ceil_div(M * N, block) * sizeof(float2)) : 0;
  const int64_t lim = (int64_t)1 << 31;
  const bool big = ceil_div(M, QG3_BM) * ceil_div(N, QG3_BN) >= num_cus();
  // (and A's scale transpose fits its grid: M/32 workgroup rows)
  const bool scales32 = (int64_t)p.KB * M * 4 < lim && (int64_t)p.KB * N * 4 < lim && ceil_div(M, 32) < 65536;
  // the as-stored loops: one K block of 128 codes per stage, 32-bit buffer
  // offsets, B rows of whole 16-byte pieces
  p.kn = 0;
  if (aligned && block == 128 && K % 128 == 0 && big && scales32) {
    if (bits == 8 && N % 16 == 0 && M * K < lim && K * N < lim) p.kn = 1;
    if (bits == 4 && N % 32 == 0 && M * K / 2 < lim && K * N / 2 < lim) p.kn = 2;
  }
  p.req = 0;
  if (p.kn) {
    // int8 x int8 -> int16d and int4 x int4 -> int8d codes straight from the epilogue
    if (out_bits > 0 && N % 128 == 0 && out_bits == (p.kn == 1 ? 16 : 8)) {
      p.req = out_bits;
      p.c_bytes = p.q_bytes = 0;
    }
    p.direct_a = true;
    p.v2 = p.v3 = true;
    p.a_bytes = p.b_bytes = 0;
    p.sa_bytes = up((size_t)p.KB * (size_t)M * sizeof(float));
    p.su_bytes = p.kn == 2 ? p.sa_bytes + 256 : 0;  // unscaled SA and the exact flag
    p.sb_bytes = up((size_t)p.KB * (size_t)N * sizeof(float));
    return p;
  }
  // small int8 shapes: one launch on the operands and scales as stored
  p.small = aligned && bits == 8 && (block == 128 || block == 64) && K % block == 0 && N % 16 == 0 && !big &&
            M * K < lim &&
            K * N < lim && (int64_t)p.KB * M * 4 < lim && (int64_t)p.KB * N * 4 < lim &&
            ceil_div(M, QGS_TILE) < 65536;
  if (p.small) {
    p.direct_a = true;
    p.v2 = p.v3 = false;
    p.a_bytes = p.b_bytes = p.sa_bytes = p.sb_bytes = p.su_bytes = 0;
    return p;
  }
  p.su_bytes = 0;
  p.direct_a = (bits == 8 && block % 64 == 0 && K % block == 0);
  p.a_bytes = p.direct_a ? 0 : up((size_t)p.Mpad * (size_t)p.KBP);
  p.b_bytes = up((size_t)p.Npad * (size_t)p.KBP);
  p.v2 = p.BP == 128 && p.KB < 65536 && ceil_div(M, 32) < 65536;  // (k_transpose_sa's grid)
  // v3 addresses A8, B8 and the scale arrays with 32-bit buffer offsets
  const int64_t a_span = p.direct_a ? M * K : p.Mpad * p.KBP;
  const bool fits32 = a_span < lim && p.Npad * p.KBP < lim && scales32;
  p.v3 = p.v2 && fits32 && big;
  p.sa_bytes = p.v2 ? up((size_t)p.KB * (size_t)M * sizeof(float)) : 0;
  p.sb_bytes = p.v3 ? up((size_t)p.KB * (size_t)N * sizeof(float)) : 0;  // ones, when B's scales do not fit
  return p;
}

// ---------------------------------------------------------------- int8 x int8 linear
// fused_int8_linear's operands: x [M][K] and W [N][K] codes, both with K
// contiguous, each with one scale per flat block (Bx, Bw elements).  The
// MFMA kernels need one scale per row per K chunk of kblk (128: v2/v3, 64:
// the one-stage kernel), which holds when kblk divides K, Bx and Bw.
struct I8LinPlan {
  int kblk, KB;
  bool direct_x, direct_w, v2, v3;
  int64_t Mpad, Npad;
  size_t x_bytes, w_bytes, sa_bytes, sb_bytes;
};

static I8LinPlan plan_i8lin(int64_t M, int64_t K, int64_t N, int xbits, int wbits, int64_t xb, int64_t wb) {
  I8LinPlan p{};
  p.kblk = (K % 128 == 0 && xb % 128 == 0 && wb % 128 == 0) ? 128
           : ((K % 64 == 0 && xb % 64 == 0 && wb % 64 == 0) ? 64 : 0);
  if (p.kblk == 0) return p;
  p.KB = (int)(K / p.kblk);
  p.Mpad = ceil_div(M, QG_BM) * QG_BM;
  p.Npad = ceil_div(N, QG_BN) * QG_BN;
  p.direct_x = xbits == 8;
  p.direct_w = wbits == 8;
  auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
  p.x_bytes = p.direct_x ? 0 : up((size_t)p.Mpad * (size_t)K);
  p.w_bytes = p.direct_w ? 0 : up((size_t)p.Npad * (size_t)K);
  p.sa_bytes = up((size_t)p.KB * (size_t)M * sizeof(float));
  p.sb_bytes = up((size_t)p.KB * (size_t)N * sizeof(float));
  p.v2 = p.kblk == 128 && p.KB < 65536;
  const int64_t lim = (int64_t)1 << 31;
  const bool fits32 = (p.direct_x ? M : p.Mpad) * K < lim && (p.direct_w ? N : p.Npad) * K < lim &&
                      (int64_t)p.KB * M * 4 < lim && (int64_t)p.KB * N * 4 < lim;
  p.v3 = p.v2 && fits32 && ceil_div(M, QG3_BM) * ceil_div(N, QG3_BN) >= num_cus();
  return p;
}

}  // namespace mxk

using namespace mxk;

extern "C" {

static size_t qgemm_workspace(int64_t M, int64_t K, int64_t N, int bits, int block, int out_bits, bool aligned) {
  if (M <= 0 || K <= 0 || N <= 0 || block <= 0) return 0;
  const GemmPlan p = plan_gemm(M, K, N, bits, block, out_bits, aligned);
  return p.a_bytes + p.b_bytes + p.c_bytes + p.q_bytes + p.sa_bytes + p.sb_bytes + p.su_bytes + 1024;
}

size_t mxk_qgemm_workspace(int64_t M, int64_t K, int64_t N, int bits, int block, int out_bits) {
  return qgemm_workspace(M, K, N, bits, block, out_bits, true);
}

size_t mxk_qgemm_workspace_any(int64_t M, int64_t K, int64_t N, int bits, int block, int out_bits) {
  // operands not on 16 bytes take the unpacking path, whose buffers the aligned plan leaves out
  return std::max(qgemm_workspace(M, K, N, bits, block, out_bits, true),
                  qgemm_workspace(M, K, N, bits, block, out_bits, false));
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
  GemmPlan p = plan_gemm(M, K, N, bits, block, out_bits, aligned16(a_packed) && aligned16(b_packed));
  // the fused requantization stores whole 16-byte pieces of packed rows
  // (else: two passes, with the buffers mxk_qgemm_workspace_any counts)
  if (p.req && !aligned16(c_packed)) {
    p.req = 0;
    p.c_bytes = (((size_t)M * (size_t)N * sizeof(float)) + 255) & ~(size_t)255;
    p.q_bytes = (((size_t)ceil_div(M * N, block) * sizeof(float2)) + 255) & ~(size_t)255;
  }
  const size_t need = p.a_bytes + p.b_bytes + p.c_bytes + p.q_bytes + p.sa_bytes + p.sb_bytes + p.su_bytes;
  if (!workspace || workspace_nbytes < need)
    return fail(MXK_EINVAL, (aligned16(a_packed) && aligned16(b_packed))
                                ? "qgemm: workspace too small"
                                : "qgemm: workspace too small (packed operands not on 16 bytes take the unpacking "
                                  "path: size the workspace with mxk_qgemm_workspace_any)");
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  const int a_ok = a_nscales == M * p.KB;
  const int b_ok = b_nscales == (int64_t)p.KB * N;
  if (p.kn) {
    // operands as stored: no unpacking or transposing pass
    float* Cb = c_f32 ? c_f32 : (p.c_bytes ? reinterpret_cast<float*>(ws) : nullptr);
    void* qw = ws + p.c_bytes;
    float* sa_s = reinterpret_cast<float*>(ws + p.c_bytes + p.q_bytes);
    float* sb_one = reinterpret_cast<float*>(ws + p.c_bytes + p.q_bytes + p.sa_bytes);
    float* sa_u = p.kn == 2 ? reinterpret_cast<float*>(ws + p.c_bytes + p.q_bytes + p.sa_bytes + p.sb_bytes)
                            : nullptr;
    int* exact = p.kn == 2 ? reinterpret_cast<int*>(reinterpret_cast<uint8_t*>(sa_u) + p.sa_bytes) : nullptr;
    if (!Cb && !acc_i32 && !p.req) return fail(MXK_EINVAL, "qgemm: no output requested");
    const int cap = num_cus() * 8;
    const dim3 tg((unsigned)ceil_div(p.KB, 32), (unsigned)ceil_div(M, 32));
    if (p.kn == 2) {
      hipLaunchKernelGGL(k_zero_flag, dim3(1), dim3(1), 0, st, exact);
      hipLaunchKernelGGL(k_prep_sa4, tg, dim3(256), 0, st, a_ok ? a_scales : nullptr, M, (int64_t)p.KB, sa_s, sa_u,
                         exact);
    } else if (a_ok) {
      hipLaunchKernelGGL(k_transpose_sa, tg, dim3(256), 0, st, a_scales, M, (int64_t)p.KB, sa_s);
    } else {
      hipLaunchKernelGGL(k_fill_ones, dim3((unsigned)std::min<int64_t>(ceil_div((int64_t)p.KB * M, 256), cap)),
                         dim3(256), 0, st, sa_s, (int64_t)p.KB * M);
    }
    const float* sbs = b_scales;
    if (!b_ok) {
      hipLaunchKernelGGL(k_fill_ones, dim3((unsigned)std::min<int64_t>(ceil_div((int64_t)p.KB * N, 256), cap)),
                         dim3(256), 0, st, sb_one, (int64_t)p.KB * N);
      sbs = sb_one;
    }
    const int64_t tiles_m = ceil_div(M, QG3_BM), tiles_n = ceil_div(N, QG3_BN);
    const int grouped = (tiles_m % 8 == 0 && tiles_n % 8 == 0 && (tiles_m * tiles_n) % 512 == 0) ? 1 : 0;
    const dim3 g1((unsigned)(tiles_m * tiles_n));
    const int8_t* A = (const int8_t*)a_packed;
    const int8_t* B = (const int8_t*)b_packed;
    const int64_t lda = p.kn == 2 ? K / 2 : K, ldb = p.kn == 2 ? N / 2 : N;
#define QG_KN_LAUNCH(MODE, WA, WC, REQ)                                                                         \
  hipLaunchKernelGGL((k_qgemm_kn<MODE, WA, WC, REQ>), g1, dim3(512), 0, st, A, lda, M, B, ldb, K, sa_s, sa_u, exact, \
                     sbs, M, N, p.KB, Cb, acc_i32, grouped, (uint8_t*)c_packed, c_scales)
    if (p.req) {
      // c_f32 and acc_i32 (when asked for) are written as well; no workspace C, no second pass
      if (p.kn == 1) {
        if (acc_i32 && c_f32) QG_KN_LAUNCH(1, true, true, 16);
        else if (acc_i32) QG_KN_LAUNCH(1, true, false, 16);
        else if (c_f32) QG_KN_LAUNCH(1, false, true, 16);
        else QG_KN_LAUNCH(1, false, false, 16);
      } else {
        if (acc_i32 && c_f32) QG_KN_LAUNCH(2, true, true, 8);
        else if (acc_i32) QG_KN_LAUNCH(2, true, false, 8);
        else if (c_f32) QG_KN_LAUNCH(2, false, true, 8);
        else QG_KN_LAUNCH(2, false, false, 8);
      }
      return check_launch("qgemm");
    }
    if (p.kn == 1) {
      if (acc_i32 && Cb) QG_KN_LAUNCH(1, true, true, 0);
      else if (acc_i32) QG_KN_LAUNCH(1, true, false, 0);
      else QG_KN_LAUNCH(1, false, true, 0);
    } else {
      if (acc_i32 && Cb) QG_KN_LAUNCH(2, true, true, 0);
      else if (acc_i32) QG_KN_LAUNCH(2, true, false, 0);
      else QG_KN_LAUNCH(2, false, true, 0);
    }
#undef QG_KN_LAUNCH
    int rc = check_launch("qgemm");
    if (rc != MXK_OK) return rc;
    if (out_bits > 0)
      return requant_vec_f32(Cb, M * N, out_bits, block, c_packed, c_packed_nbytes, c_scales, M * N, qw, p.q_bytes,
                             st);
    return MXK_OK;
  }
  if (p.small) {
    float* Cb = c_f32 ? c_f32 : (p.c_bytes ? reinterpret_cast<float*>(ws) : nullptr);
    if (!Cb && !acc_i32) return fail(MXK_EINVAL, "qgemm: no output requested");
    const dim3 grid((unsigned)ceil_div(N, QGS_TILE), (unsigned)ceil_div(M, QGS_TILE));
    const int8_t* A = (const int8_t*)a_packed;
    const int8_t* B = (const int8_t*)b_packed;
#define QGS_LAUNCH(WA, WC, BLK)                                                                               \
  hipLaunchKernelGGL((k_qgemm_small<WA, WC, BLK>), grid, dim3(256), 0, st, A, B, a_scales, b_scales, a_ok, b_ok, M, \
                     K, N, p.KB, Cb, acc_i32)
    if (block == 128) {
      if (acc_i32 && Cb) QGS_LAUNCH(true, true, 128);
      else if (acc_i32) QGS_LAUNCH(true, false, 128);
      else QGS_LAUNCH(false, true, 128);
    } else {
      if (acc_i32 && Cb) QGS_LAUNCH(true, true, 64);
      else if (acc_i32) QGS_LAUNCH(true, false, 64);
      else QGS_LAUNCH(false, true, 64);
    }
#undef QGS_LAUNCH
    const int rc = check_launch("qgemm");
    if (rc != MXK_OK || out_bits <= 0) return rc;
    return requant_vec_f32(Cb, M * N, out_bits, block, c_packed, c_packed_nbytes, c_scales, M * N, ws + p.c_bytes,
                           p.q_bytes, st);
  }
  int8_t* A8 = p.direct_a ? (int8_t*)a_packed : reinterpret_cast<int8_t*>(ws);
  int8_t* B8 = reinterpret_cast<int8_t*>(ws + p.a_bytes);
  float* Cbuf = c_f32 ? c_f32 : (p.c_bytes ? reinterpret_cast<float*>(ws + p.a_bytes + p.b_bytes) : nullptr);
  void* qws = ws + p.a_bytes + p.b_bytes + p.c_bytes;
  float* sa_t = p.v2 ? reinterpret_cast<float*>(ws + p.a_bytes + p.b_bytes + p.c_bytes + p.q_bytes) : nullptr;
  float* sb_one = p.v3 ? reinterpret_cast<float*>(ws + p.a_bytes + p.b_bytes + p.c_bytes + p.q_bytes + p.sa_bytes)
                       : nullptr;
  const int64_t a_bytes_src = mxk_packed_nbytes(bits, M * K);
  const int64_t b_bytes_src = mxk_packed_nbytes(bits, K * N);
  const int cap = num_cus() * 8;
  if (!p.direct_a) {
    const int64_t total = p.Mpad * (p.KBP / 16);
    hipLaunchKernelGGL(k_unpack_rows, dim3((int)std::min<int64_t>(ceil_div(total, 256), cap)), dim3(256), 0, st,
                       (const uint8_t*)a_packed, a_bytes_src, bits, M, p.Mpad, K, K, 1, block, p.BP, p.KB, A8);
  }
  if (bits == 8 && p.BP == block && N % 16 == 0 && (reinterpret_cast<uintptr_t>(b_packed) & 15u) == 0 &&
      ceil_div(p.KBP, 64) < 65536) {
    const dim3 tg((unsigned)ceil_div(p.Npad, 64), (unsigned)ceil_div(p.KBP, 64));
    hipLaunchKernelGGL(k_transpose_b8, tg, dim3(256), 0, st, (const int8_t*)b_packed, K, N, p.Npad, p.KBP, B8);
  } else {
    const int64_t total = p.Npad * (p.KBP / 16);
    hipLaunchKernelGGL(k_unpack_rows, dim3((int)std::min<int64_t>(ceil_div(total, 256), cap)), dim3(256), 0, st,
                       (const uint8_t*)b_packed, b_bytes_src, bits, N, p.Npad, K, 1, N, block, p.BP, p.KB, B8);
  }
  dim3 grid((unsigned)ceil_div(N, QG_BN), (unsigned)ceil_div(M, QG_BM));
  const int64_t lda = p.direct_a ? K : p.KBP;
  const int64_t arows = p.direct_a ? M : p.Mpad;
  const bool wc = Cbuf != nullptr;
  if (!wc && !acc_i32) return fail(MXK_EINVAL, "qgemm: no output requested");
  if (p.v3) {
    const int64_t tiles_m = ceil_div(M, QG3_BM), tiles_n = ceil_div(N, QG3_BN);
    const int grouped = (tiles_m % 8 == 0 && tiles_n % 8 == 0 && (tiles_m * tiles_n) % 512 == 0) ? 1 : 0;
    const dim3 g1((unsigned)(tiles_m * tiles_n));
    if (a_ok) {
      const dim3 tg((unsigned)ceil_div(p.KB, 32), (unsigned)ceil_div(M, 32));
      hipLaunchKernelGGL(k_transpose_sa, tg, dim3(256), 0, st, a_scales, M, (int64_t)p.KB, sa_t);
    } else {
      hipLaunchKernelGGL(k_fill_ones, dim3((unsigned)std::min<int64_t>(ceil_div((int64_t)p.KB * M, 256), cap)),
                         dim3(256), 0, st, sa_t, (int64_t)p.KB * M);
    }
    const float* sbs = b_scales;
    if (!b_ok) {
      hipLaunchKernelGGL(k_fill_ones, dim3((unsigned)std::min<int64_t>(ceil_div((int64_t)p.KB * N, 256), cap)),
                         dim3(256), 0, st, sb_one, (int64_t)p.KB * N);
      sbs = sb_one;
    }
    if (acc_i32 && wc)
      hipLaunchKernelGGL((k_qgemm_i8_v3<true, true>), g1, dim3(512), 0, st, A8, lda, arows, B8, p.KBP, p.Npad, sa_t,
                         sbs, M, N, p.KB, Cbuf, acc_i32, grouped, nullptr);
    else if (acc_i32)
      hipLaunchKernelGGL((k_qgemm_i8_v3<true, false>), g1, dim3(512), 0, st, A8, lda, arows, B8, p.KBP, p.Npad,
                         sa_t, sbs, M, N, p.KB, Cbuf, acc_i32, grouped, nullptr);
    else
      hipLaunchKernelGGL((k_qgemm_i8_v3<false, true>), g1, dim3(512), 0, st, A8, lda, arows, B8, p.KBP, p.Npad,
                         sa_t, sbs, M, N, p.KB, Cbuf, acc_i32, grouped, nullptr);
  } else if (p.v2) {
    const int64_t tiles_m = ceil_div(M, QG_BM), tiles_n = ceil_div(N, QG_BN);
    const int grouped = (tiles_m % 8 == 0 && tiles_n % 8 == 0 && (tiles_m * tiles_n) % 512 == 0) ? 1 : 0;
    const dim3 g1((unsigned)(tiles_m * tiles_n));
    if (a_ok) {
      const dim3 tg((unsigned)ceil_div(p.KB, 32), (unsigned)ceil_div(M, 32));
      hipLaunchKernelGGL(k_transpose_sa, tg, dim3(256), 0, st, a_scales, M, (int64_t)p.KB, sa_t);
    }
    if (acc_i32 && wc)
      hipLaunchKernelGGL((k_qgemm_i8_v2<true, true>), g1, dim3(256), 0, st, A8, lda, arows, B8, p.KBP, p.Npad, sa_t,
                         a_ok, b_scales, b_ok, M, N, p.KB, Cbuf, acc_i32, grouped, nullptr);
    else if (acc_i32)
      hipLaunchKernelGGL((k_qgemm_i8_v2<true, false>), g1, dim3(256), 0, st, A8, lda, arows, B8, p.KBP, p.Npad,
                         sa_t, a_ok, b_scales, b_ok, M, N, p.KB, Cbuf, acc_i32, grouped, nullptr);
    else
      hipLaunchKernelGGL((k_qgemm_i8_v2<false, true>), g1, dim3(256), 0, st, A8, lda, arows, B8, p.KBP, p.Npad,
                         sa_t, a_ok, b_scales, b_ok, M, N, p.KB, Cbuf, acc_i32, grouped, nullptr);
  } else if (acc_i32 && wc)
    hipLaunchKernelGGL((k_qgemm_i8<true, true>), grid, dim3(256), 0, st, A8, lda, arows, B8, p.KBP, p.Npad, a_scales,
                       a_ok, b_scales, b_ok, M, N, p.KB, p.BP, Cbuf, acc_i32, nullptr);
  else if (acc_i32)
    hipLaunchKernelGGL((k_qgemm_i8<true, false>), grid, dim3(256), 0, st, A8, lda, arows, B8, p.KBP, p.Npad,
                       a_scales, a_ok, b_scales, b_ok, M, N, p.KB, p.BP, Cbuf, acc_i32, nullptr);
  else
    hipLaunchKernelGGL((k_qgemm_i8<false, true>), grid, dim3(256), 0, st, A8, lda, arows, B8, p.KBP, p.Npad,
                       a_scales, a_ok, b_scales, b_ok, M, N, p.KB, p.BP, Cbuf, acc_i32, nullptr);
  int rc = check_launch("qgemm");
  if (rc != MXK_OK) return rc;
  if (out_bits > 0)
    return requant_vec_f32(Cbuf, M * N, out_bits, block, c_packed, c_packed_nbytes, c_scales, M * N, qws,
                                     p.q_bytes, st);
  return MXK_OK;
}

size_t mxk_linear_i8_workspace(int64_t M, int64_t K, int64_t N, int x_bits, int w_bits, int64_t x_block,
                               int64_t w_block) {
  if (M <= 0 || K <= 0 || N <= 0 || x_block <= 0 || w_block <= 0) return 0;
  I8LinPlan p = plan_i8lin(M, K, N, x_bits, w_bits, x_block, w_block);
  if (p.kblk == 0) return 0;
  return p.x_bytes + p.w_bytes + p.sa_bytes + p.sb_bytes;
}

int mxk_linear_i8(const void* x_packed, int64_t x_nbytes, const float* x_scales, int64_t x_nscales, int64_t x_block,
                  int x_bits, const void* w_packed, int64_t w_nbytes, const float* w_scales, int64_t w_nscales,
                  int64_t w_block, int w_bits, int64_t M, int64_t K, int64_t N, const float* bias, float* out,
                  void* workspace, size_t workspace_nbytes, void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (M <= 0 || K <= 0 || N <= 0 || x_block <= 0 || w_block <= 0)
    return fail(MXK_EINVAL, "linear_i8: sizes must be positive");
  if (!x_packed || !w_packed || !x_scales || !w_scales || !out) return fail(MXK_EINVAL, "linear_i8: null pointer");
  auto width_ok = [](int b) { return b == 2 || b == 4 || b == 8; };
  if (!width_ok(x_bits) || !width_ok(w_bits))
    return fail(MXK_EUNSUPPORTED, "linear_i8: int code widths 2, 4 and 8 are implemented");
  I8LinPlan p = plan_i8lin(M, K, N, x_bits, w_bits, x_block, w_block);
  if (p.kblk == 0)
    return fail(MXK_EUNSUPPORTED, "linear_i8: needs 64 (or 128) dividing K and both block sizes");
  if (x_nbytes < mxk_packed_nbytes(x_bits, M * K) || w_nbytes < mxk_packed_nbytes(w_bits, N * K))
    return fail(MXK_EINVAL, "linear_i8: packed operand shorter than its codes");
  if (x_nscales < ceil_div(M * K, x_block) || w_nscales < ceil_div(N * K, w_block))
    return fail(MXK_EINVAL, "linear_i8: fewer scales than blocks");
  if ((p.direct_x && !aligned16(x_packed)) || (p.direct_w && !aligned16(w_packed)))
    return fail(MXK_EINVAL, "linear_i8: 8-bit codes must be 16-byte aligned");
  const size_t need = p.x_bytes + p.w_bytes + p.sa_bytes + p.sb_bytes;
  if (!workspace || workspace_nbytes < need) return fail(MXK_EINVAL, "linear_i8: workspace too small");
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  const int8_t* A8 = p.direct_x ? (const int8_t*)x_packed : reinterpret_cast<int8_t*>(ws);
  const int8_t* B8 = p.direct_w ? (const int8_t*)w_packed : reinterpret_cast<int8_t*>(ws + p.x_bytes);
  float* sa = reinterpret_cast<float*>(ws + p.x_bytes + p.w_bytes);
  float* sb = reinterpret_cast<float*>(ws + p.x_bytes + p.w_bytes + p.sa_bytes);
  const int cap = num_cus() * 8;
  if (!p.direct_x) {
    const int64_t total = p.Mpad * (K / 16);
    hipLaunchKernelGGL(k_unpack_rows, dim3((unsigned)std::min<int64_t>(ceil_div(total, 256), cap)), dim3(256), 0, st,
                       (const uint8_t*)x_packed, x_nbytes, x_bits, M, p.Mpad, K, K, 1, p.kblk, p.kblk, p.KB,
                       (int8_t*)A8);
  }
  if (!p.direct_w) {
    const int64_t total = p.Npad * (K / 16);
    hipLaunchKernelGGL(k_unpack_rows, dim3((unsigned)std::min<int64_t>(ceil_div(total, 256), cap)), dim3(256), 0, st,
                       (const uint8_t*)w_packed, w_nbytes, w_bits, N, p.Npad, K, K, 1, p.kblk, p.kblk, p.KB,
                       (int8_t*)B8);
  }
  // SA: [KB][M] for v2/v3, [M][KB] for the one-stage kernel; SB: [KB][N]
  hipLaunchKernelGGL(k_gather_scales, dim3((unsigned)std::min<int64_t>(ceil_div(M * p.KB, 256), cap)), dim3(256), 0,
                     st, x_scales, x_nscales, M, K, x_block, p.kblk, p.KB, p.v2 ? 1 : 0, sa);
  hipLaunchKernelGGL(k_gather_scales, dim3((unsigned)std::min<int64_t>(ceil_div(N * p.KB, 256), cap)), dim3(256), 0,
                     st, w_scales, w_nscales, N, K, w_block, p.kblk, p.KB, 1, sb);
  const int64_t arows = p.direct_x ? M : p.Mpad, brows = p.direct_w ? N : p.Npad;
  if (p.v3) {
    const int64_t tiles_m = ceil_div(M, QG3_BM), tiles_n = ceil_div(N, QG3_BN);
    const int grouped = (tiles_m % 8 == 0 && tiles_n % 8 == 0 && (tiles_m * tiles_n) % 512 == 0) ? 1 : 0;
    // per-token activations (one x scale per row): the row scale leaves the K loop
    if (x_block % K == 0)
      hipLaunchKernelGGL((k_qgemm_i8_v3<false, true, true>), dim3((unsigned)(tiles_m * tiles_n)), dim3(512), 0, st,
                         A8, K, arows, B8, K, brows, sa, sb, M, N, p.KB, out, nullptr, grouped, bias);
    else
      hipLaunchKernelGGL((k_qgemm_i8_v3<false, true>), dim3((unsigned)(tiles_m * tiles_n)), dim3(512), 0, st, A8, K,
                         arows, B8, K, brows, sa, sb, M, N, p.KB, out, nullptr, grouped, bias);
  } else if (p.v2) {
    const int64_t tiles_m = ceil_div(M, QG_BM), tiles_n = ceil_div(N, QG_BN);
    const int grouped = (tiles_m % 8 == 0 && tiles_n % 8 == 0 && (tiles_m * tiles_n) % 512 == 0) ? 1 : 0;
    hipLaunchKernelGGL((k_qgemm_i8_v2<false, true>), dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, st, A8, K,
                       arows, B8, K, brows, sa, 1, sb, 1, M, N, p.KB, out, nullptr, grouped, bias);
  } else {
    const dim3 grid((unsigned)ceil_div(N, QG_BN), (unsigned)ceil_div(M, QG_BM));
    hipLaunchKernelGGL((k_qgemm_i8<false, true>), grid, dim3(256), 0, st, A8, K, arows, B8, K, brows, sa, 1, sb, 1,
                       M, N, p.KB, p.kblk, out, nullptr, bias);
  }
  return check_launch("linear_i8");
}

}  // extern "C"
