// Weight-only quantized linear for gfx950: y = x.float() @ dequant(W) (+ bias)
// with W stored as quantize(weight.t()) -> [K=in, N=out] row-major, blocks of
// `block` consecutive flat elements (mx_linear.from_linear / forward,
// mxtorch.py:7439-7473).  The dequantized weight is the reference's
// RN(code * s) (mxtorch.py:1573-1575) and never touches memory.
//
// Generic kernel: 64x64 output tiles, K steps of 16, weights decoded into
// LDS, fp32 FMA accumulation.  Any M, K, N, width and block size.  With WT
// the weight is stored [N][K] instead (y = x @ dequant(W)^T, the layout of
// mx_dynamic_linear's weight, mxtorch.py:8916-8917, and of the input
// gradient of _MXLinearAutograd, mxtorch.py:6729-6740).
#include "mxk_internal.h"

#include <algorithm>
#include <mutex>
#include <vector>

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

template <typename T, int MODE, int BITS, bool WT>
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
      // w tile: [BK][BN]; consecutive threads walk the weight's contiguous dimension
      {
        const int kk = WT ? e % BK : e / BN, nn = WT ? e / BK : e % BN;
        const int64_t gk = k0 + kk, gn = n0 + nn;
        const int64_t flat = WT ? gn * K + gk : gk * N + gn;
        sw[kk][nn] = (gk < K && gn < N) ? decode_weight<MODE, BITS>(packed, pbytes, scales, flat, block, sG) : 0.0f;
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

// ---------------------------------------------------------------- int4 decode (M <= 16)
// y[m, n] = sum_k x[m,k] * RN(code[k,n] * s[k, n/128]), weights int4 [K][N]
// packed along N (LSB nibble = even column), block 128 along N.  The kernel
// reads the scales block-major, sT[n/128][k] (mxk_linear_prepack_scales), so
// that a block's scales along K are contiguous.
//
// Work split: a workgroup of 16 waves (4 per SIMD) owns NBW scale blocks
// (NBW*128 output columns) and R = 16/NBW * RPW rows of K.  Wave w takes
// block w % NBW and row group w / NBW.
//
// Start-up order.  Each CU returns memory data in request order, and at
// launch every workgroup asks for its weights at once, so whatever is queued
// first arrives first.  Every wave therefore requests its share of the x rows
// (staged once in LDS as float, rows m >= M and rows past K as zeros) and its
// RPW scales (one 16-byte load per lane); one barrier (no memory wait) puts
// all of these ahead of any weight request; then each wave requests its
// whole P-deep weight prefetch.  It waits for x and the scales only, stages
// them, passes a second barrier that leaves the weight loads in flight, and
// computes step by step as the weights arrive.
//
// Range.  x is staged as x * 2^ex with ex chosen per (row m, row group) so
// that the group's largest |x| lies in [1, 2), and each wave's scales as
// s * 2^es with its largest scale in [2^13, 2^14).  Every product x*s then
// lies below 2^15, inside the f16 range, for inputs of any magnitude; the
// epilogue multiplies by 2^-(ex + es).
//
// Per 32-row step a wave runs v_mfma_f32_16x16x32_f16 on
//   A[m][k] = x[m,k] * s[k,nb]          split as f16 hi + f16 lo (22 bits)
//   B[k][c] = f16 denormal (code+8) * 2^-24 (even column: low nibble in bits
//             0-3) or (code+8) * 2^-20 (odd column: high nibble in bits 4-7)
// over 8 tiles of 16 columns.  Lane (j = lane&15, g = lane>>4) loads the u32
// holding columns 8j..8j+7 of rows 8g..8g+7; tile t takes nibble t of each,
// so tile t covers columns {8j + t}.  Per row one v_bitop3 isolates the low
// nibbles (and flips the code's sign bit, giving code+8), one the high
// nibbles; one v_perm_b32 then builds a B dword from two rows.  The +8 offset
// is removed with a correction tile D_corr (B = 8 * 2^-20):
//   odd tiles  y = 2^20 * (D - D_corr),  even tiles  y = 2^24 * (D - D_corr / 16).
//
// Reductions are deterministic.  The waves' 16 x 128 partials meet in LDS
// (reusing the x rows once every wave has left the loop) and every thread
// sums its float4s over the row groups in order.  Workgroups that split K
// write their partials with write-through (sc1) stores, then count arrivals
// on a 64-bit counter per column group holding one 8-bit count per XCC (the
// XCC_ID hardware register).  The last arrival sums the partials in split
// order and resets the counter.  When every split ran on its own XCC, which
// shares one L2, it reads the partials through L2 (sc0); otherwise past it
// (sc1).  When the column groups divide evenly over the 8 XCDs (workgroup b
// runs on XCD b % 8), all splits of a column group are placed on one XCD;
// the protocol does not depend on it.
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

#define DEC_WAVES 16
#define DEC_THREADS (64 * DEC_WAVES)
#define DEC_COUNTER_BYTES 65536  // split-K counters: 8192 column groups of 8 bytes
#define DEC_XPAD 4               // LDS row padding of the staged x (floats)
#define DEC_RS 132               // LDS row stride of a wave partial (floats)
#define DEC_OOB 0x80000000u      // buffer offset past every range: the load returns zeros

// A = x * s as f16 hi + f16 lo: hi = RZ(x*s), lo = RZ(fma(x, s, -hi))
__device__ __forceinline__ void split_hi_lo(const f32x4& x0, const f32x4& x1, const f32x4& s0, const f32x4& s1,
                                            f16x8& hi, f16x8& lo) {
  const float xa[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
  const float sa[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
  uint32_t h[4], l[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    auto hp = __builtin_amdgcn_cvt_pkrtz(xa[2 * q] * sa[2 * q], xa[2 * q + 1] * sa[2 * q + 1]);
    const float r0 = __builtin_fmaf(xa[2 * q], sa[2 * q], -(float)hp[0]);
    const float r1 = __builtin_fmaf(xa[2 * q + 1], sa[2 * q + 1], -(float)hp[1]);
    auto lp = __builtin_amdgcn_cvt_pkrtz(r0, r1);
    h[q] = __builtin_bit_cast(uint32_t, hp);
    l[q] = __builtin_bit_cast(uint32_t, lp);
  }
  hi = __builtin_bit_cast(f16x8, u32x4v{h[0], h[1], h[2], h[3]});
  lo = __builtin_bit_cast(f16x8, u32x4v{l[0], l[1], l[2], l[3]});
}

// s_barrier without the memory fence of __syncthreads: the fence would make
// every wave wait for all of its weight loads still in flight.
__device__ __forceinline__ void dec_barrier_nofence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int STEPS, int NBW>
struct DecGeom {
  static constexpr int RPW = STEPS * 32;        // rows per wave
  static constexpr int RG = DEC_WAVES / NBW;    // row groups per workgroup
  static constexpr int R = RG * RPW;            // rows per workgroup
  static constexpr int XS = R + DEC_XPAD;       // LDS row stride of the staged x
  static constexpr int LX = 16 * XS > DEC_WAVES * 16 * DEC_RS ? 16 * XS : DEC_WAVES * 16 * DEC_RS;
  // reduction: TPB threads per block, CPT (a multiple of 4) outputs each
  static constexpr int TPB = DEC_THREADS / NBW > 512 ? 512 : DEC_THREADS / NBW;
  static constexpr int RT = TPB * NBW;          // threads taking part in the reduction
  static constexpr int CPT = 2048 / TPB;
};

template <typename T, int STEPS, int NBW, int P, int BITS = 4, bool FP = false>
__global__ __launch_bounds__(DEC_THREADS, 1) void k_linear_w4_decode(
    const T* __restrict__ x, int M, int64_t K, int64_t N, const uint32_t* __restrict__ w,
    const float* __restrict__ scales_t, const float* __restrict__ bias, float* __restrict__ out,
    float* __restrict__ partials, unsigned long long* __restrict__ counters, int S, int xcd_map) {
  using G = DecGeom<STEPS, NBW>;
  constexpr int RPW = G::RPW, RG = G::RG, R = G::R, XS = G::XS, TPB = G::TPB, RT = G::RT, CPT = G::CPT;
  constexpr int EPL = 16 / (int)sizeof(T);        // x elements per 16-byte load
  constexpr int XL = 16 * R / EPL / DEC_THREADS;  // x loads per thread
  static_assert(XL * DEC_THREADS * EPL == 16 * R, "x staging must divide evenly");
  static_assert(RPW / 4 <= 64, "one 16-byte scale load per lane");
  static_assert(CPT % 4 == 0 && TPB * CPT == 2048, "reduction split");
  constexpr int XG = RPW / EPL;  // consecutive lanes whose x loads make up one (row, row group)
  static_assert(XG >= 1 && XG <= 64 && (XG & (XG - 1)) == 0 && (R / EPL) % XG == 0, "x row-group lanes");
  // x rows during the loop, then the waves' partials
  __shared__ __attribute__((aligned(16))) float sX[G::LX];
  __shared__ __attribute__((aligned(16))) float sS[DEC_WAVES * RPW];
  // power-of-two exponent each (row m, row group) of x was staged with
  __shared__ int sXe[16 * RG];
  __shared__ int s_flags;
  // the wave index goes through readfirstlane so that everything derived
  // from it (row ranges, scalar buffer offsets) is known to be wave-uniform
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int nbl = wave % NBW, rg = wave / NBW;
  const int64_t NB = N / 128;
  int64_t cg;
  int ks;
  if (xcd_map) {
    const int i = (int)(blockIdx.x >> 3);
    cg = (int64_t)(i / S) * 8 + (blockIdx.x & 7);
    ks = i % S;
  } else {
    cg = blockIdx.x / S;
    ks = blockIdx.x % S;
  }
  const int64_t nb = cg * NBW + nbl;
  const int64_t k0w = (int64_t)ks * R;                 // first row of the workgroup
  const int kv = (int)(K - k0w < R ? K - k0w : R);     // its rows inside K (a multiple of 32)
  const int64_t kw = k0w + (int64_t)rg * RPW;          // this wave's first row

  // ---- requests in arrival order: x rows and scales of every wave, then
  // the whole weight prefetch
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)((int64_t)M * K * sizeof(T)));
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(scales_t, (uint32_t)(K * NB * 4));
  u32x4 xst[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int e = threadIdx.x + DEC_THREADS * i;
    const int m = e / (R / EPL), c = e % (R / EPL);
    const bool ok = m < M && c * EPL < kv;
    xst[i] = buf_load_b128(rx, ok ? (uint32_t)(((int64_t)m * K + k0w + (int64_t)c * EPL) * sizeof(T)) : DEC_OOB, 0u);
  }
  const int64_t r4 = kw + 4 * lane;  // K % 4 == 0: a 16-byte group is wholly in or out
  const u32x4 sst = buf_load_b128_nt(rs, (lane < RPW / 4 && r4 < K) ? (uint32_t)((nb * K + r4) * 4) : DEC_OOB, 0u);
  // every wave's x and scale requests are issued before any wave's weight
  // requests: the CU returns data in request order, so x arrives first while
  // the weight stream is already queued behind it
  __builtin_amdgcn_sched_barrier(0);

  // ---- weight prefetch, P steps deep over a fully unrolled step sequence:
  // step st computes from slot st % P, then the slot is refilled with step
  // st + P.  Buffer loads carry one per-lane offset (lane's k-group and
  // column word) and the step's row in the scalar offset.  The hardware
  // range check does not cover the scalar offset, so every address is kept
  // valid by construction: a step past K (only in the last split when K is
  // not a multiple of R) re-reads rows 0..31, and its x rows and scales are
  // zeros.
  // BITS = 8 (int8 or FP8 codes, exact f16 operands with no offset): 8
  // bytes of a row per lane, words 2r and 2r + 1 of row r; the prefetch is
  // P steps deep as for 4-bit codes (the caller halves P).  int4 codes go
  // in as (c + 8) at bits 0-3 or 4-7 of an f16 half, a denormal, the offset
  // taken back by one correction MFMA.  FP: sorted-grid float codes (FP4 E2M1, FP8 E4M3),
  // whose B operands are the format's values v * 2^-E exactly (E = 14 or 8,
  // no offset), and the epilogue takes 2^E * RN(1 / vmax).
  // BITS = 2 (int2 codes): 16 bits of a row per lane, as (c + 2) at bits
  // 0-1 of an f16 half with the int4 correction scaled by 2/128.
  // BITS = 1 (int1 codes, 0 is +1 and 1 is -1): one byte of a row per lane,
  // the code the sign bit of the f16 1.0 (exact, no correction).
  static_assert(BITS == 1 || BITS == 2 || BITS == 4 || BITS == 8, "1-, 2-, 4- or 8-bit codes");
  static_assert(!FP || BITS >= 4, "no 1- or 2-bit float grid");
  constexpr int WPR = BITS == 8 ? 2 : 1;  // 32-bit words of a lane's 8 columns in one row (int2: 16 bits)
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)(K * N * BITS / 8));
  const uint32_t row_bytes = (uint32_t)(N * BITS / 8);
  const uint32_t vw = (uint32_t)(8 * g * row_bytes + (nb * 16 + j) * BITS);  // a lane's 8 columns: BITS bytes
  uint32_t wv[P][8 * WPR];
  auto issue = [&](int slot, int st) {
    const int64_t k0 = kw + (int64_t)st * 32;
    const uint32_t kr = k0 < K ? (uint32_t)k0 : 0u;  // wave-uniform
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      if constexpr (BITS == 1) {
        wv[slot][r] = buf_load_b8_nt(rw, vw, (kr + r) * row_bytes);
      } else if constexpr (BITS == 2) {
        wv[slot][r] = buf_load_b16_nt(rw, vw, (kr + r) * row_bytes);
      } else if constexpr (BITS == 4) {
        wv[slot][r] = buf_load_b32_nt(rw, vw, (kr + r) * row_bytes);
      } else {
        const uint2 v = buf_load_b64_nt(rw, vw, (kr + r) * row_bytes);
        wv[slot][2 * r] = v.x;
        wv[slot][2 * r + 1] = v.y;
      }
    }
  };
  issue(0, 0);
  // keep the loads where they are written (the scheduler would otherwise
  // sink them next to their first use)
  __builtin_amdgcn_sched_barrier(0);

  // ---- range: the MFMA operand A = x*s is an f16 pair (hi + lo), so x and
  // the scales are brought to fixed binades by powers of two first (exact),
  // and the powers return in the epilogue.  x: each (row m, row group) is
  // scaled so that its largest |x| lies in [1, 2); its XG loads sit in XG
  // consecutive lanes.  Scales: each wave's largest scale goes to
  // [2^13, 2^14).  Every product then lies below 2^15, within the f16 range,
  // and a product 2^k below its row group's largest one keeps full
  // precision down to k = 28 (f16 normals for hi, then lo).
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int e = threadIdx.x + DEC_THREADS * i;
    const int m = e / (R / EPL), c = e % (R / EPL);
    float v[EPL];
    if constexpr (EPL == 4) {
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = __uint_as_float(xst[i][u]);
    } else {
      const T* tt = reinterpret_cast<const T*>(&xst[i]);
#pragma unroll
      for (int u = 0; u < EPL; ++u) v[u] = ElemT<T>::cvt(tt[u]);
    }
    float mx = 0.0f;
#pragma unroll
    for (int u = 0; u < EPL; ++u) mx = fmaxf(mx, __builtin_fabsf(v[u]));
    mx = group_max<XG>(mx);
    const int be = (int)((__float_as_uint(mx) >> 23) & 0xFFu);
    const int xe = be == 0xFF ? 0 : 127 - (be == 0 ? 1 : be);  // zero rows: any shift
#pragma unroll
    for (int u = 0; u < EPL; ++u) v[u] = __builtin_ldexpf(v[u], xe);
    float* dst = sX + m * XS + c * EPL;
#pragma unroll
    for (int u = 0; u < EPL; u += 4) *reinterpret_cast<f32x4*>(dst + u) = f32x4{v[u], v[u + 1], v[u + 2], v[u + 3]};
    if ((lane & (XG - 1)) == 0) sXe[m * RG + (c * EPL) / RPW] = xe;
  }
  float sv[4];
  float smx = 0.0f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    sv[u] = __uint_as_float(sst[u]);
    smx = fmaxf(smx, __builtin_fabsf(sv[u]));
  }
  smx = group_max<64>(smx);
  const int sbe = (int)((__float_as_uint(smx) >> 23) & 0xFFu);
  const int se = sbe == 0xFF ? 0 : 140 - (sbe == 0 ? 1 : sbe);  // largest scale to [2^13, 2^14)
  float* wS = sS + wave * RPW;
  if (lane < RPW / 4)
    *reinterpret_cast<f32x4*>(wS + 4 * lane) = f32x4{__builtin_ldexpf(sv[0], se), __builtin_ldexpf(sv[1], se),
                                                     __builtin_ldexpf(sv[2], se), __builtin_ldexpf(sv[3], se)};
  // LDS writes done, then a barrier that leaves the weight loads in flight
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt untouched
  dec_barrier_nofence();
#pragma unroll
  for (int q = 1; q < P && q < STEPS; ++q) issue(q, q);
  __builtin_amdgcn_sched_barrier(0);

  f32x4 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 corr = f32x4{0.f, 0.f, 0.f, 0.f};
  const f16x8 b8 = __builtin_bit_cast(f16x8, u32x4v{0x00800080u, 0x00800080u, 0x00800080u, 0x00800080u});
  const float* xrow = sX + j * XS + rg * RPW + 8 * g;
  const float* srow = wS + 8 * g;
#pragma unroll
  for (int st = 0; st < STEPS; ++st) {
    const int q = st % P;
    const f32x4 x0 = *reinterpret_cast<const f32x4*>(xrow + st * 32);
    const f32x4 x1 = *reinterpret_cast<const f32x4*>(xrow + st * 32 + 4);
    const f32x4 s0 = *reinterpret_cast<const f32x4*>(srow + st * 32);
    const f32x4 s1 = *reinterpret_cast<const f32x4*>(srow + st * 32 + 4);
    f16x8 ahi, alo;
    split_hi_lo(x0, x1, s0, s1, ahi, alo);
    // int4: lo4 / hi4 hold the low / high nibbles of each row word xor 8
    // (c + 8, at bits 0-3 / 4-7 of a byte); int8: the row words themselves
    uint32_t lo4[8 * WPR], hi4[BITS == 4 && !FP ? 8 : 1];
#pragma unroll
    for (int r = 0; r < 8 * WPR; ++r) {
      if constexpr (BITS == 4 && !FP) {
        lo4[r] = (wv[q][r] & 0x0F0F0F0Fu) ^ 0x08080808u;
        hi4[r] = (wv[q][r] & 0xF0F0F0F0u) ^ 0x80808080u;
      } else if constexpr (BITS <= 2) {
        // rows 2h and 2h + 1 side by side (odd r: the upper half)
        lo4[r] = (r & 1) ? wv[q][r] << 16 : wv[q][r];
      } else {
        lo4[r] = wv[q][r];
      }
    }
    if (st + P < STEPS) issue(q, st + P);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      // int4: byte t / 2 of rows 2h and 2h + 1; int8: byte t % 4 of word t / 4
      const uint32_t p = BITS == 4 ? (uint32_t)(t >> 1) : (uint32_t)(t & 3);
      const uint32_t sel = 0x0C000C00u | ((4u + p) << 16) | p;
      uint32_t bq[4];
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        if constexpr (FP && BITS == 4) {
          // byte t / 2 of rows 2h, 2h + 1 at bytes 0 and 2; odd tiles the high nibbles
          const uint32_t d = __builtin_amdgcn_perm(lo4[2 * h + 1], lo4[2 * h], sel);
          bq[h] = fp_code_pair_f16<4>((t & 1) ? d >> 4 : d);
        } else if constexpr (FP) {
          // byte t % 4 of word t / 4 of rows 2h, 2h + 1 at bytes 1 and 3
          const int wd = t >> 2;
          const uint32_t selh = 0x0Cu | (p << 8) | 0x0C0000u | ((4u + p) << 24);
          bq[h] = fp_code_pair_f16<8>(__builtin_amdgcn_perm(lo4[2 * (2 * h + 1) + wd], lo4[2 * (2 * h) + wd], selh));
        } else if constexpr (BITS == 1) {
          // column 8j + t at bit t of each row's byte: the sign of +-1.0
          bq[h] = ((((lo4[2 * h] | lo4[2 * h + 1]) >> t) & 0x00010001u) << 15) | 0x3C003C00u;
        } else if constexpr (BITS == 2) {
          // column 8j + t at bits 2t of each row's 16 bits: c ^ 2 = c + 2, the denormal (c + 2) * 2^-24
          bq[h] = (((lo4[2 * h] | lo4[2 * h + 1]) >> (2 * t)) & 0x00030003u) ^ 0x00020002u;
        } else if constexpr (BITS == 4) {
          const uint32_t a0 = (t & 1) ? hi4[2 * h] : lo4[2 * h];
          const uint32_t a1 = (t & 1) ? hi4[2 * h + 1] : lo4[2 * h + 1];
          bq[h] = __builtin_amdgcn_perm(a1, a0, sel);
        } else {
          // 0x6400 | (c ^ 0x80) is the f16 1024 + (c + 128): less 1152, c
          // itself, exact (an offset taken back after the sum, as for int4,
          // would leave each sum's rounding relative to 128 * A, not c * A)
          const int wd = t >> 2;
          const uint32_t e =
              __builtin_amdgcn_perm(lo4[2 * (2 * h + 1) + wd], lo4[2 * (2 * h) + wd], sel) ^ 0x64806480u;
          const f16x2v r = __builtin_bit_cast(f16x2v, e) - f16x2v{(_Float16)1152.0f, (_Float16)1152.0f};
          bq[h] = __builtin_bit_cast(uint32_t, r);
        }
      }
      const f16x8 bt = __builtin_bit_cast(f16x8, u32x4v{bq[0], bq[1], bq[2], bq[3]});
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bt, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bt, acc[t], 0, 0, 0);
    }
    if constexpr (!FP && (BITS == 2 || BITS == 4)) {
      corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, b8, corr, 0, 0, 0);
      corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, b8, corr, 0, 0, 0);
    }
  }

  // ---- wave partial (rows 4g+i, columns 8j+t of block nb) to LDS, after
  // every wave has finished reading the x rows it overwrites
  __syncthreads();
  float* red = sX;
  float* rwv = red + wave * 16 * DEC_RS;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // undo the code placement (2^24 even, 2^20 odd) and the range scaling of
    // x row 4g+i and of this wave's scales
    const int sh = -sXe[(4 * g + i) * RG + rg] - se;
    float v[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      if constexpr (FP)  // v * 2^-E for the grid value RN(v / vmax)
        v[t] = __builtin_ldexpf(acc[t][i], (BITS == 4 ? 14 : 8) + sh) * (BITS == 4 ? 1.0f / 6.0f : 1.0f / 480.0f);
      else if constexpr (BITS == 8 || BITS == 1)  // exact codes
        v[t] = __builtin_ldexpf(acc[t][i], sh);
      else if constexpr (BITS == 2)  // (c + 2) * 2^-24, corr the sum of 128 * 2^-24 terms
        v[t] = __builtin_ldexpf(acc[t][i] - corr[i] * 0.015625f, 24 + sh);
      else
        v[t] = (t & 1) ? __builtin_ldexpf(acc[t][i] - corr[i], 20 + sh)
                       : __builtin_ldexpf(acc[t][i] - corr[i] * 0.0625f, 24 + sh);
    }
    float* dst = rwv + (4 * g + i) * DEC_RS + 8 * j;
    *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(dst + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
  __syncthreads();
  // thread (< RT): block b of the group, row m, columns c .. c+CPT-1,
  // summed over the row groups in order
  const bool rt = threadIdx.x < RT;
  const int b = rt ? threadIdx.x / TPB : 0, r = threadIdx.x % TPB;
  const int m = r / (128 / CPT), c = CPT * (r % (128 / CPT));
  f32x4 sum[CPT / 4];
#pragma unroll
  for (int h = 0; h < CPT / 4; ++h) {
    sum[h] = *reinterpret_cast<const f32x4*>(red + (b * 16 + m) * DEC_RS + c + 4 * h);
#pragma unroll
    for (int q = 1; q < RG; ++q)
      sum[h] += *reinterpret_cast<const f32x4*>(red + ((q * NBW + b) * 16 + m) * DEC_RS + c + 4 * h);
  }
  const int64_t nbb = cg * NBW + b;
  const int64_t col = nbb * 128 + c;
  if (S == 1) {
    if (rt && m < M) {
#pragma unroll
      for (int h = 0; h < CPT / 4; ++h) {
        f32x4 o = sum[h];
        if (bias) o += *reinterpret_cast<const f32x4*>(bias + col + 4 * h);
        *reinterpret_cast<f32x4*>(out + (int64_t)m * N + col + 4 * h) = o;
      }
    }
    return;
  }
  // partials: [S][N/128][16 rows][128 columns] floats, written through to
  // memory before the workgroup is counted
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(partials, (uint32_t)((int64_t)S * NB * 16 * 128 * 4));
  const uint32_t poff = (uint32_t)(((nbb * 16 + m) * 128 + c) * 4);
  const uint32_t split_stride = (uint32_t)(NB * 16 * 128 * 4);
  if (rt) {
#pragma unroll
    for (int h = 0; h < CPT / 4; ++h)
      __builtin_amdgcn_raw_buffer_store_b128(sum[h], rp, poff + 16u * h, (uint32_t)ks * split_stride, 16);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    xcc &= 7u;
    const unsigned long long inc = 1ull << (8 * xcc);
    const unsigned long long now =
        __hip_atomic_fetch_add(&counters[cg], inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + inc;
    unsigned total = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) total += (unsigned)((now >> (8 * q)) & 0xFFull);
    const bool same = ((now >> (8 * xcc)) & 0xFFull) == (unsigned long long)S;
    const bool last = total == (unsigned)S;
    // no split of this call touches the counter again: reset it now, so
    // that the reset's round trip overlaps the reads below
    if (last) __hip_atomic_store(&counters[cg], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_flags = (last ? 1 : 0) | (same ? 2 : 0);
  }
  __syncthreads();
  const int fl = s_flags;
  if (!(fl & 1) || !rt) return;
  // last arrival: sum the S partials in split order (its own from registers)
  f32x4 tot[CPT / 4];
  for (int sb = 0; sb < S; sb += 8) {
    f32x4 part[8][CPT / 4];
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int h = 0; h < CPT / 4; ++h) {
        const bool ld = sb + u < S && sb + u != ks;
        const uint32_t soff = ld ? (uint32_t)(sb + u) * split_stride : 0u;
        if (!ld)
          part[u][h] = sum[h];
        else if (fl & 2)
          part[u][h] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, poff + 16u * h, soff, 1));
        else
          part[u][h] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, poff + 16u * h, soff, 16));
      }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (sb + u < S)
#pragma unroll
        for (int h = 0; h < CPT / 4; ++h) tot[h] = (sb + u == 0) ? part[u][h] : tot[h] + part[u][h];
  }
  if (m < M) {
#pragma unroll
    for (int h = 0; h < CPT / 4; ++h) {
      f32x4 o = tot[h];
      if (bias) o += *reinterpret_cast<const f32x4*>(bias + col + 4 * h);
      *reinterpret_cast<f32x4*>(out + (int64_t)m * N + col + 4 * h) = o;
    }
  }
}

// ---------------------------------------------------------------- int4 decode, tiled weight copy
// The same product as k_linear_w4_decode, y[m, n] = sum_k x[m,k] *
// RN(code[k,n] * s[k, n/128]), read from a tiled copy of the weight
// (mxk_linear_prepack_weight) laid out so that every 16-byte load of a wave
// is contiguous and every MFMA B operand comes out of the loaded words with
// one v_bitop3 (no byte permutes):
//   chunk (block nb, 32-row step ks): 2048 bytes at (nb * K/32 + ks) * 2048;
//   lane l = j + 16 g reads 16 bytes at +16 l (words 0..3) and +1024 + 16 l
//   (words 4..7).  Word 2p + e holds the byte of columns 8j + 2p, 8j + 2p + 1
//   (low nibble = even column) of rows 8g + 4e + {0, 2, 1, 3} in its bytes
//   0..3.  So (w & 0x000F000F) is the f16 pair of rows 8g+4e, +1 of column
//   8j + 2p as denormals code * 2^-24, (w >> 8) & 0x000F000F the pair of
//   rows +2, +3, and the masks 0x00F000F0 give column 8j + 2p + 1 as
//   code * 2^-20; xor with 8 per nibble turns the two's complement code into
//   code + 8, removed by the correction tile as in k_linear_w4_decode.
//
// Work split: one 128-column block per workgroup (the tiled rows are whole
// lines at any width), W waves of RPW = 32 * STEPS rows each, so K splits
// S = ceil(K / (W * RPW)) ways.  Long waves (8 waves of 8 steps, two per
// SIMD) cost less than 16 waves of 4 steps over the same rows: each wave's
// fixed work (scale range, epilogue, its partial in the LDS reduction) is
// paid half as often.  Each wave reads its own x rows
// row-contiguously (one load covering 16 rows 32 KiB apart would put every
// request on one memory channel), turns them into the A-fragment order
// through its own LDS slot (no workgroup barrier), scales them per row into
// [1, 2), and only then requests its weights, so that x is not queued behind
// the weight stream.  The partial reduction and the split-K hand-off are
// those of k_linear_w4_decode.
// FP: FP4 E2M1 sorted-grid codes instead of int4 (B operands v * 2^-14,
// exact, no offset; the epilogue takes 2^14 * RN(1/6))
template <typename T, int STEPS, int W, bool FP = false>
__global__ __launch_bounds__(W * 64, 1) void k_linear_w4_decode_tiled(
    const T* __restrict__ x, int M, int64_t K, int64_t N, const uint32_t* __restrict__ wt,
    const float* __restrict__ scales_t, const float* __restrict__ bias, float* __restrict__ out,
    float* __restrict__ partials, unsigned long long* __restrict__ counters, int S, int xcd_map) {
  constexpr int RPW = 32 * STEPS, R = W * RPW;
  constexpr int TPB = W * 64 > 512 ? 512 : W * 64, RT = TPB, CPT = 2048 / TPB;
  constexpr int XS = (RPW > 128 ? RPW : 128) + 4;  // row stride of a wave's LDS slot (floats)
  constexpr int EPL = 16 / (int)sizeof(T);   // x elements per 16-byte load
  constexpr int LPR = RPW / EPL;             // lanes per x row in one load
  constexpr int RPL = 64 / LPR;              // x rows per load
  constexpr int XLD = 16 / RPL;              // x loads per lane
  static_assert(LPR >= 1 && RPL * LPR == 64 && XLD * RPL == 16, "x loads");
  static_assert(RPW / 4 <= 64 && XS >= DEC_RS, "scales and x rows of a wave");
  static_assert(CPT % 4 == 0 && TPB * CPT == 2048, "reduction split");
  // each wave's slot of 16 rows of XS floats holds its x rows, then its partial
  __shared__ __attribute__((aligned(16))) float sR[W * 16 * XS];
  __shared__ __attribute__((aligned(16))) float sS[W * RPW];
  __shared__ int sXe[W * 16];
  __shared__ int s_flags;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int64_t NB = N / 128;
  int64_t nb;
  int ks;
  if (xcd_map) {
    const int i = (int)(blockIdx.x >> 3);
    nb = (int64_t)(i / S) * 8 + (blockIdx.x & 7);
    ks = i % S;
  } else {
    nb = blockIdx.x / S;
    ks = blockIdx.x % S;
  }
  const int64_t kw = (int64_t)ks * R + (int64_t)wave * RPW;  // this wave's first row

  // ---- x rows and scales of this wave
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)((int64_t)M * K * sizeof(T)));
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(scales_t, (uint32_t)(K * NB * 4));
  u32x4 xr[XLD];
#pragma unroll
  for (int q = 0; q < XLD; ++q) {
    const int m = q * RPL + lane / LPR;
    const int64_t kk = kw + (int64_t)EPL * (lane % LPR);
    const bool ok = m < M && kk < K;  // K % 32 == 0: a load is wholly in or out
    xr[q] = buf_load_b128(rx, ok ? (uint32_t)(((int64_t)m * K + kk) * sizeof(T)) : DEC_OOB, 0u);
  }
  const int64_t r4 = kw + 4 * lane;
  const u32x4 sst = buf_load_b128_nt(rs, (lane < RPW / 4 && r4 < K) ? (uint32_t)((nb * K + r4) * 4) : DEC_OOB, 0u);
  __builtin_amdgcn_sched_barrier(0);

  // ---- x into the A-fragment order (lane (j, g): row j, columns
  // 32 st + 8 g .. +7) through the wave's slot; LDS runs a wave's accesses in
  // order, so only the compiler needs holding back.  Range as in
  // k_linear_w4_decode: row j's largest |x| in this wave to [1, 2), the
  // wave's largest scale to [2^13, 2^14).
  float* xs = sR + wave * 16 * XS;
#pragma unroll
  for (int q = 0; q < XLD; ++q) {
    const int m = q * RPL + lane / LPR;
    const int c = EPL * (lane % LPR);
    float v[EPL];
    if constexpr (EPL == 4) {
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = __uint_as_float(xr[q][u]);
    } else {
      const T* tt = reinterpret_cast<const T*>(&xr[q]);
#pragma unroll
      for (int u = 0; u < EPL; ++u) v[u] = ElemT<T>::cvt(tt[u]);
    }
#pragma unroll
    for (int u = 0; u < EPL; u += 4)
      *reinterpret_cast<f32x4*>(xs + m * XS + c + u) = f32x4{v[u], v[u + 1], v[u + 2], v[u + 3]};
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float xv[STEPS * 8];
#pragma unroll
  for (int st = 0; st < STEPS; ++st)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(xs + j * XS + 32 * st + 8 * g + 4 * h);
#pragma unroll
      for (int u = 0; u < 4; ++u) xv[8 * st + 4 * h + u] = t[u];
    }
  float mx = 0.0f;
#pragma unroll
  for (int u = 0; u < STEPS * 8; ++u) mx = fmaxf(mx, __builtin_fabsf(xv[u]));
  // row j sits in lanes j, j + 16, j + 32, j + 48
  mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(mx), 0x401F)));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const int be = (int)((__float_as_uint(mx) >> 23) & 0xFFu);
  const int xe = be == 0xFF ? 0 : 127 - (be == 0 ? 1 : be);  // zero rows: any shift
#pragma unroll
  for (int u = 0; u < STEPS * 8; ++u) xv[u] = __builtin_ldexpf(xv[u], xe);
  if (g == 0) sXe[wave * 16 + j] = xe;
  float sv[4];
  float smx = 0.0f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    sv[u] = __uint_as_float(sst[u]);
    smx = fmaxf(smx, __builtin_fabsf(sv[u]));
  }
  smx = group_max<64>(smx);
  const int sbe = (int)((__float_as_uint(smx) >> 23) & 0xFFu);
  const int se = sbe == 0xFF ? 0 : 140 - (sbe == 0 ? 1 : sbe);  // largest scale to [2^13, 2^14)
  float* wS = sS + wave * RPW;
  if (lane < RPW / 4)
    *reinterpret_cast<f32x4*>(wS + 4 * lane) = f32x4{__builtin_ldexpf(sv[0], se), __builtin_ldexpf(sv[1], se),
                                                     __builtin_ldexpf(sv[2], se), __builtin_ldexpf(sv[3], se)};
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- weights of every step, requested once this wave's x is in.  A step
  // past K (only in the last split) re-reads chunk 0 of the block; its x rows
  // and scales are zeros.
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(wt, (uint32_t)(K * N / 2));
  u32x4 wq[STEPS][2];
#pragma unroll
  for (int st = 0; st < STEPS; ++st) {
    const int64_t k0 = kw + (int64_t)st * 32;
    const uint32_t kr = k0 < K ? (uint32_t)k0 : 0u;  // wave-uniform
    const uint32_t cbase = (uint32_t)((nb * (K / 32) + kr / 32) * 2048);
    wq[st][0] = buf_load_b128_nt(rw, 16u * lane, cbase);
    wq[st][1] = buf_load_b128_nt(rw, 16u * lane, cbase + 1024u);
  }
  __builtin_amdgcn_sched_barrier(0);

  f32x4 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 corr = f32x4{0.f, 0.f, 0.f, 0.f};
  const f16x8 b8 = __builtin_bit_cast(f16x8, u32x4v{0x00800080u, 0x00800080u, 0x00800080u, 0x00800080u});
  const float* srow = wS + 8 * g;
#pragma unroll
  for (int st = 0; st < STEPS; ++st) {
    const f32x4 x0 = f32x4{xv[8 * st], xv[8 * st + 1], xv[8 * st + 2], xv[8 * st + 3]};
    const f32x4 x1 = f32x4{xv[8 * st + 4], xv[8 * st + 5], xv[8 * st + 6], xv[8 * st + 7]};
    const f32x4 s0 = *reinterpret_cast<const f32x4*>(srow + st * 32);
    const f32x4 s1 = *reinterpret_cast<const f32x4*>(srow + st * 32 + 4);
    f16x8 ahi, alo;
    split_hi_lo(x0, x1, s0, s1, ahi, alo);
    uint32_t wr[8], w8[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      wr[r] = r < 4 ? wq[st][0][r] : wq[st][1][r - 4];
      w8[r] = wr[r] >> 8;
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      // tile t: column 8j + t; even tiles the low nibbles (code * 2^-24),
      // odd tiles the high nibbles (code * 2^-20)
      const int p = t >> 1;
      u32x4v bq;
      if constexpr (FP) {
        const int sh = 4 * (t & 1);
        bq = u32x4v{fp_code_pair_f16<4>(wr[2 * p] >> sh), fp_code_pair_f16<4>(w8[2 * p] >> sh),
                    fp_code_pair_f16<4>(wr[2 * p + 1] >> sh), fp_code_pair_f16<4>(w8[2 * p + 1] >> sh)};
      } else {
        const uint32_t msk = (t & 1) ? 0x00F000F0u : 0x000F000Fu;
        const uint32_t off8 = (t & 1) ? 0x00800080u : 0x00080008u;
        bq = u32x4v{(wr[2 * p] & msk) ^ off8, (w8[2 * p] & msk) ^ off8, (wr[2 * p + 1] & msk) ^ off8,
                    (w8[2 * p + 1] & msk) ^ off8};
      }
      const f16x8 bt = __builtin_bit_cast(f16x8, bq);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bt, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bt, acc[t], 0, 0, 0);
    }
    if constexpr (!FP) {
      corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, b8, corr, 0, 0, 0);
      corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, b8, corr, 0, 0, 0);
    }
  }

  // ---- wave partial (rows 4g+i, columns 8j+t) into its own slot: no
  // barrier first, nothing else uses the slot
  float* rwv = sR + wave * 16 * XS;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int sh = -sXe[wave * 16 + 4 * g + i] - se;
    float v[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      if constexpr (FP)
        v[t] = __builtin_ldexpf(acc[t][i], 14 + sh) * (1.0f / 6.0f);
      else
        v[t] = (t & 1) ? __builtin_ldexpf(acc[t][i] - corr[i], 20 + sh)
                       : __builtin_ldexpf(acc[t][i] - corr[i] * 0.0625f, 24 + sh);
    }
    float* dst = rwv + (4 * g + i) * XS + 8 * j;
    *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(dst + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
  __syncthreads();
  // thread (< RT): row m, columns c .. c+CPT-1, summed over the waves in order
  const bool rt = threadIdx.x < RT;
  const int r = threadIdx.x % TPB;
  const int m = r / (128 / CPT), c = CPT * (r % (128 / CPT));
  f32x4 sum[CPT / 4];
#pragma unroll
  for (int h = 0; h < CPT / 4; ++h) {
    sum[h] = *reinterpret_cast<const f32x4*>(sR + m * XS + c + 4 * h);
#pragma unroll
    for (int q = 1; q < W; ++q) sum[h] += *reinterpret_cast<const f32x4*>(sR + (q * 16 + m) * XS + c + 4 * h);
  }
  const int64_t col = nb * 128 + c;
  if (S == 1) {
    if (rt && m < M) {
#pragma unroll
      for (int h = 0; h < CPT / 4; ++h) {
        f32x4 o = sum[h];
        if (bias) o += *reinterpret_cast<const f32x4*>(bias + col + 4 * h);
        *reinterpret_cast<f32x4*>(out + (int64_t)m * N + col + 4 * h) = o;
      }
    }
    return;
  }
  // split-K hand-off as in k_linear_w4_decode: partials [S][N/128][16][128]
  // written through, arrivals counted per XCC, the last arrival sums in
  // split order
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(partials, (uint32_t)((int64_t)S * NB * 16 * 128 * 4));
  const uint32_t poff = (uint32_t)(((nb * 16 + m) * 128 + c) * 4);
  const uint32_t split_stride = (uint32_t)(NB * 16 * 128 * 4);
  if (rt) {
#pragma unroll
    for (int h = 0; h < CPT / 4; ++h)
      __builtin_amdgcn_raw_buffer_store_b128(sum[h], rp, poff + 16u * h, (uint32_t)ks * split_stride, 16);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    xcc &= 7u;
    const unsigned long long inc = 1ull << (8 * xcc);
    const unsigned long long now =
        __hip_atomic_fetch_add(&counters[nb], inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + inc;
    unsigned total = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) total += (unsigned)((now >> (8 * q)) & 0xFFull);
    const bool same = ((now >> (8 * xcc)) & 0xFFull) == (unsigned long long)S;
    const bool last = total == (unsigned)S;
    if (last) __hip_atomic_store(&counters[nb], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_flags = (last ? 1 : 0) | (same ? 2 : 0);
  }
  __syncthreads();
  const int fl = s_flags;
  if (!(fl & 1) || !rt) return;
  f32x4 tot[CPT / 4];
  for (int sb = 0; sb < S; sb += 8) {
    f32x4 part[8][CPT / 4];
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int h = 0; h < CPT / 4; ++h) {
        const bool ld = sb + u < S && sb + u != ks;
        const uint32_t soff = ld ? (uint32_t)(sb + u) * split_stride : 0u;
        if (!ld)
          part[u][h] = sum[h];
        else if (fl & 2)
          part[u][h] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, poff + 16u * h, soff, 1));
        else
          part[u][h] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, poff + 16u * h, soff, 16));
      }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (sb + u < S)
#pragma unroll
        for (int h = 0; h < CPT / 4; ++h) tot[h] = (sb + u == 0) ? part[u][h] : tot[h] + part[u][h];
  }
  if (m < M) {
#pragma unroll
    for (int h = 0; h < CPT / 4; ++h) {
      f32x4 o = tot[h];
      if (bias) o += *reinterpret_cast<const f32x4*>(bias + col + 4 * h);
      *reinterpret_cast<f32x4*>(out + (int64_t)m * N + col + 4 * h) = o;
    }
  }
}

// The tiled copy of an int4 [K][N] weight (layout above): thread (block nb,
// 32-row step ks, lane j + 16 g) reads the 4-byte word of columns 8j..8j+7
// from rows 8g..8g+7 and writes its 32 bytes of the chunk.
__global__ __launch_bounds__(256) void k_tile_w4(const uint32_t* __restrict__ w, int64_t K, int64_t N,
                                                 uint32_t* __restrict__ wt) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t steps = K / 32, NB = N / 128;
  if (tid >= NB * steps * 64) return;
  const int lane = (int)(tid & 63);
  const int64_t chunk = tid >> 6;  // nb * steps + ks
  const int64_t nb = chunk / steps, ks = chunk % steps;
  const int j = lane & 15, g = lane >> 4;
  const int64_t words = N / 8;  // 4-byte words per row
  uint32_t rw[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) rw[r] = w[(ks * 32 + 8 * g + r) * words + nb * 16 + j];
  uint32_t o[8];
#pragma unroll
  for (int p = 0; p < 4; ++p)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t b0 = (rw[4 * e + 0] >> (8 * p)) & 0xFFu, b1 = (rw[4 * e + 2] >> (8 * p)) & 0xFFu;
      const uint32_t b2 = (rw[4 * e + 1] >> (8 * p)) & 0xFFu, b3 = (rw[4 * e + 3] >> (8 * p)) & 0xFFu;
      o[2 * p + e] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
    }
  uint32_t* dst = wt + chunk * 512 + 4 * lane;
  *reinterpret_cast<u32x4v*>(dst) = u32x4v{o[0], o[1], o[2], o[3]};
  *reinterpret_cast<u32x4v*>(dst + 256) = u32x4v{o[4], o[5], o[6], o[7]};
}

// The inverse of k_tile_w4: thread (block nb, step ks, lane j + 16 g) reads
// its 32 bytes of the chunk and writes the 4-byte words of columns
// 8j..8j+7 of rows 8g..8g+7 (byte q of word 2p + e is row 4e + {0,2,1,3}[q],
// a permutation that is its own inverse).
__global__ __launch_bounds__(256) void k_untile_w4(const uint32_t* __restrict__ wt, int64_t K, int64_t N,
                                                   uint32_t* __restrict__ w) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t steps = K / 32, NB = N / 128;
  if (tid >= NB * steps * 64) return;
  const int lane = (int)(tid & 63);
  const int64_t chunk = tid >> 6;
  const int64_t nb = chunk / steps, ks = chunk % steps;
  const int j = lane & 15, g = lane >> 4;
  const uint32_t* src = wt + chunk * 512 + 4 * lane;
  const u32x4v lo = *reinterpret_cast<const u32x4v*>(src), hi = *reinterpret_cast<const u32x4v*>(src + 256);
  const uint32_t o[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  constexpr int inv[4] = {0, 2, 1, 3};
  const int64_t words = N / 8;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    uint32_t v = 0u;
#pragma unroll
    for (int p = 0; p < 4; ++p) v |= ((o[2 * p + (r >> 2)] >> (8 * inv[r & 3])) & 0xFFu) << (8 * p);
    w[(ks * 32 + 8 * g + r) * words + nb * 16 + j] = v;
  }
}

// sT[b][k] = s[k][b]: the reference's scales of a [K, N] weight with blocks
// of 128 along N ([K][NB] row-major) to the block-major order the decode
// kernel reads ([NB][K]).  32x32 tiles through LDS, both sides coalesced.
__global__ __launch_bounds__(256) void k_transpose_scales(const float* __restrict__ s, int64_t K, int64_t NB,
                                                          float* __restrict__ sT) {
  __shared__ float tile[32][33];
  const int64_t b0 = (int64_t)blockIdx.x * 32, k0 = (int64_t)blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int i = ty; i < 32; i += 8) {
    const int64_t k = k0 + i, b = b0 + tx;
    tile[i][tx] = (k < K && b < NB) ? s[k * NB + b] : 0.0f;
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    const int64_t b = b0 + i, k = k0 + tx;
    if (b < NB && k < K) sT[b * K + k] = tile[tx][i];
  }
}

static void launch_transpose_scales(const float* s, int64_t K, int64_t NB, float* sT, hipStream_t st) {
  const dim3 grid((unsigned)ceil_div(NB, 32), (unsigned)ceil_div(K, 32));
  hipLaunchKernelGGL(k_transpose_scales, grid, dim3(256), 0, st, s, K, NB, sT);
}

// ---------------------------------------------------------------- int4 decode, weight [N][K]
// y[m, n] = sum_k x[m,k] * RN(code[n,k] * s[n, k/128]) for a weight stored
// [N][K] with blocks of 128 along K (mx_dynamic_linear's quantize(weight),
// mxtorch.py:8916-8917; the input gradient of mx_linear / _MXLinearAutograd,
// mxtorch.py:6729-6740), M <= 16.
//
// A workgroup of 16 waves owns 256 columns (rows of W) and 8 blocks of K.
// Wave (q, h) takes block q and the 8 tiles of 16 columns of half h.  The
// scale of a block is one per column, so x needs no scaling: the workgroup
// stages x[16][1024] once in LDS as f16 hi + lo (22 significant bits), in
// the v_mfma_f32_16x16x32_f16 A layout, and every wave reads it.
//
// Lane (j = lane&15, g = lane>>4) loads the 16 bytes at byte 16g of column
// n's 64-byte block segment: codes k = 32g .. 32g+31 of the block.  MFMA
// step s takes codes 32g+8s .. 32g+8s+7 of every lane group, so the A lane
// (i, g) of step s holds x[i][32g+8s .. 32g+8s+7]: the sum over k is the
// same, taken in another order.  B holds code+8 as the f16 denormal
// (code+8)*2^-24 (nibble isolated, sign bit flipped, placed by v_perm_b32);
// a correction tile with B = 8*2^-24 removes the offset:
//   y += s * 2^24 * (D - D_corr).
// x is staged as x * 2^-e, the power of two that puts the workgroup's
// largest |x| in [2^14, 2^15); 2^e returns after the scale.
//
// Each wave runs its tiles in load order, so the MFMAs of the first tiles
// overlap the arrival of the last.  The 8 waves of a column half meet in LDS
// and sum their partials in block order.  With more than one K split the
// workgroup publishes its partial (partials[split][16][N], write-through
// stores) and counts its arrival; the last workgroup of the column group
// reads the others past the L2s, adds the S partials in split order
// (+ bias) and resets the counter.
#define NT_WAVES 16
#define NT_THREADS 1024
#define NT_COLS 256
#define NT_BLKS 8
#define NT_RED_STRIDE 260  // LDS row stride of the partial sums (floats)

template <typename T>
__global__ __launch_bounds__(NT_THREADS, 1) void k_linear_w4t_decode(
    const T* __restrict__ x, int M, int64_t K, int64_t N, const uint8_t* __restrict__ w,
    const float* __restrict__ scales, int scales_kb_major, const float* __restrict__ bias, float* __restrict__ out,
    float* __restrict__ partials, unsigned int* __restrict__ counters, int S) {
  // A staging (8 blocks x 4 steps x hi/lo x 1 KiB = 64 KiB), then the
  // partial sums [8 blocks][16 rows][256 (+4) columns]
  __shared__ __attribute__((aligned(16))) float lds[NT_BLKS * 16 * NT_RED_STRIDE];
  __shared__ float s_wmax[NT_WAVES];
  __shared__ int s_last;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int cg = (int)(blockIdx.x / S), ks = (int)(blockIdx.x % S);
  const int64_t KB = K / 128;
  const int64_t kb0 = (int64_t)ks * NT_BLKS;
  const int q = wave & 7, h = wave >> 3;
  const int64_t kb = kb0 + q;
  const bool live = kb < KB;  // wave-uniform
  const int64_t n0 = (int64_t)cg * NT_COLS + h * 128;

  // ---- requests in arrival order: x chunks, the first weight tile; the
  // scales and the other tiles once x is staged
  constexpr int EPL = 16 / (int)sizeof(T);   // elements per 16-byte load
  constexpr int LPC = 8 / EPL;               // loads per 8-element chunk
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)((int64_t)M * K * sizeof(T)));
  u32x4 xr[2][LPC];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int c = threadIdx.x + NT_THREADS * r;   // chunk: row c >> 7, 8 elements at 8 * (c & 127)
    const int m = c >> 7, kk = c & 127;
    const int64_t k = kb0 * 128 + 8 * kk;
    const bool ok = m < M && k < K;
#pragma unroll
    for (int l = 0; l < LPC; ++l)
      xr[r][l] = buf_load_b128(rx, ok ? (uint32_t)(((int64_t)m * K + k + l * EPL) * sizeof(T)) : DEC_OOB, 0u);
  }
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)(N * K / 2));
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(scales, (uint32_t)(N * KB * 4));
  u32x4 wv[8];
  float sc[8];
  auto load_tile = [&](int t) {
    const int64_t n = std::min<int64_t>(n0 + 16 * t + j, N - 1);
    wv[t] = buf_load_b128_nt(rw, (uint32_t)(n * (K / 2) + kb * 64 + 16 * g), 0u);
  };
  // only the first tile before x is staged: requests queued ahead of x delay it
  if (live) load_tile(0);
  __builtin_amdgcn_sched_barrier(0);

  // ---- x to float, the workgroup's largest |x|
  float xv[2][8];
  float mx = 0.0f;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    if constexpr (EPL == 4) {
#pragma unroll
      for (int l = 0; l < 2; ++l)
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[r][4 * l + e] = __uint_as_float(xr[r][l][e]);
    } else {
      const T* tt = reinterpret_cast<const T*>(&xr[r][0]);
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[r][e] = ElemT<T>::cvt(tt[e]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = fmaxf(mx, __builtin_fabsf(xv[r][e]));
  }
  mx = group_max<64>(mx);
  if (lane == 0) s_wmax[wave] = mx;
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the LDS write above (vmcnt untouched)
  dec_barrier_nofence();
  float wmax = 0.0f;
#pragma unroll
  for (int i = 0; i < NT_WAVES; ++i) wmax = fmaxf(wmax, s_wmax[i]);
  // 2^-shift brings the largest |x| into [2^14, 2^15): within the f16 range,
  // and the rest of x as far above the f16 denormals as it can be
  const int bexp = (int)((__float_as_uint(wmax) >> 23) & 0xFFu);
  const int shift = (bexp == 0 || bexp == 0xFF) ? 0 : bexp - 127 - 14;
  const float xs = __builtin_ldexpf(1.0f, -shift);

  // ---- stage hi / lo: chunk (m, kk) -> block kk >> 4, lane group (kk >> 2) & 3, step kk & 3
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int c = threadIdx.x + NT_THREADS * r;
    const int m = c >> 7, kk = c & 127;
    const int blk = kk >> 4, gg = (kk >> 2) & 3, st = kk & 3;
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = xv[r][2 * e] * xs, b = xv[r][2 * e + 1] * xs;
      auto hp = __builtin_amdgcn_cvt_pkrtz(a, b);
      auto lp = __builtin_amdgcn_cvt_pkrtz(a - (float)hp[0], b - (float)hp[1]);
      hw[e] = __builtin_bit_cast(uint32_t, hp);
      lw[e] = __builtin_bit_cast(uint32_t, lp);
    }
    float* base = lds + ((blk * 4 + st) * 2) * 256 + (m + 16 * gg) * 4;
    *reinterpret_cast<u32x4*>(base) = u32x4{hw[0], hw[1], hw[2], hw[3]};
    *reinterpret_cast<u32x4*>(base + 256) = u32x4{lw[0], lw[1], lw[2], lw[3]};
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);
  dec_barrier_nofence();
  if (live) {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int64_t n = std::min<int64_t>(n0 + 16 * t + j, N - 1);
      const int64_t si = scales_kb_major ? kb * N + n : n * KB + kb;
      sc[t] = __uint_as_float(buf_load_b32_nt(rs, (uint32_t)(si * 4), 0u));
    }
#pragma unroll
    for (int t = 1; t < 8; ++t) load_tile(t);
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- MFMA, tile by tile as the weights arrive: the x fragments of the
  // wave's block stay in registers; 4 steps x hi/lo per tile
  f32x4 res[8];
  if (live) {
    f16x8 ahi[4], alo[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const float* ab = lds + ((q * 4 + st) * 2) * 256 + lane * 4;
      ahi[st] = __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4*>(ab));
      alo[st] = __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4*>(ab + 256));
    }
    const f16x8 b8 = __builtin_bit_cast(f16x8, u32x4v{0x00080008u, 0x00080008u, 0x00080008u, 0x00080008u});
    f32x4 corr = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[st], b8, corr, 0, 0, 0);
      corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[st], b8, corr, 0, 0, 0);
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const uint32_t wd = wv[t][st];
        const uint32_t lo = (wd & 0x0F0F0F0Fu) ^ 0x08080808u;
        const uint32_t hi = ((wd >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;
        const uint32_t d0 = __builtin_amdgcn_perm(hi, lo, 0x0C040C00u);
        const uint32_t d1 = __builtin_amdgcn_perm(hi, lo, 0x0C050C01u);
        const uint32_t d2 = __builtin_amdgcn_perm(hi, lo, 0x0C060C02u);
        const uint32_t d3 = __builtin_amdgcn_perm(hi, lo, 0x0C070C03u);
        const f16x8 bt = __builtin_bit_cast(f16x8, u32x4v{d0, d1, d2, d3});
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[st], bt, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[st], bt, acc, 0, 0, 0);
      }
      const float sf = sc[t] * 16777216.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) res[t][i] = __builtin_ldexpf(sf * (acc[i] - corr[i]), shift);
    }
  } else {
#pragma unroll
    for (int t = 0; t < 8; ++t) res[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // every wave is done reading the staged x before the partials overwrite it
  __syncthreads();
  {
    float* red = lds + (q * 16) * NT_RED_STRIDE + h * 128;
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[(4 * g + i) * NT_RED_STRIDE + 16 * t + j] = res[t][i];
  }
  __syncthreads();
  // thread: row m, columns c .. c+3, summed over the 8 blocks in order
  const int m = threadIdx.x >> 6, c = 4 * (threadIdx.x & 63);
  f32x4 sum = *reinterpret_cast<const f32x4*>(lds + m * NT_RED_STRIDE + c);
#pragma unroll
  for (int b = 1; b < NT_BLKS; ++b) sum += *reinterpret_cast<const f32x4*>(lds + (b * 16 + m) * NT_RED_STRIDE + c);
  const int64_t n = (int64_t)cg * NT_COLS + c;
  const bool mine = m < M && n < N;
  if (S == 1) {
    if (!mine) return;
    if (bias) sum += *reinterpret_cast<const f32x4*>(bias + n);
    *reinterpret_cast<f32x4*>(out + (int64_t)m * N + n) = sum;
    return;
  }
  // split K: publish the partial with write-through (sc1) stores, wait for
  // them, count the arrival; the last workgroup of the column group reads
  // the other partials past the L2s (sc1), adds the S partials in split
  // order and resets the counter
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(partials, (uint32_t)((int64_t)S * 16 * N * 4));
  const uint32_t poff = (uint32_t)(((int64_t)m * N + n) * 4);
  const uint32_t split_stride = (uint32_t)(16 * N * 4);
  if (mine) __builtin_amdgcn_raw_buffer_store_b128(sum, rp, poff, (uint32_t)ks * split_stride, 16);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = __hip_atomic_fetch_add(counters + cg, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == (unsigned)(S - 1) ? 1 : 0;
  }
  __syncthreads();
  if (!s_last) return;
  if (mine) {
    f32x4 tot = sum;
    for (int sp = 0; sp < S; ++sp) {
      const f32x4 pv = sp == ks ? sum
                                : __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                rp, poff, (uint32_t)sp * split_stride, 16));
      tot = sp == 0 ? pv : tot + pv;
    }
    if (bias) tot += *reinterpret_cast<const f32x4*>(bias + n);
    *reinterpret_cast<f32x4*>(out + (int64_t)m * N + n) = tot;
  }
  if (threadIdx.x == 0) __hip_atomic_store(counters + cg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- int4 decode, [N][K] weight, long waves
// The product of k_linear_w4t_decode with the work split of
// k_linear_w4_decode_tiled: one 128-column block (rows n0 .. n0+127 of W) per
// workgroup, W waves of KBW = 4 * STEPS / 16 blocks of K each (STEPS steps of
// 32 rows), so K splits S = ceil(K / (W * 32 * STEPS)) ways.  Each wave reads
// its own x rows row-contiguously, turns them into the A-fragment order of
// k_linear_w4t_decode through its own LDS slot (lane (j, g) of step st of
// block b: row j, codes 128 b + 32 g + 8 st .. +7), scales each row's
// largest |x| of the wave into [2^14, 2^15) (the power of two returns in the
// epilogue), and only then requests its scales and weights, so that x is not
// queued behind them.  Tile t of block b: lane (j, g) loads the 16 bytes at
// byte 64 b + 16 g of row n0 + 16 t + j (codes 128 b + 32 g .. +31), as
// stored (the B operand and the correction tile of k_linear_w4t_decode), or
// (TILED) the same codes from the tiled copy of mxk_linear_prepack_weight_nt,
// where the 16 lanes of a tile read 1 KiB contiguously and every B operand
// comes out of the words with masks (k_tile_w4t).  Each block's tile sums are
// scaled by that block's scale of the column before they are added.  The
// partial reduction and the split-K hand-off are those of
// k_linear_w4_decode_tiled.
template <typename T, int STEPS, int W, bool TILED>
__global__ __launch_bounds__(W * 64, 1) void k_linear_w4t_decode_long(
    const T* __restrict__ x, int M, int64_t K, int64_t N, const uint8_t* __restrict__ w,
    const float* __restrict__ scales, int scales_kb_major, const float* __restrict__ bias, float* __restrict__ out,
    float* __restrict__ partials, unsigned long long* __restrict__ counters, int S, int xcd_map) {
  constexpr int RPW = 32 * STEPS, R = W * RPW, KBW = RPW / 128;
  constexpr int TPB = W * 64 > 512 ? 512 : W * 64, RT = TPB, CPT = 2048 / TPB;
  constexpr int XS = RPW + 4;                // row stride of a wave's LDS slot (floats)
  constexpr int EPL = 16 / (int)sizeof(T);   // x elements per 16-byte load
  constexpr int LPR = RPW / EPL;             // lanes per x row in one load
  constexpr int RPL = 64 / LPR;              // x rows per load
  constexpr int XLD = 16 / RPL;              // x loads per lane
  static_assert(RPW % 128 == 0 && LPR >= 1 && RPL * LPR == 64 && XLD * RPL == 16, "x loads");
  static_assert(XS >= DEC_RS, "a wave's slot holds its partial");
  static_assert(CPT % 4 == 0 && TPB * CPT == 2048, "reduction split");
  __shared__ __attribute__((aligned(16))) float sR[W * 16 * XS];
  __shared__ int sXe[W * 16];
  __shared__ int s_flags;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int64_t NB = N / 128, KB = K / 128;
  int64_t nb;
  int ks;
  if (xcd_map) {
    const int i = (int)(blockIdx.x >> 3);
    nb = (int64_t)(i / S) * 8 + (blockIdx.x & 7);
    ks = i % S;
  } else {
    nb = blockIdx.x / S;
    ks = blockIdx.x % S;
  }
  const int64_t kw = (int64_t)ks * R + (int64_t)wave * RPW;  // this wave's first row of K
  const int64_t n0 = nb * 128;

  // ---- x rows of this wave
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)((int64_t)M * K * sizeof(T)));
  u32x4 xr[XLD];
#pragma unroll
  for (int q = 0; q < XLD; ++q) {
    const int m = q * RPL + lane / LPR;
    const int64_t kk = kw + (int64_t)EPL * (lane % LPR);
    const bool ok = m < M && kk < K;  // K % 128 == 0: a load is wholly in or out
    xr[q] = buf_load_b128(rx, ok ? (uint32_t)(((int64_t)m * K + kk) * sizeof(T)) : DEC_OOB, 0u);
  }
  __builtin_amdgcn_sched_barrier(0);

  float* xs = sR + wave * 16 * XS;
#pragma unroll
  for (int q = 0; q < XLD; ++q) {
    const int m = q * RPL + lane / LPR;
    const int c = EPL * (lane % LPR);
    float v[EPL];
    if constexpr (EPL == 4) {
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = __uint_as_float(xr[q][u]);
    } else {
      const T* tt = reinterpret_cast<const T*>(&xr[q]);
#pragma unroll
      for (int u = 0; u < EPL; ++u) v[u] = ElemT<T>::cvt(tt[u]);
    }
#pragma unroll
    for (int u = 0; u < EPL; u += 4)
      *reinterpret_cast<f32x4*>(xs + m * XS + c + u) = f32x4{v[u], v[u + 1], v[u + 2], v[u + 3]};
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // xv[8 (4 b + st) + e]: row j, codes 128 b + 32 g + 8 st + e of the wave's rows
  float xv[STEPS * 8];
#pragma unroll
  for (int b = 0; b < KBW; ++b)
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const f32x4 t = *reinterpret_cast<const f32x4*>(xs + j * XS + 128 * b + 32 * g + 8 * st + 4 * h);
#pragma unroll
        for (int u = 0; u < 4; ++u) xv[8 * (4 * b + st) + 4 * h + u] = t[u];
      }
  float mx = 0.0f;
#pragma unroll
  for (int u = 0; u < STEPS * 8; ++u) mx = fmaxf(mx, __builtin_fabsf(xv[u]));
  // row j sits in lanes j, j + 16, j + 32, j + 48
  mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(mx), 0x401F)));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const int be = (int)((__float_as_uint(mx) >> 23) & 0xFFu);
  const int xe = be == 0xFF ? 0 : 141 - (be == 0 ? 1 : be);  // largest |x| to [2^14, 2^15); zero rows: any
  f16x8 ahi[STEPS], alo[STEPS];
#pragma unroll
  for (int s8 = 0; s8 < STEPS; ++s8) {
    uint32_t hw[4], lw[4];
    // TILED: the odd steps meet B operands 16 times larger (high nibbles), so
    // their A is built at 2^-4 and every step sums into one accumulator
    const int xs8 = (TILED && (s8 & 1)) ? xe - 4 : xe;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = __builtin_ldexpf(xv[8 * s8 + 2 * e], xs8), b = __builtin_ldexpf(xv[8 * s8 + 2 * e + 1], xs8);
      auto hp = __builtin_amdgcn_cvt_pkrtz(a, b);
      auto lp = __builtin_amdgcn_cvt_pkrtz(a - (float)hp[0], b - (float)hp[1]);
      hw[e] = __builtin_bit_cast(uint32_t, hp);
      lw[e] = __builtin_bit_cast(uint32_t, lp);
    }
    ahi[s8] = __builtin_bit_cast(f16x8, u32x4v{hw[0], hw[1], hw[2], hw[3]});
    alo[s8] = __builtin_bit_cast(f16x8, u32x4v{lw[0], lw[1], lw[2], lw[3]});
  }
  if (g == 0) sXe[wave * 16 + j] = xe;

  // ---- scales and weights, requested once this wave's x is in.  A block
  // past K (only in the last split) re-reads block 0; its x rows are zeros.
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)(N * K / 2));
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(scales, (uint32_t)(N * KB * 4));
  float sc[KBW][8];
  u32x4 wv[KBW][8];
#pragma unroll
  for (int b = 0; b < KBW; ++b) {
    const int64_t kb0 = kw / 128 + b;
    const int64_t kb = kb0 < KB ? kb0 : 0;  // wave-uniform
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int64_t n = n0 + 16 * t + j;
      const int64_t si = scales_kb_major ? kb * N + n : n * KB + kb;
      sc[b][t] = __uint_as_float(buf_load_b32_nt(rs, (uint32_t)(si * 4), 0u));
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      if constexpr (TILED)
        wv[b][t] = buf_load_b128_nt(rw, 16u * lane, (uint32_t)(((nb * 8 + t) * KB + kb) * 1024));
      else
        wv[b][t] = buf_load_b128_nt(rw, (uint32_t)((n0 + 16 * t + j) * (K / 2) + 16 * g), (uint32_t)(kb * 64));
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- MFMA per block and tile; each block's sums scaled by its column scale
  f32x4 res[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) res[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  if constexpr (TILED) {
    // steps 0 and 2 from the low nibbles (code + 8) * 2^-24, steps 1 and 3
    // from the high nibbles (code + 8) * 2^-20 against A at 2^-4: word
    // 2 sp + h, byte q holds codes (step 2 sp, i) | (step 2 sp + 1, i) << 4
    // with i = 4 h + {0, 2, 1, 3}[q], so (w & 0x000F000F) and ((w >> 8) &
    // 0x000F000F) are the f16 pairs (i, i + 1) of the low step, the masks
    // 0x00F000F0 those of the high step
    const f16x8 bl = __builtin_bit_cast(f16x8, u32x4v{0x00080008u, 0x00080008u, 0x00080008u, 0x00080008u});
    const f16x8 bh = __builtin_bit_cast(f16x8, u32x4v{0x00800080u, 0x00800080u, 0x00800080u, 0x00800080u});
#pragma unroll
    for (int b = 0; b < KBW; ++b) {
      f32x4 corr = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int sp = 0; sp < 2; ++sp) {
        corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[4 * b + 2 * sp], bl, corr, 0, 0, 0);
        corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[4 * b + 2 * sp], bl, corr, 0, 0, 0);
        corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[4 * b + 2 * sp + 1], bh, corr, 0, 0, 0);
        corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[4 * b + 2 * sp + 1], bh, corr, 0, 0, 0);
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int sp = 0; sp < 2; ++sp) {
          const uint32_t w0 = wv[b][t][2 * sp], w1 = wv[b][t][2 * sp + 1];
          const uint32_t s0 = w0 >> 8, s1 = w1 >> 8;
          const f16x8 btl = __builtin_bit_cast(
              f16x8, u32x4v{(w0 & 0x000F000Fu) ^ 0x00080008u, (s0 & 0x000F000Fu) ^ 0x00080008u,
                            (w1 & 0x000F000Fu) ^ 0x00080008u, (s1 & 0x000F000Fu) ^ 0x00080008u});
          const f16x8 bth = __builtin_bit_cast(
              f16x8, u32x4v{(w0 & 0x00F000F0u) ^ 0x00800080u, (s0 & 0x00F000F0u) ^ 0x00800080u,
                            (w1 & 0x00F000F0u) ^ 0x00800080u, (s1 & 0x00F000F0u) ^ 0x00800080u});
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[4 * b + 2 * sp], btl, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[4 * b + 2 * sp], btl, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[4 * b + 2 * sp + 1], bth, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[4 * b + 2 * sp + 1], bth, acc, 0, 0, 0);
        }
        const float sf = sc[b][t] * 16777216.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) res[t][i] += sf * (acc[i] - corr[i]);
      }
    }
  } else {
    const f16x8 b8 = __builtin_bit_cast(f16x8, u32x4v{0x00080008u, 0x00080008u, 0x00080008u, 0x00080008u});
#pragma unroll
    for (int b = 0; b < KBW; ++b) {
      f32x4 corr = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[4 * b + st], b8, corr, 0, 0, 0);
        corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[4 * b + st], b8, corr, 0, 0, 0);
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const uint32_t wd = wv[b][t][st];
          const uint32_t lo = (wd & 0x0F0F0F0Fu) ^ 0x08080808u;
          const uint32_t hi = ((wd >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;
          const uint32_t d0 = __builtin_amdgcn_perm(hi, lo, 0x0C040C00u);
          const uint32_t d1 = __builtin_amdgcn_perm(hi, lo, 0x0C050C01u);
          const uint32_t d2 = __builtin_amdgcn_perm(hi, lo, 0x0C060C02u);
          const uint32_t d3 = __builtin_amdgcn_perm(hi, lo, 0x0C070C03u);
          const f16x8 bt = __builtin_bit_cast(f16x8, u32x4v{d0, d1, d2, d3});
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[4 * b + st], bt, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[4 * b + st], bt, acc, 0, 0, 0);
        }
        const float sf = sc[b][t] * 16777216.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) res[t][i] += sf * (acc[i] - corr[i]);
      }
    }
  }

  // ---- wave partial (rows 4g+i, columns 16t+j) into its own slot: no
  // barrier first, nothing else uses the slot
  float* rwv = sR + wave * 16 * XS;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int sh = -sXe[wave * 16 + 4 * g + i];
#pragma unroll
    for (int t = 0; t < 8; ++t) rwv[(4 * g + i) * XS + 16 * t + j] = __builtin_ldexpf(res[t][i], sh);
  }
  __syncthreads();
  // thread (< RT): row m, columns c .. c+CPT-1, summed over the waves in order
  const bool rt = threadIdx.x < RT;
  const int r = threadIdx.x % TPB;
  const int m = r / (128 / CPT), c = CPT * (r % (128 / CPT));
  f32x4 sum[CPT / 4];
#pragma unroll
  for (int h = 0; h < CPT / 4; ++h) {
    sum[h] = *reinterpret_cast<const f32x4*>(sR + m * XS + c + 4 * h);
#pragma unroll
    for (int q = 1; q < W; ++q) sum[h] += *reinterpret_cast<const f32x4*>(sR + (q * 16 + m) * XS + c + 4 * h);
  }
  const int64_t col = nb * 128 + c;
  if (S == 1) {
    if (rt && m < M) {
#pragma unroll
      for (int h = 0; h < CPT / 4; ++h) {
        f32x4 o = sum[h];
        if (bias) o += *reinterpret_cast<const f32x4*>(bias + col + 4 * h);
        *reinterpret_cast<f32x4*>(out + (int64_t)m * N + col + 4 * h) = o;
      }
    }
    return;
  }
  // split-K hand-off as in k_linear_w4_decode: partials [S][N/128][16][128]
  // written through, arrivals counted per XCC, the last arrival sums in
  // split order
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(partials, (uint32_t)((int64_t)S * NB * 16 * 128 * 4));
  const uint32_t poff = (uint32_t)(((nb * 16 + m) * 128 + c) * 4);
  const uint32_t split_stride = (uint32_t)(NB * 16 * 128 * 4);
  if (rt) {
#pragma unroll
    for (int h = 0; h < CPT / 4; ++h)
      __builtin_amdgcn_raw_buffer_store_b128(sum[h], rp, poff + 16u * h, (uint32_t)ks * split_stride, 16);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    xcc &= 7u;
    const unsigned long long inc = 1ull << (8 * xcc);
    const unsigned long long now =
        __hip_atomic_fetch_add(&counters[nb], inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + inc;
    unsigned total = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) total += (unsigned)((now >> (8 * q)) & 0xFFull);
    const bool same = ((now >> (8 * xcc)) & 0xFFull) == (unsigned long long)S;
    const bool last = total == (unsigned)S;
    if (last) __hip_atomic_store(&counters[nb], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_flags = (last ? 1 : 0) | (same ? 2 : 0);
  }
  __syncthreads();
  const int fl = s_flags;
  if (!(fl & 1) || !rt) return;
  f32x4 tot[CPT / 4];
  for (int sb = 0; sb < S; sb += 8) {
    f32x4 part[8][CPT / 4];
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int h = 0; h < CPT / 4; ++h) {
        const bool ld = sb + u < S && sb + u != ks;
        const uint32_t soff = ld ? (uint32_t)(sb + u) * split_stride : 0u;
        if (!ld)
          part[u][h] = sum[h];
        else if (fl & 2)
          part[u][h] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, poff + 16u * h, soff, 1));
        else
          part[u][h] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, poff + 16u * h, soff, 16));
      }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (sb + u < S)
#pragma unroll
        for (int h = 0; h < CPT / 4; ++h) tot[h] = (sb + u == 0) ? part[u][h] : tot[h] + part[u][h];
  }
  if (m < M) {
#pragma unroll
    for (int h = 0; h < CPT / 4; ++h) {
      f32x4 o = tot[h];
      if (bias) o += *reinterpret_cast<const f32x4*>(bias + col + 4 * h);
      *reinterpret_cast<f32x4*>(out + (int64_t)m * N + col + 4 * h) = o;
    }
  }
}


// The tiled copy of an int4 [N][K] weight (k_linear_w4t_decode_long<.., true>):
// chunk (16-row group nt, block kb of K): 1024 bytes at (nt * K/128 + kb) *
// 1024.  Its 16 bytes at +16 l (l = j + 16 g) hold the codes of row
// 16 nt + j at k = 128 kb + 32 g + 8 st + i (st < 4, i < 8), the 16 bytes
// the plain kernel's lane (j, g) loads, rearranged: word 2 sp + h, byte q is
// code (2 sp, i) | code (2 sp + 1, i) << 4 with i = 4 h + {0, 2, 1, 3}[q].
// One thread per 16-byte unit.
__global__ __launch_bounds__(256) void k_tile_w4t(const u32x4v* __restrict__ w, int64_t K, int64_t N,
                                                  u32x4v* __restrict__ wt) {
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t KB = K / 128;
  if (u >= N * K / 32) return;
  const int64_t nt = u / (KB * 64), rem = u % (KB * 64);
  const int64_t kb = rem / 64;
  const int l = (int)(rem % 64);
  const int64_t n = 16 * nt + (l & 15);
  const u32x4v src = w[(n * (K / 2) + kb * 64 + 16 * (l >> 4)) / 16];
  // code c of the unit (c = 8 st + i): nibble c & 1 of byte c >> 1
  auto code = [&](int c) -> uint32_t { return (src[c >> 3] >> (4 * (c & 7))) & 0xFu; };
  constexpr int ord[4] = {0, 2, 1, 3};
  u32x4v o;
#pragma unroll
  for (int wd = 0; wd < 4; ++wd) {
    const int sp = wd >> 1, h = wd & 1;
    uint32_t word = 0u;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = 4 * h + ord[q];
      word |= (code(16 * sp + i) | (code(16 * sp + 8 + i) << 4)) << (8 * q);
    }
    o[wd] = word;
  }
  wt[u] = o;
}

// The inverse of k_tile_w4t: the packed [N][K] codes of a tiled copy.  Code
// c = 8 st + i of a unit sits in word 2 (c >> 4) + (i >> 2), byte
// {0, 2, 1, 3}[i & 3] (the order is its own inverse), nibble (c >> 3) & 1.
// One thread per 16-byte unit.
__global__ __launch_bounds__(256) void k_untile_w4t(const u32x4v* __restrict__ wt, int64_t K, int64_t N,
                                                    u32x4v* __restrict__ w) {
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t KB = K / 128;
  if (u >= N * K / 32) return;
  const int64_t nt = u / (KB * 64), rem = u % (KB * 64);
  const int64_t kb = rem / 64;
  const int l = (int)(rem % 64);
  const int64_t n = 16 * nt + (l & 15);
  const u32x4v t = wt[u];
  constexpr int ord[4] = {0, 2, 1, 3};
  auto code = [&](int c) -> uint32_t {
    const int i = c & 7;
    return (t[2 * (c >> 4) + (i >> 2)] >> (8 * ord[i & 3] + 4 * ((c >> 3) & 1))) & 0xFu;
  };
  u32x4v o;
#pragma unroll
  for (int wd = 0; wd < 4; ++wd) {
    uint32_t word = 0u;
#pragma unroll
    for (int b = 0; b < 4; ++b) word |= (code(8 * wd + 2 * b) | (code(8 * wd + 2 * b + 1) << 4)) << (8 * b);
    o[wd] = word;
  }
  w[(n * (K / 2) + kb * 64 + 16 * (l >> 4)) / 16] = o;
}

static int nt_splits(int64_t K) { return (int)ceil_div(K / 128, NT_BLKS); }

static bool nt_decode_eligible(int64_t M, int64_t K, int64_t N, int kind, int bits, int block, const void* x,
                               int x_type, int64_t w_nbytes, int64_t w_nscales) {
  if (kind != MXK_KIND_INT || bits != 4 || block != 128) return false;
  if (M < 1 || M > 16 || K % 128 != 0 || N % 16 != 0) return false;
  if (ceil_div(N, NT_COLS) * 4 > DEC_COUNTER_BYTES) return false;
  if (!aligned16(x) || w_nbytes < N * K / 2 || w_nscales < N * (K / 128)) return false;
  const int esz = x_type == MXK_IN_F32 ? 4 : 2;
  const int64_t lim = int64_t(1) << 31;
  return N * K / 2 < lim && N * (K / 128) * 4 < lim && 16 * K * esz < lim &&
         (int64_t)nt_splits(K) * 16 * N * 4 < lim;
}


// The long-wave kernel: 8 waves of 8 steps (two blocks of K) per workgroup,
// 2048 rows of K per split.
#define NT_LONG_ROWS 2048
static int nt_long_splits(int64_t K) { return (int)ceil_div(K, NT_LONG_ROWS); }

static bool nt_long_eligible(int64_t K, int64_t N) {
  if (N % 128 != 0 || N / 128 > DEC_COUNTER_BYTES / 8) return false;
  const int64_t S = nt_long_splits(K);
  return S <= 255 && S * (N / 128) * 8192 < (int64_t(1) << 31);
}

// workspace: arrival counters (DEC_COUNTER_BYTES, zero between calls: one
// 32-bit count per 256-column group, or one 64-bit count of 8 per-XCC bytes
// per 128-column block for the long-wave kernel), then the partials:
// [S][16][N] or [S][N/128][16][128]
static size_t nt_workspace_bytes(int64_t K, int64_t N) {
  const int S = nt_splits(K);
  size_t need = S > 1 ? DEC_COUNTER_BYTES + (size_t)S * 16 * (size_t)N * 4 : 0;
  if (nt_long_eligible(K, N)) {
    const int SL = nt_long_splits(K);
    if (SL > 1) need = std::max(need, (size_t)DEC_COUNTER_BYTES + (size_t)SL * (size_t)(N / 128) * 8192);
  }
  return need;
}

template <typename T, bool TILED>
static int launch_nt_long(const T* x, int64_t M, int64_t K, int64_t N, const uint8_t* w, const float* scales,
                          int scales_kb_major, const float* bias, float* out, uint8_t* ws, hipStream_t st) {
  const int SL = nt_long_splits(K);
  const int64_t NB = N / 128;
  unsigned long long* lc = SL > 1 ? reinterpret_cast<unsigned long long*>(ws) : nullptr;
  float* lp = SL > 1 ? reinterpret_cast<float*>(ws + DEC_COUNTER_BYTES) : nullptr;
  hipLaunchKernelGGL((k_linear_w4t_decode_long<T, 8, 8, TILED>), dim3((unsigned)(NB * SL)), dim3(512), 0, st, x,
                     (int)M, K, N, w, scales, scales_kb_major, bias, out, lp, lc, SL, NB % 8 == 0 ? 1 : 0);
  return check_launch(TILED ? "linear_wq_nt_tiled" : "linear_wq_nt(decode)");
}

template <typename T>
static int launch_nt_decode(const T* x, int64_t M, int64_t K, int64_t N, const uint8_t* w, const float* scales,
                            int scales_kb_major, const float* bias, float* out, uint8_t* ws, hipStream_t st) {
  if (nt_long_eligible(K, N)) return launch_nt_long<T, false>(x, M, K, N, w, scales, scales_kb_major, bias, out, ws, st);
  const int S = nt_splits(K);
  const int64_t groups = ceil_div(N, NT_COLS);
  unsigned int* counters = S > 1 ? reinterpret_cast<unsigned int*>(ws) : nullptr;
  float* partials = S > 1 ? reinterpret_cast<float*>(ws + DEC_COUNTER_BYTES) : nullptr;
  hipLaunchKernelGGL((k_linear_w4t_decode<T>), dim3((unsigned)(groups * S)), dim3(NT_THREADS), 0, st, x, (int)M, K,
                     N, w, scales, scales_kb_major, bias, out, partials, counters, S);
  return check_launch("linear_wq_nt(decode)");
}

struct DecodePlan {
  int S, steps, nbw, xcd_map;
  size_t partial_bytes, counter_bytes, scales_t_bytes;
};

static int64_t dec_rows(int nbw, int steps) { return (int64_t)(DEC_WAVES / nbw) * 32 * steps; }

static DecodePlan plan_decode(int64_t K, int64_t N) {
  DecodePlan p;
  const int64_t NB = N / 128;
  // two-block column groups (x staged once for two blocks, 128-byte weight
  // rows) with the longest waves that still give every CU a workgroup; then
  // single blocks; else the shape with the most workgroups
  static const int cand[][2] = {{2, 4}, {2, 2}, {1, 4}, {1, 2}, {1, 1}};
  const int64_t target = num_cus();
  p.nbw = 1;
  p.steps = 1;
  int64_t best = -1;
  for (const auto& c : cand) {
    const int nbw = c[0], steps = c[1];
    if (NB % nbw) continue;
    const int64_t S = ceil_div(K, dec_rows(nbw, steps));
    if (S > 255) continue;  // 8-bit arrival counts per XCC
    const int64_t grid = (NB / nbw) * S;
    if (grid > best) {
      best = grid;
      p.nbw = nbw;
      p.steps = steps;
    }
    if (grid >= target) {
      p.nbw = nbw;
      p.steps = steps;
      break;
    }
  }
  p.S = (int)ceil_div(K, dec_rows(p.nbw, p.steps));
  p.xcd_map = (NB / p.nbw) % 8 == 0 ? 1 : 0;
  p.partial_bytes = p.S > 1 ? (((size_t)p.S * (size_t)NB * 8192 + 255) & ~(size_t)255) : 0;
  // the counters live in a fixed prefix that nothing else overwrites, so a
  // zero-filled workspace stays valid across calls of any shape (each call
  // resets the counters it used)
  p.counter_bytes = DEC_COUNTER_BYTES;
  // room for block-major scales when the caller has no prepacked copy
  p.scales_t_bytes = ((size_t)K * (size_t)NB * 4 + 255) & ~(size_t)255;
  return p;
}

// 8-bit codes: half the prefetch depth (the same bytes and registers in flight)
template <typename T, int STEPS, int NBW, int BITS, bool FP>
static void launch_decode_t(const DecodePlan& p, hipStream_t st, const void* x, int64_t M, int64_t K, int64_t N,
                            const uint32_t* w, const float* scales, const float* bias, float* out, float* partials,
                            unsigned long long* counters) {
  const dim3 grid((unsigned)((N / 128 / NBW) * p.S));
  hipLaunchKernelGGL((k_linear_w4_decode<T, STEPS, NBW, BITS == 8 ? 2 : 4, BITS, FP>), grid, dim3(DEC_THREADS), 0,
                     st, (const T*)x, (int)M, K, N, w, scales, bias, out, partials, counters, p.S, p.xcd_map);
}

template <typename T>
static void launch_decode(const DecodePlan& p, hipStream_t st, const void* x, int64_t M, int64_t K, int64_t N,
                          const uint32_t* w, const float* scales, const float* bias, float* out, float* partials,
                          unsigned long long* counters, int bits, int kind) {
#define MXK_DEC_K(STEPS, NBW, B, F) \
  launch_decode_t<T, STEPS, NBW, B, F>(p, st, x, M, K, N, w, scales, bias, out, partials, counters)
#define MXK_DEC(STEPS, NBW)                                                          \
  if (p.steps == STEPS && p.nbw == NBW) {                                           \
    const bool fp = kind == MXK_KIND_FLOAT;                                         \
    if (bits == 8) {                                                                \
      if (fp) MXK_DEC_K(STEPS, NBW, 8, true); else MXK_DEC_K(STEPS, NBW, 8, false); \
    } else if (bits == 2) {                                                         \
      MXK_DEC_K(STEPS, NBW, 2, false);                                              \
    } else if (bits == 1) {                                                         \
      MXK_DEC_K(STEPS, NBW, 1, false);                                              \
    } else {                                                                        \
      if (fp) MXK_DEC_K(STEPS, NBW, 4, true); else MXK_DEC_K(STEPS, NBW, 4, false); \
    }                                                                               \
    return;                                                                         \
  }
  MXK_DEC(4, 2)
  MXK_DEC(2, 2)
  MXK_DEC(4, 1)
  MXK_DEC(2, 1)
  MXK_DEC(1, 1)
#undef MXK_DEC
#undef MXK_DEC_K
}

// The tiled kernel: one block per workgroup, the longest waves that still
// give every CU a workgroup, else the shape with the most workgroups.  Waves
// of 8 steps come 8 to a workgroup (two per SIMD, 169 VGPRs), shorter ones 16.
static int tiled_waves(int steps) { return steps >= 4 ? 8 : 16; }
static int64_t tiled_rows(int steps) { return (int64_t)tiled_waves(steps) * 32 * steps; }

// x of 16-bit elements (half the bytes per row) streams faster with twice
// the workgroups (8 waves of 4 steps, two workgroups per CU: config 2 with
// bf16 x 12.77 -> 12.25 us per step); fp32 x with 8 waves of 8 steps (the
// same split measured 12.1 -> 12.8 us).
static DecodePlan plan_decode_tiled(int64_t K, int64_t N, int esz) {
  DecodePlan p;
  const int64_t NB = N / 128;
  const int64_t target = num_cus();
  p.nbw = 1;
  p.steps = 1;
  int64_t best = -1;
  for (const int steps : {esz == 2 ? 4 : 8, 2, 1}) {
    const int64_t S = ceil_div(K, tiled_rows(steps));
    if (S > 255) continue;  // 8-bit arrival counts per XCC
    const int64_t grid = NB * S;
    if (grid > best) {
      best = grid;
      p.steps = steps;
    }
    if (grid >= target) {
      p.steps = steps;
      break;
    }
  }
  p.S = (int)ceil_div(K, tiled_rows(p.steps));
  p.xcd_map = NB % 8 == 0 ? 1 : 0;
  p.partial_bytes = p.S > 1 ? (((size_t)p.S * (size_t)NB * 8192 + 255) & ~(size_t)255) : 0;
  p.counter_bytes = DEC_COUNTER_BYTES;
  p.scales_t_bytes = 0;  // the tiled path takes prepacked scales only
  return p;
}

template <typename T>
static void launch_decode_tiled(const DecodePlan& p, hipStream_t st, const void* x, int64_t M, int64_t K, int64_t N,
                                const uint32_t* wt, const float* scales_t, const float* bias, float* out,
                                float* partials, unsigned long long* counters, bool fp) {
  const dim3 grid((unsigned)((N / 128) * p.S));
#define MXK_DECT(STEPS, W)                                                                                   \
  if (p.steps == STEPS) {                                                                                   \
    if (fp)                                                                                                 \
      hipLaunchKernelGGL((k_linear_w4_decode_tiled<T, STEPS, W, true>), grid, dim3(W * 64), 0, st,          \
                         (const T*)x, (int)M, K, N, wt, scales_t, bias, out, partials, counters, p.S, p.xcd_map); \
    else                                                                                                    \
      hipLaunchKernelGGL((k_linear_w4_decode_tiled<T, STEPS, W, false>), grid, dim3(W * 64), 0, st,         \
                         (const T*)x, (int)M, K, N, wt, scales_t, bias, out, partials, counters, p.S, p.xcd_map); \
    return;                                                                                                 \
  }
  MXK_DECT(8, 8)
  MXK_DECT(4, 8)
  MXK_DECT(2, 16)
  MXK_DECT(1, 16)
#undef MXK_DECT
}

static bool decode_eligible(int64_t M, int64_t K, int64_t N, int kind, int bits, int block, const void* x,
                            int x_type, const void* w) {
  if (block != 128) return false;
  if (!(kind == MXK_KIND_INT && (bits == 1 || bits == 2 || bits == 4 || bits == 8)) &&
      !(kind == MXK_KIND_FLOAT && (bits == 4 || bits == 8)))
    return false;
  if (M < 1 || M > 16 || K % 32 != 0 || N % 128 != 0) return false;
  if (N / 128 > DEC_COUNTER_BYTES / 8 || K / 32 >= 65536) return false;
  if (!aligned16(x) || (reinterpret_cast<uintptr_t>(w) & (bits == 8 ? 7u : bits == 4 ? 3u : bits == 2 ? 1u : 0u)) != 0)
    return false;
  const int esz = x_type == MXK_IN_F32 ? 4 : 2;
  if ((K * esz) % 16 != 0) return false;
  // 32-bit buffer offsets with headroom
  if (K * N * bits / 8 >= (int64_t(1) << 31) || K * (N / 128) * 4 >= (int64_t(1) << 31) ||
      16 * K * esz >= (int64_t(1) << 31))
    return false;
  // partial buffer: S * (N/128) * 8 KiB, addressed with 32-bit offsets
  if ((K / 32 + 1) * (N / 128) * 8192 >= (int64_t(1) << 31)) return false;
  // each XCC's arrival count is 8 bits of a 64-bit counter: at most 255 splits
  return plan_decode(K, N).S <= 255;
}

// The tiled path: the decode path's shapes with a 16-byte aligned tiled
// weight and prepacked scales.
static bool decode_tiled_eligible(int64_t M, int64_t K, int64_t N, const void* x, int x_type, const void* wt,
                                  const float* scales_t) {
  if (M < 1 || M > 16 || K % 32 != 0 || N % 128 != 0) return false;
  if (N / 128 > DEC_COUNTER_BYTES / 8 || K / 32 >= 65536) return false;
  if (!aligned16(x) || !aligned16(wt) || !aligned16(scales_t)) return false;
  const int esz = x_type == MXK_IN_F32 ? 4 : 2;
  if ((K * esz) % 16 != 0) return false;
  if (K * N / 2 >= (int64_t(1) << 31) || K * (N / 128) * 4 >= (int64_t(1) << 31) || 16 * K * esz >= (int64_t(1) << 31))
    return false;
  if ((K / 32 + 1) * (N / 128) * 8192 >= (int64_t(1) << 31)) return false;
  return plan_decode_tiled(K, N, esz).S <= 255;
}

template <bool WT, typename T, int MODE, int BITS>
static int launch_linear(const T* x, int64_t M, int64_t K, int64_t N, const uint8_t* packed, int64_t pbytes,
                         const float* scales, int block, const float* bias, float* out, hipStream_t st) {
  dim3 grid((unsigned)ceil_div(N, 64), (unsigned)ceil_div(M, 64));
  hipLaunchKernelGGL((k_linear_generic<T, MODE, BITS, WT>), grid, dim3(256), 0, st, x, M, K, N, packed, pbytes,
                     scales, block, bias, out);
  return check_launch(WT ? "linear_wq_nt" : "linear_wq");
}

template <bool WT, typename T>
static int linear_t(const T* x, int64_t M, int64_t K, int64_t N, const uint8_t* packed, int64_t pbytes,
                    const float* scales, int kind, int bits, int block, const float* bias, float* out,
                    hipStream_t st) {
#define MXK_L(MODE, BITS) \
  if (mode == MODE && bits == BITS) return launch_linear<WT, T, MODE, BITS>(x, M, K, N, packed, pbytes, scales, block, bias, out, st);
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

// ---------------------------------------------------------------- allocation-free entry
// mxk_linear_wq_noalloc runs the decode linear with its split-K workspace in
// this file-scope array instead of a caller-provided buffer.  Each GPU holds
// its own copy until the process ends.  Host code never passes the array's
// name to a kernel (on the host it is only a stand-in): it uses the device
// address that hipGetSymbolAddress returns for the current device, kept per
// device.  The first NOALLOC_COUNTER_BYTES are the arrival counters, which
// must start at zero and which every call leaves zero.
#define NOALLOC_SCRATCH_BYTES (8u << 20)
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

__global__ void k_zero_words(uint32_t* __restrict__ p, uint32_t words) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < words; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// The current device's copy of `scratch`; on the first call for a device
// (with that device current) its address is looked up and its counter
// prefix is cleared by a fill kernel on `st` (no memset, so the call may
// also be captured into a graph).  Returns nullptr on failure (message set).
static void* noalloc_scratch(hipStream_t st) {
  static std::mutex mu;
  static std::vector<void*> ptrs;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    fail(MXK_ELAUNCH, "linear_wq_noalloc: hipGetDevice failed");
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(mu);
  if ((int)ptrs.size() <= dev) ptrs.resize(dev + 1, nullptr);
  if (!ptrs[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      fail(MXK_ELAUNCH, std::string("linear_wq_noalloc: hipGetSymbolAddress(scratch) failed: ") +
                            hipGetErrorString(e));
      return nullptr;
    }
    hipLaunchKernelGGL(k_zero_words, dim3(16), dim3(256), 0, st, reinterpret_cast<uint32_t*>(ptr),
                       (uint32_t)(DEC_COUNTER_BYTES / 4));
    if (check_launch("linear_wq_noalloc(clear counters)") != MXK_OK) return nullptr;
    ptrs[dev] = ptr;
  }
  return ptrs[dev];
}

}  // namespace mxk

using namespace mxk;

extern "C" {

size_t mxk_linear_workspace(int64_t M, int64_t K, int64_t N, int bits, int block) {
  // the MFMA path (any M, int4/int8 codes); its buffers start past the decode counters
  const size_t c = M > 0 && K > 0 && N > 0 ? linear_mfma_workspace(M, K, N, bits, block, false) : 0;
  if (M < 1 || M > 16 || (bits != 1 && bits != 2 && bits != 4 && bits != 8) || block != 128 || K <= 0 || N <= 0 ||
      K % 32 != 0 || N % 128 != 0)
    return c;
  // enough for mxk_linear_wq's decode path and for mxk_linear_wq_tiled
  const DecodePlan p = plan_decode(K, N), q = plan_decode_tiled(K, N, 4), q2 = plan_decode_tiled(K, N, 2);
  const size_t a = p.S <= 255 ? p.counter_bytes + p.partial_bytes + p.scales_t_bytes : 0;  // else generic kernel
  const size_t b = std::max(q.S <= 255 ? q.counter_bytes + q.partial_bytes : 0,
                            q2.S <= 255 ? q2.counter_bytes + q2.partial_bytes : 0);
  return std::max(std::max(a, b), c);
}

int mxk_linear_prepack_weight(const void* w_packed, int64_t K, int64_t N, int bits, int block, void* w_tiled,
                              void* stream) {
  if (!w_packed || !w_tiled) return fail(MXK_EINVAL, "linear_prepack_weight: null pointer");
  if (bits != 4 || block != 128 || K <= 0 || N <= 0 || K % 32 != 0 || N % 128 != 0)
    return fail(MXK_EINVAL, "linear_prepack_weight: needs int4 codes, block 128, K a multiple of 32 and N of 128");
  if ((reinterpret_cast<uintptr_t>(w_packed) & 3u) != 0 || !aligned16(w_tiled))
    return fail(MXK_EINVAL, "linear_prepack_weight: w_packed must be 4-byte and w_tiled 16-byte aligned");
  const int64_t threads = (N / 128) * (K / 32) * 64;
  if (ceil_div(threads, 256) >= (int64_t(1) << 31)) return fail(MXK_EUNSUPPORTED, "linear_prepack_weight: too large");
  hipLaunchKernelGGL(k_tile_w4, dim3((unsigned)ceil_div(threads, 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const uint32_t*>(w_packed), K, N,
                     reinterpret_cast<uint32_t*>(w_tiled));
  return check_launch("linear_prepack_weight");
}

int mxk_linear_unpack_weight(const void* w_tiled, int64_t K, int64_t N, int bits, int block, void* w_packed,
                             void* stream) {
  if (!w_packed || !w_tiled) return fail(MXK_EINVAL, "linear_unpack_weight: null pointer");
  if (bits != 4 || block != 128 || K <= 0 || N <= 0 || K % 32 != 0 || N % 128 != 0)
    return fail(MXK_EINVAL, "linear_unpack_weight: needs int4 codes, block 128, K a multiple of 32 and N of 128");
  if ((reinterpret_cast<uintptr_t>(w_packed) & 3u) != 0 || !aligned16(w_tiled))
    return fail(MXK_EINVAL, "linear_unpack_weight: w_packed must be 4-byte and w_tiled 16-byte aligned");
  const int64_t threads = (N / 128) * (K / 32) * 64;
  if (ceil_div(threads, 256) >= (int64_t(1) << 31)) return fail(MXK_EUNSUPPORTED, "linear_unpack_weight: too large");
  hipLaunchKernelGGL(k_untile_w4, dim3((unsigned)ceil_div(threads, 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const uint32_t*>(w_tiled), K, N,
                     reinterpret_cast<uint32_t*>(w_packed));
  return check_launch("linear_unpack_weight");
}

int mxk_linear_wq_tiled(const void* x, int x_type, int64_t M, int64_t K, const void* w_tiled, const float* w_scales_t,
                        int64_t N, int kind, const float* bias, float* out, void* workspace, size_t workspace_nbytes,
                        void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (M <= 0 || K <= 0 || N <= 0) return fail(MXK_EINVAL, "linear_wq_tiled: sizes must be positive");
  if (!x || !w_tiled || !w_scales_t || !out) return fail(MXK_EINVAL, "linear_wq_tiled: null pointer");
  if (kind != MXK_KIND_INT && kind != MXK_KIND_FLOAT)
    return fail(MXK_EINVAL, "linear_wq_tiled: kind must be int (int4 codes) or float (FP4 codes)");
  const bool fp = kind == MXK_KIND_FLOAT;
  if (x_type != MXK_IN_F32 && x_type != MXK_IN_F16 && x_type != MXK_IN_BF16)
    return fail(MXK_EINVAL, "linear_wq_tiled: bad input type");
  if ((bias && !aligned16(bias)) || !aligned16(out))
    return fail(MXK_EINVAL, "linear_wq_tiled: bias and out must be 16-byte aligned");
  if (!decode_tiled_eligible(M, K, N, x, x_type, w_tiled, w_scales_t)) {
    // more than 16 rows (or x not on 16 bytes): the MFMA path reads the tiled copy too
    if (K % 32 == 0 && aligned16(w_tiled) && aligned16(w_scales_t)) {
      const int rc = linear_mfma_kn_tiled(x, x_type, M, K, w_tiled, w_scales_t, N, kind, bias, out, workspace,
                                          workspace_nbytes, st);
      if (rc != MXK_EUNSUPPORTED) return rc;
    }
    return fail(MXK_EUNSUPPORTED, "linear_wq_tiled: needs K % 32 == 0, N % 128 == 0, 16-byte aligned w_tiled "
                                  "and w_scales_t (use mxk_linear_wq)");
  }
  const DecodePlan p = plan_decode_tiled(K, N, x_type == MXK_IN_F32 ? 4 : 2);
  const size_t need = p.counter_bytes + p.partial_bytes;
  if (p.S > 1 && (!workspace || workspace_nbytes < need))
    return fail(MXK_EINVAL, "linear_wq_tiled: needs a zero-initialised workspace of mxk_linear_workspace() bytes");
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  unsigned long long* counters = p.S > 1 ? reinterpret_cast<unsigned long long*>(ws) : nullptr;
  float* partials = p.S > 1 ? reinterpret_cast<float*>(ws + p.counter_bytes) : nullptr;
  const uint32_t* wt = reinterpret_cast<const uint32_t*>(w_tiled);
  if (x_type == MXK_IN_F32)
    launch_decode_tiled<float>(p, st, x, M, K, N, wt, w_scales_t, bias, out, partials, counters, fp);
  else if (x_type == MXK_IN_F16)
    launch_decode_tiled<__half>(p, st, x, M, K, N, wt, w_scales_t, bias, out, partials, counters, fp);
  else launch_decode_tiled<hip_bfloat16>(p, st, x, M, K, N, wt, w_scales_t, bias, out, partials, counters, fp);
  return check_launch("linear_wq_tiled");
}

int mxk_linear_prepack_scales(const float* w_scales, int64_t K, int64_t N, int block, float* w_scales_t,
                              void* stream) {
  if (!w_scales || !w_scales_t) return fail(MXK_EINVAL, "linear_prepack_scales: null pointer");
  if (block != 128 || K <= 0 || N <= 0 || N % 128 != 0)
    return fail(MXK_EINVAL, "linear_prepack_scales: needs block 128, K > 0 and N a multiple of 128");
  if (ceil_div(K, 32) >= 65536) return fail(MXK_EUNSUPPORTED, "linear_prepack_scales: K too large");
  launch_transpose_scales(w_scales, K, N / 128, w_scales_t, reinterpret_cast<hipStream_t>(stream));
  return check_launch("linear_prepack_scales");
}

// mxk_linear_wq with the MFMA path switched on or off (off: the
// allocation-free entry when its scratch is too small for that path)
static int linear_wq_impl(const void* x, int x_type, int64_t M, int64_t K, const void* w_packed,
                          const float* w_scales, const float* w_scales_t, int64_t N, int kind, int bits, int block,
                          const float* bias, float* out, void* workspace, size_t workspace_nbytes, void* stream,
                          bool mfma) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (M <= 0 || K <= 0 || N <= 0 || block <= 0) return fail(MXK_EINVAL, "linear_wq: sizes must be positive");
  if (!x || !w_packed || !w_scales || !out) return fail(MXK_EINVAL, "linear_wq: null pointer");
  if (decode_eligible(M, K, N, kind, bits, block, x, x_type, w_packed)) {
    DecodePlan p = plan_decode(K, N);
    const size_t need = p.counter_bytes + p.partial_bytes + (w_scales_t ? 0 : p.scales_t_bytes);
    if (need > 0 && (!workspace || workspace_nbytes < need))
      return fail(MXK_EINVAL, "linear_wq: decode path needs a zero-initialised workspace of mxk_linear_workspace() bytes");
    uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
    unsigned long long* counters = p.S > 1 ? reinterpret_cast<unsigned long long*>(ws) : nullptr;
    float* partials = p.S > 1 ? reinterpret_cast<float*>(ws + p.counter_bytes) : nullptr;
    const float* sT = w_scales_t;
    if (!sT) {
      float* tmp = reinterpret_cast<float*>(ws + p.counter_bytes + p.partial_bytes);
      launch_transpose_scales(w_scales, K, N / 128, tmp, st);
      sT = tmp;
    }
    const uint32_t* wq = reinterpret_cast<const uint32_t*>(w_packed);
    if (x_type == MXK_IN_F32)
      launch_decode<float>(p, st, x, M, K, N, wq, sT, bias, out, partials, counters, bits, kind);
    else if (x_type == MXK_IN_F16)
      launch_decode<__half>(p, st, x, M, K, N, wq, sT, bias, out, partials, counters, bits, kind);
    else launch_decode<hip_bfloat16>(p, st, x, M, K, N, wq, sT, bias, out, partials, counters, bits, kind);
    return check_launch("linear_wq(decode)");
  }
  if (mfma) {
    const int rc = linear_mfma_kn(x, x_type, M, K, w_packed, w_scales, w_scales_t, N, kind, bits, block, bias, out,
                                  workspace, workspace_nbytes, st);
    if (rc != MXK_EUNSUPPORTED) return rc;
  }
  const int64_t nb = ceil_div(K * N, block);
  const int64_t pbytes = mxk_packed_nbytes(bits, nb * block);
  const uint8_t* pk = reinterpret_cast<const uint8_t*>(w_packed);
  if (x_type == MXK_IN_F32)
    return linear_t<false, float>((const float*)x, M, K, N, pk, pbytes, w_scales, kind, bits, block, bias, out, st);
  if (x_type == MXK_IN_F16)
    return linear_t<false, __half>((const __half*)x, M, K, N, pk, pbytes, w_scales, kind, bits, block, bias, out, st);
  if (x_type == MXK_IN_BF16)
    return linear_t<false, hip_bfloat16>((const hip_bfloat16*)x, M, K, N, pk, pbytes, w_scales, kind, bits, block,
                                         bias, out, st);
  return fail(MXK_EINVAL, "linear_wq: bad input type");
}

int mxk_linear_wq(const void* x, int x_type, int64_t M, int64_t K, const void* w_packed, const float* w_scales,
                  const float* w_scales_t, int64_t N, int kind, int bits, int block, const float* bias, float* out,
                  void* workspace, size_t workspace_nbytes, void* stream) {
  return linear_wq_impl(x, x_type, M, K, w_packed, w_scales, w_scales_t, N, kind, bits, block, bias, out, workspace,
                        workspace_nbytes, stream, true);
}

int mxk_linear_wq_noalloc(const void* x, int x_type, int64_t M, int64_t K, const void* w_packed,
                          const float* w_scales, const float* w_scales_t, int64_t N, int kind, int bits, int block,
                          const float* bias, float* out, void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (M <= 0 || K <= 0 || N <= 0 || block <= 0) return fail(MXK_EINVAL, "linear_wq_noalloc: sizes must be positive");
  if (!x || !w_packed || !w_scales || !out) return fail(MXK_EINVAL, "linear_wq_noalloc: null pointer");
  size_t need = 0;
  bool mfma = false;
  if (decode_eligible(M, K, N, kind, bits, block, x, x_type, w_packed)) {
    const DecodePlan p = plan_decode(K, N);
    need = p.counter_bytes + p.partial_bytes + (w_scales_t ? 0 : p.scales_t_bytes);
    if (need > NOALLOC_SCRATCH_BYTES)
      return fail(MXK_EINVAL, "linear_wq_noalloc: this shape needs " + std::to_string(need) +
                                  " bytes of split-K workspace, more than the " +
                                  std::to_string(NOALLOC_SCRATCH_BYTES) +
                                  "-byte static scratch (pass w_scales_t, or use mxk_linear_wq with a workspace)");
  } else {
    // the MFMA path when its buffers fit the scratch; the generic kernel otherwise
    const size_t m = linear_mfma_workspace(M, K, N, bits, block, false);
    if (m > 0 && m <= NOALLOC_SCRATCH_BYTES) {
      need = m;
      mfma = true;
    }
  }
  void* ws = nullptr;
  if (need > 0 && !(ws = noalloc_scratch(st))) return MXK_ELAUNCH;
  return linear_wq_impl(x, x_type, M, K, w_packed, w_scales, w_scales_t, N, kind, bits, block, bias, out, ws,
                        need > 0 ? NOALLOC_SCRATCH_BYTES : 0, stream, mfma);
}

size_t mxk_linear_nt_workspace(int64_t M, int64_t K, int64_t N, int bits, int block) {
  const size_t c = M > 0 && K > 0 && N > 0 ? linear_mfma_workspace(M, K, N, bits, block, true) : 0;
  if (M < 1 || M > 16 || bits != 4 || block != 128 || K <= 0 || N <= 0 || K % 128 != 0 || N % 16 != 0) return c;
  return std::max(nt_workspace_bytes(K, N), c);
}

int mxk_linear_wq_nt(const void* x, int x_type, int64_t M, int64_t K, const void* w_packed, int64_t w_nbytes,
                     const float* w_scales, int64_t w_nscales, const float* w_scales_t, int64_t N, int kind,
                     int bits, int block, const float* bias, float* out, void* workspace, size_t workspace_nbytes,
                     void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (M <= 0 || K <= 0 || N <= 0 || block <= 0) return fail(MXK_EINVAL, "linear_wq_nt: sizes must be positive");
  if (!x || !w_packed || !w_scales || !out) return fail(MXK_EINVAL, "linear_wq_nt: null pointer");
  if (w_nscales < ceil_div(N * K, block)) return fail(MXK_EINVAL, "linear_wq_nt: fewer scales than blocks");
  if (w_nbytes < mxk_packed_nbytes(bits, N * K)) return fail(MXK_EINVAL, "linear_wq_nt: packed weight too short");
  const uint8_t* pk = reinterpret_cast<const uint8_t*>(w_packed);
  if (nt_decode_eligible(M, K, N, kind, bits, block, x, x_type, w_nbytes, w_nscales)) {
    const size_t need = nt_workspace_bytes(K, N);
    if (need > 0 && (!workspace || workspace_nbytes < need))
      return fail(MXK_EINVAL, "linear_wq_nt: decode path needs a zero-initialised workspace of "
                              "mxk_linear_nt_workspace() bytes");
    uint8_t* part = reinterpret_cast<uint8_t*>(workspace);
    const float* sc = w_scales_t ? w_scales_t : w_scales;
    const int kbm = w_scales_t ? 1 : 0;
    if (x_type == MXK_IN_F32)
      return launch_nt_decode((const float*)x, M, K, N, pk, sc, kbm, bias, out, part, st);
    if (x_type == MXK_IN_F16)
      return launch_nt_decode((const __half*)x, M, K, N, pk, sc, kbm, bias, out, part, st);
    if (x_type == MXK_IN_BF16)
      return launch_nt_decode((const hip_bfloat16*)x, M, K, N, pk, sc, kbm, bias, out, part, st);
  }
  {
    const int rc = linear_mfma_nk(x, x_type, M, K, w_packed, w_scales, w_scales_t, N, kind, bits, block, bias, out,
                                  workspace, workspace_nbytes, st);
    if (rc != MXK_EUNSUPPORTED) return rc;
  }
  if (x_type == MXK_IN_F32)
    return linear_t<true, float>((const float*)x, M, K, N, pk, w_nbytes, w_scales, kind, bits, block, bias, out, st);
  if (x_type == MXK_IN_F16)
    return linear_t<true, __half>((const __half*)x, M, K, N, pk, w_nbytes, w_scales, kind, bits, block, bias, out,
                                  st);
  if (x_type == MXK_IN_BF16)
    return linear_t<true, hip_bfloat16>((const hip_bfloat16*)x, M, K, N, pk, w_nbytes, w_scales, kind, bits, block,
                                        bias, out, st);
  return fail(MXK_EINVAL, "linear_wq_nt: bad input type");
}

int mxk_linear_prepack_weight_nt(const void* w_packed, int64_t N, int64_t K, int bits, int block, void* w_tiled,
                                 void* stream) {
  if (!w_packed || !w_tiled) return fail(MXK_EINVAL, "linear_prepack_weight_nt: null pointer");
  if (bits != 4 || block != 128 || K <= 0 || N <= 0 || K % 128 != 0 || N % 128 != 0)
    return fail(MXK_EINVAL, "linear_prepack_weight_nt: needs int4 codes, block 128, K and N multiples of 128");
  if (!aligned16(w_packed) || !aligned16(w_tiled))
    return fail(MXK_EINVAL, "linear_prepack_weight_nt: w_packed and w_tiled must be 16-byte aligned");
  const int64_t units = N * K / 32;
  if (ceil_div(units, 256) >= (int64_t(1) << 31)) return fail(MXK_EUNSUPPORTED, "linear_prepack_weight_nt: too large");
  hipLaunchKernelGGL(k_tile_w4t, dim3((unsigned)ceil_div(units, 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const u32x4v*>(w_packed), K, N,
                     reinterpret_cast<u32x4v*>(w_tiled));
  return check_launch("linear_prepack_weight_nt");
}

int mxk_linear_unpack_weight_nt(const void* w_tiled, int64_t N, int64_t K, int bits, int block, void* w_packed,
                                void* stream) {
  if (!w_packed || !w_tiled) return fail(MXK_EINVAL, "linear_unpack_weight_nt: null pointer");
  if (bits != 4 || block != 128 || K <= 0 || N <= 0 || K % 128 != 0 || N % 128 != 0)
    return fail(MXK_EINVAL, "linear_unpack_weight_nt: needs int4 codes, block 128, K and N multiples of 128");
  if (!aligned16(w_packed) || !aligned16(w_tiled))
    return fail(MXK_EINVAL, "linear_unpack_weight_nt: w_packed and w_tiled must be 16-byte aligned");
  const int64_t units = N * K / 32;
  if (ceil_div(units, 256) >= (int64_t(1) << 31)) return fail(MXK_EUNSUPPORTED, "linear_unpack_weight_nt: too large");
  hipLaunchKernelGGL(k_untile_w4t, dim3((unsigned)ceil_div(units, 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const u32x4v*>(w_tiled), K, N,
                     reinterpret_cast<u32x4v*>(w_packed));
  return check_launch("linear_unpack_weight_nt");
}

int mxk_linear_wq_nt_tiled(const void* x, int x_type, int64_t M, int64_t K, const void* w_tiled,
                           const float* w_scales_t, int64_t N, const float* bias, float* out, void* workspace,
                           size_t workspace_nbytes, void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (M <= 0 || K <= 0 || N <= 0) return fail(MXK_EINVAL, "linear_wq_nt_tiled: sizes must be positive");
  if (!x || !w_tiled || !w_scales_t || !out) return fail(MXK_EINVAL, "linear_wq_nt_tiled: null pointer");
  if (x_type != MXK_IN_F32 && x_type != MXK_IN_F16 && x_type != MXK_IN_BF16)
    return fail(MXK_EINVAL, "linear_wq_nt_tiled: bad input type");
  if ((bias && !aligned16(bias)) || !aligned16(out))
    return fail(MXK_EINVAL, "linear_wq_nt_tiled: bias and out must be 16-byte aligned");
  const int esz = x_type == MXK_IN_F32 ? 4 : 2;
  const int64_t lim = int64_t(1) << 31;
  if (K % 128 != 0 || N % 128 != 0 || !aligned16(w_tiled) || !aligned16(w_scales_t))
    return fail(MXK_EUNSUPPORTED, "linear_wq_nt_tiled: needs K and N multiples of 128 and 16-byte aligned w_tiled "
                                  "and w_scales_t (use mxk_linear_wq_nt)");
  if (M > 16 || !nt_long_eligible(K, N) || !aligned16(x) || N * K / 2 >= lim || N * (K / 128) * 4 >= lim ||
      16 * K * esz >= lim) {
    // the other shapes: the MFMA kernel on the same tiled copy
    const int rc = linear_mfma_nk_tiled(x, x_type, M, K, w_tiled, w_scales_t, N, bias, out, workspace,
                                        workspace_nbytes, st);
    if (rc != MXK_EUNSUPPORTED) return rc;
    return fail(MXK_EUNSUPPORTED, "linear_wq_nt_tiled: shape not supported on the tiled copy (use mxk_linear_wq_nt)");
  }
  const size_t need = nt_workspace_bytes(K, N);
  if (nt_long_splits(K) > 1 && (!workspace || workspace_nbytes < need))
    return fail(MXK_EINVAL, "linear_wq_nt_tiled: needs a zero-initialised workspace of mxk_linear_nt_workspace() bytes");
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  const uint8_t* wt = reinterpret_cast<const uint8_t*>(w_tiled);
  if (x_type == MXK_IN_F32)
    return launch_nt_long<float, true>((const float*)x, M, K, N, wt, w_scales_t, 1, bias, out, ws, st);
  if (x_type == MXK_IN_F16)
    return launch_nt_long<__half, true>((const __half*)x, M, K, N, wt, w_scales_t, 1, bias, out, ws, st);
  return launch_nt_long<hip_bfloat16, true>((const hip_bfloat16*)x, M, K, N, wt, w_scales_t, 1, bias, out, ws, st);
}

}  // extern "C"
