// MFMA weight-only linear for gfx950: the shapes and formats the int4
// decode kernels do not take (more than 16 rows of x; int2d, int8d, float4d
// and float8d weights at any row count).
//
//   mx_linear.forward (mxtorch.py:7454-7473), weight [K][N] as
//   quantize(W.t()) with blocks of 128 along N:
//       y[m,n] = sum_k x[m,k] * RN(c[k,n] * s[k, n/128])
//   mx_dynamic_linear.forward (mxtorch.py:8945-8962) and the input
//   gradients of _MXLinearAutograd / mx_linear (mxtorch.py:6729-6746,
//   7473), weight [N][K] with blocks of 128 along K:
//       y[m,n] = sum_k x[m,k] * RN(c[n,k] * s[n, k/128])
//
// Both products run on v_mfma_f32_16x16x32_f16 with fp32 accumulation.  The
// codes themselves are the B operand: integers |c| <= 127 are exact f16
// values, and so are the FP4 E2M1 and FP8 E4M3 values v of the float grids,
// whose grid value RN(v / vmax) takes the factor RN(1 / vmax) in the
// epilogue instead (vmax 6 or 480).  The x side is an f16 pair hi + lo (22 significant bits), so each
// term x * s * c carries a relative error of about 2^-22 and sums in fp32;
// the reference rounds RN(c * s) and runs an fp32 sgemm (about 2^-24 per
// term, in a library-defined order).
//
// [K][N] weights.  The scale changes along the contraction, so it goes into
// the A operand: a workgroup owns one 128-column block nb and builds
// A = x * s[., nb] per k step as hi + lo (two v_fma_mix per element).
//
// [N][K] weights.  The scale is constant over each block of 128 along K, so
// A is x itself, split into hi + lo once by the prepass, and each block's
// tile sums P are scaled in the epilogue: acc = fma(P, s[n, kb], acc).
//
// Range.  A prepass scales each row of x by the power of two 2^ex[m] that
// puts its largest |x| in [1, 2) and, for [K][N], each column block's scales
// by 2^es[nb] that puts the largest in [2^13, 2^14).  Every A value then lies
// below 2^15, inside f16's range, whatever the input magnitudes; the
// epilogue multiplies by 2^-(ex + es).  Terms far below a row's largest
// keep an absolute error of at most 2^-25 of the scaled units.
//
// Work split.  A workgroup of 8 waves owns 128 output columns, BM = 32 WM
// rows and a range of K in stages of 256 rows.  Per stage the 8 waves decode
// the stage's 256 x 128 codes once into LDS as f16 B fragments (64 KiB; two
// stages in flight), then wave (wm, wk) runs the k steps wk, wk + WK, ... of
// the stage on rows 32 wm .. +31 (WK = 8 / WM): 2 row tiles x 8 column
// tiles x (hi, lo) = 32 MFMAs per k step.  Column tile t, MFMA column j is
// output column 128 nb + 8 j + t, so a lane's 8 tiles are 8 consecutive
// columns.  Waves that split K meet in LDS at the end, in wk order; K
// splits across workgroups (few rows) write partials that a second kernel
// sums in split order.  Every reduction order is fixed, so results are
// deterministic.
#include "mxk_internal.h"

#include <algorithm>
#include <type_traits>

namespace mxk {

namespace {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
typedef uint32_t u2v __attribute__((ext_vector_type(2)));

constexpr int LM_THREADS = 512;
constexpr int LM_STAGE = 256;                  // rows of K per LDS stage
constexpr int LM_FRAG = 1024;                  // one B fragment: 64 lanes x 8 f16
constexpr int LM_STAGE_BYTES = 64 * LM_FRAG;   // 8 k steps x 8 column tiles
constexpr uint32_t LM_OOB = 0x80000000u;       // past every buffer: loads return zeros
constexpr size_t LM_WS_BASE = 65536;           // workspace bytes left to the decode kernels' counters

// Slot of MFMA lane `lane` in the fragment of k step `ks`: a permutation of
// the 16 slots of each 16-lane group, so that the fragment reads (16 lanes
// per LDS cycle) stay conflict-free and the decoders' stores, whose 16-lane
// groups span k steps, spread over every bank.
__device__ __forceinline__ int lm_slot(int lane, int ks) { return lane ^ ((2 * ks + (lane >> 5)) & 15); }
__device__ __forceinline__ uint32_t lm_frag_off(int ks, int t, int lane) {
  return (uint32_t)((ks * 8 + t) * LM_FRAG + lm_slot(lane, ks) * 16);
}

// Two int4 codes at bits 0-3 and 16-19 of d (other bits ignored) as an f16
// pair: 0x6400 | (c ^ 8) is the f16 1024 + (c + 8), exact, less 1032.
__device__ __forceinline__ uint32_t lm_i4pair(uint32_t d) {
  const uint32_t e = (d & 0x000F000Fu) ^ 0x64086408u;
  const h2v r = __builtin_bit_cast(h2v, e) - h2v{(_Float16)1032.0f, (_Float16)1032.0f};
  return __builtin_bit_cast(uint32_t, r);
}
// Two int8 codes at bits 0-7 and 16-23 of d (bits 8-15, 24-31 zero):
// 0x6400 | (c ^ 0x80) is 1024 + (c + 128), less 1152.
__device__ __forceinline__ uint32_t lm_i8pair(uint32_t d) {
  const uint32_t e = d ^ 0x64806480u;
  const h2v r = __builtin_bit_cast(h2v, e) - h2v{(_Float16)1152.0f, (_Float16)1152.0f};
  return __builtin_bit_cast(uint32_t, r);
}
// Two int2 codes at bits 0-1 and 16-17 of d (other bits ignored):
// 0x6400 | (c ^ 2) is 1024 + (c + 2), less 1026.
__device__ __forceinline__ uint32_t lm_i2pair(uint32_t d) {
  const uint32_t e = (d & 0x00030003u) ^ 0x64026402u;
  const h2v r = __builtin_bit_cast(h2v, e) - h2v{(_Float16)1026.0f, (_Float16)1026.0f};
  return __builtin_bit_cast(uint32_t, r);
}
// Two int1 codes at bits 0 and 16 of d (other bits ignored): code 0 is
// +1 and code 1 is -1 (the reference's 1-bit grid), so the code is the f16
// sign bit of 1.0.
__device__ __forceinline__ uint32_t lm_i1pair(uint32_t d) { return ((d & 0x00010001u) << 15) | 0x3C003C00u; }
// Weight formats: the code width in the low 4 bits, 16 for float grids
enum : int { LM_I1 = 1, LM_I2 = 2, LM_I4 = 4, LM_I8 = 8, LM_F4 = 16 + 4, LM_F8 = 16 + 8 };
__host__ __device__ constexpr int lm_bits(int fmt) { return fmt & 15; }
// The factor the outputs take for B fragments that hold v * 2^-P instead of
// the grid value v / vmax: RN(1/6) * 2^14, RN(1/480) * 2^8, or 1 for integer
// codes.
__host__ __device__ constexpr float lm_post(int fmt) {
  return fmt == LM_F4 ? (1.0f / 6.0f) * 16384.0f : fmt == LM_F8 ? (1.0f / 480.0f) * 256.0f : 1.0f;
}
inline int lm_format(int kind, int bits) {
  if (kind == MXK_KIND_INT) return bits == 1 ? LM_I1 : bits == 2 ? LM_I2 : bits == 4 ? LM_I4 : bits == 8 ? LM_I8 : 0;
  if (kind == MXK_KIND_FLOAT) return bits == 4 ? LM_F4 : bits == 8 ? LM_F8 : 0;
  return 0;
}
// Two codes of a format (layout of its width) as an f16 B-operand pair
template <int FMT>
__device__ __forceinline__ uint32_t lm_pair(uint32_t d) {
  if constexpr (FMT == LM_I4) return lm_i4pair(d);
  else if constexpr (FMT == LM_I8) return lm_i8pair(d);
  else if constexpr (FMT == LM_I2) return lm_i2pair(d);
  else if constexpr (FMT == LM_I1) return lm_i1pair(d);
  else return fp_code_pair_f16<lm_bits(FMT)>(d);
}

// v_perm_b32 selector: byte a of s1 into byte 0, byte b of s0 into byte 2, zeros in bytes 1 and 3
__host__ __device__ constexpr uint32_t lm_sel(int a, int b) {
  return (uint32_t)a | 0x0C00u | ((uint32_t)(4 + b) << 16) | 0x0C000000u;
}
// the same bytes into bytes 1 and 3 (FP8 codes at the top of each half), zeros in bytes 0 and 2
__host__ __device__ constexpr uint32_t lm_selh(int a, int b) {
  return 0x0Cu | ((uint32_t)a << 8) | 0x0C0000u | ((uint32_t)(4 + b) << 24);
}
// the byte-pair selector a format's pair decoder takes
template <int FMT>
__host__ __device__ constexpr uint32_t lm_sel_f(int a, int b) {
  return FMT == LM_F8 ? lm_selh(a, b) : lm_sel(a, b);
}

// p = x * s as f16 hi + lo for two elements: hi = RN16(x*s), lo =
// RN16(x*s - hi), each one v_fma_mix (fp32 product, f16 result), so
// |x*s - hi - lo| <= 2^-22 |x*s| (less for values whose lo is subnormal:
// at most 2^-25 absolute).
__device__ __forceinline__ void lm_split2(float x0, float s0, float x1, float s1, uint32_t& hi, uint32_t& lo) {
  uint32_t h, l;
  asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[0,0,0]" : "=v"(h) : "v"(x0), "v"(s0));
  asm("v_fma_mixhi_f16 %0, %1, %2, 0 op_sel_hi:[0,0,0]" : "+v"(h) : "v"(x1), "v"(s1));
  asm("v_fma_mixlo_f16 %0, %1, %2, -%3 op_sel_hi:[0,0,1]" : "=v"(l) : "v"(x0), "v"(s0), "v"(h));
  asm("v_fma_mixhi_f16 %0, %1, %2, -%3 op_sel:[0,0,1] op_sel_hi:[0,0,1]" : "+v"(l) : "v"(x1), "v"(s1), "v"(h));
  hi = h;
  lo = l;
}

// s_barrier after this wave's LDS stores are done; global loads still in
// flight (prefetches) stay in flight.
__device__ __forceinline__ void lm_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------- [K][N] stage decode
// Thread (r8 = tid / 16, c8 = tid % 16) decodes rows 8 r8 .. +7 and columns
// 8 c8 .. +7 of the stage: for column tile t the 8 codes of column 8 c8 + t,
// which are the B fragment of MFMA lane c8 + 16 (r8 % 4) in k step r8 / 4.
// A wave's threads are k step w, lanes 0..63 in order.
template <int BITS>
struct KnCodes {
  uint32_t w[BITS == 8 ? 16 : 8];
};

// `dead` is 0 or LM_OOB: every loader's byte offsets are or-ed with it, so
// that a load the caller does not need still issues (the compiler's wait
// counts then stay exact across loop iterations) and reads zeros.
template <int BITS>
__device__ __forceinline__ void kn_load(KnCodes<BITS>& c, __amdgpu_buffer_rsrc_t rw, int64_t k0, int64_t N,
                                        int64_t nb, int tid, uint32_t dead) {
  const int r8 = tid >> 4, c8 = tid & 15;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t row = k0 + 8 * r8 + i;
    if constexpr (BITS == 1) {
      c.w[i] = __builtin_amdgcn_raw_buffer_load_b8(rw, (int)((uint32_t)(row * (N / 8) + nb * 16 + c8) | dead), 0, 0);
    } else if constexpr (BITS == 2) {
      c.w[i] = __builtin_amdgcn_raw_buffer_load_b16(rw, (int)((uint32_t)(row * (N / 4) + nb * 32 + 2 * c8) | dead),
                                                    0, 0);
    } else if constexpr (BITS == 4) {
      c.w[i] = buf_load_b32(rw, (uint32_t)(row * (N / 2) + nb * 64 + 4 * c8) | dead, 0u);
    } else {
      const auto v =
          __builtin_amdgcn_raw_buffer_load_b64(rw, (int)((uint32_t)(row * N + nb * 128 + 8 * c8) | dead), 0, 0);
      c.w[2 * i] = v[0];
      c.w[2 * i + 1] = v[1];
    }
  }
}

// the B fragment of column tile t (column 8 c8 + t) from the thread's block
template <int FMT>
__device__ __forceinline__ u4v kn_frag(const KnCodes<lm_bits(FMT)>& c, int t) {
  constexpr int BITS = lm_bits(FMT);
  u4v f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if constexpr (BITS == 1) {
      // rows 2q and 2q+1 (8 bits each) 16 bits apart: column 8 c8 + t at bits t, 16 + t
      const uint32_t d = c.w[2 * q] | (c.w[2 * q + 1] << 16);
      f[q] = lm_pair<FMT>(d >> t);
    } else if constexpr (BITS == 2) {
      // rows 2q and 2q+1 (16 bits each) side by side: column 8 c8 + t at bits 2t, 2t + 1
      const uint32_t d = c.w[2 * q] | (c.w[2 * q + 1] << 16);
      f[q] = lm_pair<FMT>(d >> (2 * t));
    } else if constexpr (BITS == 4) {
      // byte t/2 of rows 2q and 2q+1: the low nibbles are column 8 c8 + t for even t
      const uint32_t d = __builtin_amdgcn_perm(c.w[2 * q + 1], c.w[2 * q], lm_sel(t >> 1, t >> 1));
      f[q] = lm_pair<FMT>((t & 1) ? d >> 4 : d);
    } else {
      const int h = t >> 2, u = t & 3;
      f[q] = lm_pair<FMT>(
          __builtin_amdgcn_perm(c.w[2 * (2 * q + 1) + h], c.w[2 * (2 * q) + h], lm_sel_f<FMT>(u, u)));
    }
  }
  return f;
}

template <int FMT>
__device__ __forceinline__ void kn_store(const KnCodes<lm_bits(FMT)>& c, uint8_t* sB, int tid) {
  const int ks = tid >> 6, lane = tid & 63;
#pragma unroll
  for (int t = 0; t < 8; ++t) *reinterpret_cast<u4v*>(sB + lm_frag_off(ks, t, lane)) = kn_frag<FMT>(c, t);
}

// The same 8 x 8 blocks from the tiled copy of mxk_linear_prepack_weight:
// chunk (nb, 32-row step) of 2 KiB, whose lane c8 + 16 (r8 % 4) holds the
// block as two 16-byte pieces (at +16 L and +1024 + 16 L).  Word 2p + e,
// byte q is the byte of columns 8 c8 + 2p, +1 of row 4e + {0,2,1,3}[q], so
// rows 2q', 2q'+1 of column pair p sit at bits 0-7 and 16-23 of word
// 2p + q'/2 shifted right by 8 (q' % 2): no byte permutes.
struct KnTiled {
  u4v w[2];
};

__device__ __forceinline__ void kn_load_tiled(KnTiled& c, __amdgpu_buffer_rsrc_t rw, int64_t k0, int64_t K,
                                              int64_t nb, int tid, uint32_t dead) {
  const int r8 = tid >> 4, c8 = tid & 15;
  const int64_t chunk = nb * (K / 32) + (k0 + 8 * r8) / 32;
  const uint32_t off = (uint32_t)(chunk * 2048 + 16 * (c8 + 16 * (r8 & 3))) | dead;
  c.w[0] = buf_load_b128(rw, off, 0u);
  c.w[1] = buf_load_b128(rw, off + 1024u, 0u);
}

template <int FMT>
__device__ __forceinline__ u4v kn_frag_tiled(const KnTiled& c, int t) {
  const uint32_t o[8] = {c.w[0][0], c.w[0][1], c.w[0][2], c.w[0][3], c.w[1][0], c.w[1][1], c.w[1][2], c.w[1][3]};
  const int p = t >> 1;
  u4v f;
#pragma unroll
  for (int q = 0; q < 4; ++q) f[q] = lm_pair<FMT>(o[2 * p + (q >> 1)] >> (8 * (q & 1) + 4 * (t & 1)));
  return f;
}

template <int FMT>
__device__ __forceinline__ void kn_store_tiled(const KnTiled& c, uint8_t* sB, int tid) {
  const int ks = tid >> 6, lane = tid & 63;
#pragma unroll
  for (int t = 0; t < 8; ++t) *reinterpret_cast<u4v*>(sB + lm_frag_off(ks, t, lane)) = kn_frag_tiled<FMT>(c, t);
}

// ---------------------------------------------------------------- [N][K] stage decode
// int4: lanes 8a .. 8a+7 read the 128-byte line of one column (k steps
// 0..7 of the stage, 16 bytes each); each 16 bytes are the four k octets of
// MFMA lanes j + 16 v.  The local column of pair index p = tid / 8 + 64 h is
// 16 (p / 16) + 8 (p % 2) + (p / 2) % 8, so the two columns of a 16-lane
// store group share a tile and differ in j (no bank conflicts).
// int8: 16 lanes read one column's 256 bytes; 16 bytes are two k octets.
// int2: 4 lanes read one column's 64 bytes, each 16 bytes two k steps; the
// 4 columns of a 16-lane store group share a tile and differ in j.
// int1: the same lanes and columns as int2, 8 bytes (two k steps) each.
template <int BITS>
struct NkCodes {
  u4v w[BITS == 4 ? 2 : BITS == 8 ? 4 : 1];
};

__device__ __forceinline__ int nk4_col(int p) { return 16 * (p >> 4) + 8 * (p & 1) + ((p >> 1) & 7); }
__device__ __forceinline__ int nk2_col(int p) { return ((p >> 4) & 7) + 8 * (p & 15); }

template <int BITS>
__device__ __forceinline__ void nk_load(NkCodes<BITS>& c, __amdgpu_buffer_rsrc_t rw, int64_t k0, int64_t K,
                                        int64_t nb, int tid, uint32_t dead) {
  if constexpr (BITS == 1) {
    const int64_t n = nb * 128 + nk2_col(tid >> 2);
    const auto v =
        __builtin_amdgcn_raw_buffer_load_b64(rw, (int)((uint32_t)(n * (K / 8) + k0 / 8 + 8 * (tid & 3)) | dead), 0, 0);
    c.w[0][0] = v[0];
    c.w[0][1] = v[1];
  } else if constexpr (BITS == 2) {
    const int64_t n = nb * 128 + nk2_col(tid >> 2);
    c.w[0] = buf_load_b128(rw, (uint32_t)(n * (K / 4) + k0 / 4 + 16 * (tid & 3)) | dead, 0u);
  } else if constexpr (BITS == 4) {
    const int q = tid & 7;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t n = nb * 128 + nk4_col((tid >> 3) + 64 * h);
      c.w[h] = buf_load_b128(rw, (uint32_t)(n * (K / 2) + k0 / 2 + 16 * q) | dead, 0u);
    }
  } else {
    const int h8 = tid & 15;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int64_t n = nb * 128 + (tid >> 4) + 32 * h;
      c.w[h] = buf_load_b128(rw, (uint32_t)(n * K + k0 + 16 * h8) | dead, 0u);
    }
  }
}

template <int FMT>
__device__ __forceinline__ void nk_store(const NkCodes<lm_bits(FMT)>& c, uint8_t* sB, int tid) {
  constexpr int BITS = lm_bits(FMT);
  if constexpr (BITS == 1) {
    // k step 2q + s is dword s, octet v its byte v.  Byte v of wd beside
    // byte v of wd >> 1 holds codes (0, 1) at bits 0 and 16, (2p, 2p + 1)
    // 2p bits higher.
    const int q = tid & 3, col = nk2_col(tid >> 2);
    const int t = col & 7, j = col >> 3;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const uint32_t wd = c.w[0][s], sh = wd >> 1;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint32_t d = __builtin_amdgcn_perm(sh, wd, lm_sel(v, v));
        u4v f;
#pragma unroll
        for (int p = 0; p < 4; ++p) f[p] = lm_pair<FMT>(d >> (2 * p));
        *reinterpret_cast<u4v*>(sB + lm_frag_off(2 * q + s, t, j + 16 * v)) = f;
      }
    }
  } else if constexpr (BITS == 2) {
    // k step 2q + s is dwords 2s, 2s+1; octet v is bytes 2 (v & 1), +1 of
    // dword 2s + v / 2.  Byte b of wd beside byte b of wd >> 2 holds the
    // codes (0, 1) at bits 0-1 and 16-17, and (2, 3) four bits higher.
    const int q = tid & 3, col = nk2_col(tid >> 2);
    const int t = col & 7, j = col >> 3;
#pragma unroll
    for (int sv = 0; sv < 4; ++sv) {
      const uint32_t wd = c.w[0][sv], sh = wd >> 2;
#pragma unroll
      for (int vl = 0; vl < 2; ++vl) {
        u4v f;
#pragma unroll
        for (int bb = 0; bb < 2; ++bb) {
          const uint32_t d = __builtin_amdgcn_perm(sh, wd, lm_sel(2 * vl + bb, 2 * vl + bb));
          f[2 * bb] = lm_pair<FMT>(d);
          f[2 * bb + 1] = lm_pair<FMT>(d >> 4);
        }
        *reinterpret_cast<u4v*>(sB + lm_frag_off(2 * q + (sv >> 1), t, j + 16 * (2 * (sv & 1) + vl))) = f;
      }
    }
  } else if constexpr (BITS == 4) {
    const int ks = tid & 7;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int col = nk4_col((tid >> 3) + 64 * h);
      const int t = col & 7, j = col >> 3;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint32_t lo4 = c.w[h][v] & 0x0F0F0F0Fu, hi4 = (c.w[h][v] >> 4) & 0x0F0F0F0Fu;
        u4v f;
#pragma unroll
        for (int p = 0; p < 4; ++p) f[p] = lm_pair<FMT>(__builtin_amdgcn_perm(hi4, lo4, lm_sel(p, p)));
        *reinterpret_cast<u4v*>(sB + lm_frag_off(ks, t, j + 16 * v)) = f;
      }
    }
  } else {
    const int h8 = tid & 15, ks = h8 >> 1;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int col = (tid >> 4) + 32 * h;
      const int t = col & 7, j = col >> 3;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int g = 2 * (h8 & 1) + e;
        u4v f;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const uint32_t wd = c.w[h][2 * e + (p >> 1)];
          const int b = 2 * (p & 1);
          f[p] = lm_pair<FMT>(__builtin_amdgcn_perm(wd, wd, lm_sel_f<FMT>(b, b + 1)));
        }
        *reinterpret_cast<u4v*>(sB + lm_frag_off(ks, t, j + 16 * g)) = f;
      }
    }
  }
}

// [N][K] int4 codes from the tiled copy of k_tile_w4t: the 16-byte unit of
// row n and K segment k .. k + 31 (k = 32 q within a block of 128) sits at
// ((n / 16) * K/128 + k / 128) * 1024 + 16 * (n % 16 + 16 * (k % 128) / 32),
// and word 2 sp + h, byte b of a unit holds the codes (8 st + i) with
// st = 2 sp (low nibble) and 2 sp + 1 (high nibble), i = 4 h + {0, 2, 1, 3}[b].
__device__ __forceinline__ void nk_load_tiled(NkCodes<4>& c, __amdgpu_buffer_rsrc_t rw, int64_t k0, int64_t K,
                                              int64_t nb, int tid, uint32_t dead) {
  const int q = tid & 7;
  const int64_t k = k0 + 32 * q, KB = K / 128;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t n = nb * 128 + nk4_col((tid >> 3) + 64 * h);
    c.w[h] = buf_load_b128(
        rw, (uint32_t)(((n >> 4) * KB + (k >> 7)) * 1024 + 16 * ((n & 15) + 16 * ((k >> 5) & 3))) | dead, 0u);
  }
}

// nk_store's fragments from tiled units: the pair (i, i + 1) of step st is
// (word 2 (st / 2) + i / 4) >> (8 ((i / 2) & 1) + 4 (st & 1)) under the mask
// of lm_i4pair
__device__ __forceinline__ void nk_store_tiled(const NkCodes<4>& c, uint8_t* sB, int tid) {
  const int ks = tid & 7;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int col = nk4_col((tid >> 3) + 64 * h);
    const int t = col & 7, j = col >> 3;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      u4v f;
#pragma unroll
      for (int p = 0; p < 4; ++p) f[p] = lm_i4pair(c.w[h][2 * (v >> 1) + (p >> 1)] >> (8 * (p & 1) + 4 * (v & 1)));
      *reinterpret_cast<u4v*>(sB + lm_frag_off(ks, t, j + 16 * v)) = f;
    }
  }
}

// x' (and its f16 hi / lo) in HBM as tiles of 16 rows x 8 columns of K,
// tile (m / 16, k / 8) at element ((m / 16) * Kp/8 + k / 8) * 128 and
// element (m % 16) * 8 + k % 8 inside it, so that the 64 lanes of an A
// operand load (rows j of a row tile, columns 8 g .. 8 g + 7 of a k step)
// read one contiguous 2 KiB (fp32) or 1 KiB (f16): with x' row-major the 16
// rows of one load are Kp elements apart and land on one memory channel.
__host__ __device__ __forceinline__ int64_t lm_xoff(int64_t m, int64_t k, int64_t Kp) {
  return ((m >> 4) * (Kp >> 3) + (k >> 3)) * 128 + (m & 15) * 8 + (k & 7);
}
// rows of x' the tiled layout holds (whole row tiles)
__host__ __device__ __forceinline__ int64_t lm_rows16(int64_t M) { return (M + 15) & ~(int64_t)15; }

// ---------------------------------------------------------------- the MFMA kernel
// A-operand registers of one k step: [K][N] x' (2 row tiles x 8 fp32) and
// 8 scales; [N][K] hi and lo (2 row tiles x 8 f16 each)
struct KnA {
  u4v x[2][2];
  u4v s[2];
};
struct NkA {
  u4v h[2];
  u4v l[2];
};

template <int FMT, int WM, bool NK, bool TILED = false>
__global__ __launch_bounds__(LM_THREADS, 1) void k_linear_mfma(
    const float* __restrict__ xs,        // [K][N]: x' [M][Kp] fp32
    const _Float16* __restrict__ xh,     // [N][K]: hi of x' [M][Kp]
    const _Float16* __restrict__ xl,     // [N][K]: lo of x' [M][Kp]
    const float* __restrict__ sc,        // [K][N]: block-major scales [NB][K]; [N][K]: [KB][N] or [N][KB]
    int sc_kb_major, const int* __restrict__ ex, const int* __restrict__ es, const uint8_t* __restrict__ w,
    int M, int64_t K, int64_t Kp, int64_t N, int sps, const float* __restrict__ bias, float* __restrict__ out,
    float* __restrict__ part) {
  constexpr int BITS = lm_bits(FMT), WK = 8 / WM, KPW = 8 / WK;
  using A = typename std::conditional<NK, NkA, KnA>::type;
  static_assert(!TILED || FMT == LM_I4 || (FMT == LM_F4 && !NK), "the tiled copies hold int4 (or [K][N] FP4) codes");
  using Codes = typename std::conditional<NK, NkCodes<BITS>,
                                          typename std::conditional<TILED, KnTiled, KnCodes<BITS>>::type>::type;
  __shared__ __attribute__((aligned(1024))) uint8_t sB[2 * LM_STAGE_BYTES];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WM, wk = wave / WM;
  const int j = lane & 15, g = lane >> 4;
  const int64_t nb = blockIdx.x, NB = N / 128, KB = K / 128;
  const int64_t m0 = (int64_t)blockIdx.y * (32 * WM);
  const int z = blockIdx.z;
  const int nst = (int)(Kp / LM_STAGE);
  const int st0 = z * sps, st1 = min(st0 + sps, nst);
  // whole row tiles: x' rows past M (within the last tile) hold anything,
  // and only their own output rows, never stored, see them
  const int rows = lm_rows16((int64_t)M - m0) < 32 * WM ? (int)lm_rows16((int64_t)M - m0) : 32 * WM;
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)(K * N * BITS / 8));

  // A-operand loads of k step (st, jj): rows 32 wm + 16 i + j, columns
  // kg + 8 g .. +7 (rows past M read zeros)
  __amdgpu_buffer_rsrc_t ra, rb;
  if constexpr (NK) {
    ra = make_rsrc(xh + m0 * Kp, (uint32_t)(rows * Kp * 2));
    rb = make_rsrc(xl + m0 * Kp, (uint32_t)(rows * Kp * 2));
  } else {
    ra = make_rsrc(xs + m0 * Kp, (uint32_t)(rows * Kp * 4));
    rb = make_rsrc(sc + nb * K, (uint32_t)(K * 4));  // scales past K read zeros
  }
  // [K][N]: the block's scales go to the binade of 2^13 by 2^es (the
  // largest in [2^13, 2^14), from the row prepass); the epilogue, or the
  // split reduction, takes 2^-es back out
  const int es_nb = NK ? 0 : es[nb];
  // Loads are issued whether or not their data is needed (`live` false:
  // every offset past its buffer, zeros come back), so that the number of
  // loads per step is fixed and the compiler's wait counts stay exact; with
  // conditional loads it waited for every load in flight at each step.  A
  // dead A operand is all zeros, so a dead step adds exact zeros.
  auto load_a = [&](A& a, int st, int jj, bool live) {
    const uint32_t dead = live ? 0u : LM_OOB;
    const int64_t kg = (int64_t)st * LM_STAGE + 32 * (wk + WK * jj) + 8 * g;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int64_t at = lm_xoff(32 * wm + 16 * i + j, kg, Kp);
      if constexpr (NK) {
        a.h[i] = buf_load_b128(ra, (uint32_t)(at * 2) | dead, 0u);
        a.l[i] = buf_load_b128(rb, (uint32_t)(at * 2) | dead, 0u);
      } else {
        a.x[i][0] = buf_load_b128(ra, (uint32_t)(at * 4) | dead, 0u);
        a.x[i][1] = buf_load_b128(ra, (uint32_t)(at * 4 + 16) | dead, 0u);
      }
    }
    if constexpr (!NK) {
      a.s[0] = buf_load_b128(rb, (uint32_t)(kg * 4) | dead, 0u);
      a.s[1] = buf_load_b128(rb, (uint32_t)(kg * 4 + 16) | dead, 0u);
    }
  };
  auto load_codes = [&](Codes& c, int st, bool live) {
    const uint32_t dead = live ? 0u : LM_OOB;
    if constexpr (NK && TILED) nk_load_tiled(c, rw, (int64_t)st * LM_STAGE, K, nb, tid, dead);
    else if constexpr (NK) nk_load<BITS>(c, rw, (int64_t)st * LM_STAGE, K, nb, tid, dead);
    else if constexpr (TILED) kn_load_tiled(c, rw, (int64_t)st * LM_STAGE, K, nb, tid, dead);
    else kn_load<BITS>(c, rw, (int64_t)st * LM_STAGE, N, nb, tid, dead);
  };
  auto store_codes = [&](const Codes& c, uint8_t* dst) {
    if constexpr (NK && TILED) nk_store_tiled(c, dst, tid);
    else if constexpr (NK) nk_store<FMT>(c, dst, tid);
    else if constexpr (TILED) kn_store_tiled<FMT>(c, dst, tid);
    else kn_store<FMT>(c, dst, tid);
  };

  f4v acc[2][8], P[2][8];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      acc[i][t] = f4v{0.f, 0.f, 0.f, 0.f};
      P[i][t] = f4v{0.f, 0.f, 0.f, 0.f};
    }

  // [N][K] scales of block kb for this lane's 8 columns (8 j .. 8 j + 7 of the block)
  const __amdgpu_buffer_rsrc_t rsc = make_rsrc(sc, (uint32_t)(NK ? N * KB * 4 : 4));
  auto block_scales = [&](int64_t kb, float (&s8)[8]) {
    const int64_t n0 = nb * 128 + 8 * j;
    if (kb >= KB) {
#pragma unroll
      for (int t = 0; t < 8; ++t) s8[t] = 0.0f;
    } else if (sc_kb_major) {
      const u4v a0 = buf_load_b128(rsc, (uint32_t)((kb * N + n0) * 4), 0u);
      const u4v a1 = buf_load_b128(rsc, (uint32_t)((kb * N + n0) * 4 + 16), 0u);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        s8[u] = __uint_as_float(a0[u]);
        s8[4 + u] = __uint_as_float(a1[u]);
      }
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) s8[t] = __uint_as_float(buf_load_b32(rsc, (uint32_t)(((n0 + t) * KB + kb) * 4), 0u));
    }
  };
  // fold the block sums into acc with the block's scale of each column
  // (blocks past K: padding rows, P holds exact zeros and s8 zeros)
  auto fold = [&](const float (&s8)[8]) {
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          acc[i][t][r] = __builtin_fmaf(P[i][t][r], s8[t], acc[i][t][r]);
          P[i][t][r] = 0.0f;
        }
  };

  auto build = [&](const A& a, h8v (&ahi)[2], h8v (&alo)[2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if constexpr (NK) {
        ahi[i] = __builtin_bit_cast(h8v, a.h[i]);
        alo[i] = __builtin_bit_cast(h8v, a.l[i]);
      } else {
        u4v hv, lv;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int e = 2 * q;
          const float x0 = __uint_as_float(a.x[i][e >> 2][e & 3]), x1 = __uint_as_float(a.x[i][e >> 2][(e & 3) + 1]);
          const float s0 = __builtin_ldexpf(__uint_as_float(a.s[e >> 2][e & 3]), es_nb);
          const float s1 = __builtin_ldexpf(__uint_as_float(a.s[e >> 2][(e & 3) + 1]), es_nb);
          uint32_t hh, ll;
          lm_split2(x0, s0, x1, s1, hh, ll);
          hv[q] = hh;
          lv[q] = ll;
        }
        ahi[i] = __builtin_bit_cast(h8v, hv);
        alo[i] = __builtin_bit_cast(h8v, lv);
      }
    }
  };
  // column tiles T0 .. T0 + NT - 1
  auto mfmas = [&](const h8v (&ahi)[2], const h8v (&alo)[2], const h8v* bt, int T0, int NT) {
#pragma unroll
    for (int u = 0; u < NT; ++u)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        f4v& d = NK ? P[i][T0 + u] : acc[i][T0 + u];
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[i], bt[u], d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[i], bt[u], d, 0, 0, 0);
      }
  };

  // Per k step: request the next step's A operands (a whole step ahead)
  // and this step's 8 B fragments, then build A and run the 32 MFMAs.  The
  // scheduling barriers keep every request at the top of its step.
  // A operands of this wave's k step gs (0 .. nsteps-1 over the split)
  const int nsteps = (st1 - st0) * KPW;
  auto load_step = [&](A& a, int gs) { load_a(a, st0 + gs / KPW, gs % KPW, gs < nsteps); };
  // One row tile ([K][N], WM = 1): wave w runs k step w of every stage, and
  // the fragments its lanes decode are exactly the ones they feed to the
  // MFMAs, so the codes skip LDS (and every barrier): each wave keeps DS
  // stages of its codes in flight in registers.
  constexpr bool DIRECT = !NK && WM == 1;
  constexpr int DS = BITS == 8 ? 2 : 4;
  if constexpr (DIRECT) {
   if (st0 < st1) {
    Codes cq[DS];
    A ar[2];
#pragma unroll
    for (int i = 0; i < DS; ++i) load_codes(cq[i], st0 + i, st0 + i < st1);
    load_step(ar[0], 0);
    load_step(ar[1], 1);
    // whole groups of DS stages: the steps past st1 in the last group run
    // on zero A operands
    for (int sb = st0; sb < st1; sb += DS) {
#pragma unroll
      for (int i = 0; i < DS; ++i) {
        const int st = sb + i;
        const int gs = st - st0, p = i & 1;  // DS is even, so gs % 2 = i % 2
        h8v bt[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          if constexpr (TILED) bt[t] = __builtin_bit_cast(h8v, kn_frag_tiled<FMT>(cq[i], t));
          else bt[t] = __builtin_bit_cast(h8v, kn_frag<FMT>(cq[i], t));
        }
        load_codes(cq[i], st + DS, st + DS < st1);
        h8v ahi[2], alo[2];
        build(ar[p], ahi, alo);
        load_step(ar[p], gs + 2);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(ahi, alo, bt, 0, 8);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
   }
  } else if (st0 < st1) {
    Codes cc;
    A ar[2];
    float s8[8];
    load_codes(cc, st0, true);
    load_step(ar[0], 0);
    load_step(ar[1], 1);
    store_codes(cc, sB);
    lm_barrier();
    for (int st = st0; st < st1; ++st) {
      const int buf = (st - st0) & 1;
      const bool more = st + 1 < st1;
      load_codes(cc, st + 1, more);
      const uint8_t* b = sB + buf * LM_STAGE_BYTES;
#pragma unroll
      for (int jj = 0; jj < KPW; ++jj) {
        // slot p holds step gs, the other slot step gs + 1 (KPW even: p = gs % 2)
        const int p = (KPW & 1) ? 0 : (jj & 1), ks = wk + WK * jj;
        const int gs = (st - st0) * KPW + jj;
        // [N][K]: this wave's k steps of block kb = 2 st + ks / 4 start here
        // / end here (ks = wk + WK jj with wk < WK and WK dividing 4 or
        // equal to 8, so a block starts at jj where WK jj is a multiple of 4)
        const bool kb_first = jj == 0 || (ks >> 2) != ((ks - WK) >> 2);
        const bool kb_last = jj + 1 == KPW || (ks >> 2) != ((ks + WK) >> 2);
        if (NK && kb_first) block_scales(2 * (int64_t)st + (ks >> 2), s8);
        // [N][K] (two accumulator sets) reads its fragments in two halves
        constexpr int BT = NK ? 4 : 8;
        h8v bt[BT];
#pragma unroll
        for (int t = 0; t < BT; ++t) bt[t] = *reinterpret_cast<const h8v*>(b + lm_frag_off(ks, t, lane));
        h8v ahi[2], alo[2];
        build(ar[p], ahi, alo);
        // slot p is free: step gs + 2 goes there, about two steps ahead of its use
        if constexpr ((KPW & 1) != 0) {
          ar[0] = ar[1];
          load_step(ar[1], gs + 2);
        } else {
          load_step(ar[p], gs + 2);
        }
        __builtin_amdgcn_sched_barrier(0);
        mfmas(ahi, alo, bt, 0, BT);
        if constexpr (NK) {
#pragma unroll
          for (int t = 0; t < 4; ++t) bt[t] = *reinterpret_cast<const h8v*>(b + lm_frag_off(ks, 4 + t, lane));
          mfmas(ahi, alo, bt, 4, 4);
          if (kb_last) fold(s8);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (more) store_codes(cc, sB + (buf ^ 1) * LM_STAGE_BYTES);
      lm_barrier();
    }
  }

  // ---- waves that split K meet in LDS, in wk order (the stage buffers are
  // free: every wave has passed the barrier after its last fragment reads)
  if constexpr (WK > 1) {
    f4v* red = reinterpret_cast<f4v*>(sB);
    if (wk > 0) {
      f4v* slot = red + (size_t)(wm * (WK - 1) + wk - 1) * 16 * 64;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int t = 0; t < 8; ++t) slot[(i * 8 + t) * 64 + lane] = acc[i][t];
    }
    lm_barrier();
    if (wk > 0) return;
#pragma unroll 1
    for (int u = 1; u < WK; ++u) {
      const f4v* slot = red + (size_t)(wm * (WK - 1) + u - 1) * 16 * 64;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const f4v v = slot[(i * 8 + t) * 64 + lane];
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][t][r] += v[r];
        }
    }
  }

  // ---- store: rows 4 g + r of row tile i, columns 128 nb + 8 j + t
  const int64_t n0 = nb * 128 + 8 * j;
  float bv[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) bv[t] = (bias && !part) ? bias[n0 + t] : 0.0f;
  const int esb = part ? 0 : es_nb;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t m = m0 + 32 * wm + 16 * i + 4 * g + r;
      if (m >= M) continue;
      float v[8];
      if (part) {
#pragma unroll
        for (int t = 0; t < 8; ++t) v[t] = acc[i][t][r];
        float* dst = part + ((int64_t)z * M + m) * N + n0;
        *reinterpret_cast<f4v*>(dst) = f4v{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<f4v*>(dst + 4) = f4v{v[4], v[5], v[6], v[7]};
      } else {
        const int e = -(ex[m] + esb);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          if constexpr (lm_post(FMT) != 1.0f) v[t] = __builtin_ldexpf(acc[i][t][r], e) * lm_post(FMT) + bv[t];
          else v[t] = __builtin_ldexpf(acc[i][t][r], e) + bv[t];
        }
        float* dst = out + m * N + n0;
        *reinterpret_cast<f4v*>(dst) = f4v{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<f4v*>(dst + 4) = f4v{v[4], v[5], v[6], v[7]};
      }
    }
}

// y = 2^-(ex[m] + es[n / 128]) * sum over the S splits in order * post (+ bias)
__global__ __launch_bounds__(256) void k_linear_mfma_reduce(const float* __restrict__ part, int S, int64_t M,
                                                            int64_t N, const int* __restrict__ ex,
                                                            const int* __restrict__ es, const float* __restrict__ bias,
                                                            float post, float* __restrict__ out) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;  // float4 index
  if (q >= M * N / 4) return;
  const int64_t m = (4 * q) / N, n = (4 * q) % N;
  f4v s = *reinterpret_cast<const f4v*>(part + 4 * q);
  for (int z = 1; z < S; ++z) {
    const f4v v = *reinterpret_cast<const f4v*>(part + (int64_t)z * M * N + 4 * q);
#pragma unroll
    for (int r = 0; r < 4; ++r) s[r] += v[r];
  }
  const int e = -(ex[m] + (es ? es[n / 128] : 0));
  f4v y;
#pragma unroll
  for (int r = 0; r < 4; ++r) y[r] = __builtin_ldexpf(s[r], e) * post + (bias ? bias[n + r] : 0.0f);
  *reinterpret_cast<f4v*>(out + 4 * q) = y;
}

// ---------------------------------------------------------------- prepasses
// Row m of x: ex[m] such that its largest |x| times 2^ex lies in [1, 2)
// (0 for a zero row), and x * 2^ex zero-padded to Kp columns, as fp32
// (SPLIT false) or as f16 hi + lo (SPLIT true: hi = RN16(v), lo = RN16(v - hi),
// v - hi exact in fp32).  VEC: 16-byte rows (K * sizeof(T) % 16 == 0, x
// 16-byte aligned); rows of up to 2048 16-byte chunks stay in registers
// between the maximum and the scaled copy, longer ones are read twice.
template <typename T, bool SPLIT>
__device__ __forceinline__ void lm_put(float* __restrict__ xs, _Float16* __restrict__ xh, _Float16* __restrict__ xl,
                                       int64_t at, float v) {
  if constexpr (SPLIT) {
    const _Float16 h = (_Float16)v;
    xh[at] = h;
    xl[at] = (_Float16)(v - (float)h);
  } else {
    xs[at] = v;
  }
}

//
// Workgroups M .. M + NB - 1 (the [K][N] product) find es[nb] instead: the
// power of two that puts the largest |scale| of column block nb (row nb of
// the block-major scales sT [NB][K]) in [2^13, 2^14), 0 for a zero or
// non-finite maximum.  It depends on the weight alone; computed here, it is
// ready before the main kernel starts.
template <typename T, bool SPLIT, bool VEC>
__global__ __launch_bounds__(256) void k_linear_mfma_prep_rows(const T* __restrict__ x, int64_t M, int64_t K,
                                                               int64_t Kp, float* __restrict__ xs,
                                                               _Float16* __restrict__ xh, _Float16* __restrict__ xl,
                                                               int* __restrict__ ex, const float* __restrict__ sT,
                                                               int* __restrict__ es) {
  constexpr int E = 16 / (int)sizeof(T), NCH = 8;
  __shared__ float red[4];
  const int tid = threadIdx.x;
  if ((int64_t)blockIdx.x >= M) {
    const int64_t nb = (int64_t)blockIdx.x - M;
    const float* s = sT + nb * K;
    float mx = 0.0f;
    int64_t k = tid;
    for (; k + 7 * 256 < K; k += 8 * 256) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = s[k + 256 * u];
#pragma unroll
      for (int u = 0; u < 8; ++u) mx = fmaxf(mx, __builtin_fabsf(v[u]));
    }
    for (; k < K; k += 256) mx = fmaxf(mx, __builtin_fabsf(s[k]));
    mx = group_max<64>(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    if (tid == 0) {
      mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
      const int be = (int)((__float_as_uint(mx) >> 23) & 0xFFu);
      es[nb] = (be == 0xFF || mx == 0.0f) ? 0 : 140 - (be == 0 ? 1 : be);
    }
    return;
  }
  const int64_t m = blockIdx.x;
  const T* row = x + m * K;
  const int64_t nch = K / E;
  const bool cached = VEC && nch <= (int64_t)NCH * 256;
  u4v c[NCH];
  auto elems = [&](const u4v& w, float (&v)[E]) {
    const T* t = reinterpret_cast<const T*>(&w);
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = ElemT<T>::cvt(t[e]);
  };
  float mx = 0.0f;
  if (cached) {
#pragma unroll
    for (int q = 0; q < NCH; ++q) {
      const int64_t ch = tid + 256 * q;
      c[q] = ch < nch ? *reinterpret_cast<const u4v*>(row + ch * E) : u4v{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int q = 0; q < NCH; ++q) {
      float v[E];
      elems(c[q], v);
#pragma unroll
      for (int e = 0; e < E; ++e) mx = fmaxf(mx, __builtin_fabsf(v[e]));
    }
  } else {
    for (int64_t k = tid; k < K; k += 256) mx = fmaxf(mx, __builtin_fabsf(ElemT<T>::cvt(row[k])));
  }
  mx = group_max<64>(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const int be = (int)((__float_as_uint(mx) >> 23) & 0xFFu);
  const int e = (be == 0xFF || mx == 0.0f) ? 0 : 127 - (be == 0 ? 1 : be);
  if (tid == 0) ex[m] = e;
  if (cached) {
#pragma unroll
    for (int q = 0; q < NCH; ++q) {
      const int64_t ch = tid + 256 * q;
      if (ch >= nch) break;
      float v[E];
      elems(c[q], v);
#pragma unroll
      for (int u = 0; u < E; ++u) v[u] = __builtin_ldexpf(v[u], e);
      const int64_t at = lm_xoff(m, ch * E, Kp);  // E <= 8 values within one 8-column group
      if constexpr (SPLIT) {
        _Float16 h[E], l[E];
#pragma unroll
        for (int u = 0; u < E; ++u) {
          h[u] = (_Float16)v[u];
          l[u] = (_Float16)(v[u] - (float)h[u]);
        }
        if constexpr (E == 4) {
          *reinterpret_cast<u2v*>(xh + at) = __builtin_bit_cast(u2v, h);
          *reinterpret_cast<u2v*>(xl + at) = __builtin_bit_cast(u2v, l);
        } else {
          *reinterpret_cast<u4v*>(xh + at) = __builtin_bit_cast(u4v, h);
          *reinterpret_cast<u4v*>(xl + at) = __builtin_bit_cast(u4v, l);
        }
      } else {
#pragma unroll
        for (int u = 0; u < E; u += 4) *reinterpret_cast<f4v*>(xs + at + u) = f4v{v[u], v[u + 1], v[u + 2], v[u + 3]};
      }
    }
    for (int64_t k = K + tid; k < Kp; k += 256) lm_put<T, SPLIT>(xs, xh, xl, lm_xoff(m, k, Kp), 0.0f);
  } else {
    for (int64_t k = tid; k < Kp; k += 256)
      lm_put<T, SPLIT>(xs, xh, xl, lm_xoff(m, k, Kp), k < K ? __builtin_ldexpf(ElemT<T>::cvt(row[k]), e) : 0.0f);
  }
}

// Block-major copy sT[nb][k] = s[k][nb] of a [K][N] weight's scales (when
// the caller has none)
__global__ __launch_bounds__(256) void k_linear_mfma_scales_t(const float* __restrict__ s, int64_t K, int64_t NB,
                                                              float* __restrict__ sT) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= K * NB) return;
  const int64_t nb = i / K, k = i % K;
  sT[i] = s[k * NB + nb];
}

// ---------------------------------------------------------------- plan
struct LmPlan {
  int wm = 0, S = 1, sps = 0;
  int64_t Kp = 0;
  size_t off_ex = 0, off_es = 0, off_x = 0, off_s = 0, off_p = 0, bytes = 0;
};

inline size_t lm_round(size_t v) { return (v + 255) & ~(size_t)255; }

// Largest row tile (WM) per kernel: the [N][K] kernel holds a second set of
// accumulators (the block sums), so its wider tiles would spill registers.
constexpr int lm_max_wm(bool nk, int bits) { return nk ? (bits == 8 ? 2 : 4) : 8; }

// Row tile: the largest WM (32 WM rows) that still gives every CU a
// workgroup; when none does, the fewest row tiles, and K splits across
// workgroups to fill the CUs.
LmPlan lm_plan(int64_t M, int64_t K, int64_t N, bool nk, int bits) {
  LmPlan p;
  p.Kp = ceil_div(K, LM_STAGE) * LM_STAGE;
  const int nst = (int)(p.Kp / LM_STAGE);
  const int64_t NB = N / 128, target = num_cus();
  const int64_t m32 = ceil_div(M, 32);
  int wm = 1;
  while (wm < lm_max_wm(nk, bits) && wm * 2 <= m32) wm *= 2;
  int pick = 0;
  for (int c = wm; c >= 1; c /= 2)
    if (NB * ceil_div(M, 32 * c) >= target) {
      pick = c;
      break;
    }
  int S = 1;
  if (pick) {
    wm = pick;
  } else {
    S = (int)std::min<int64_t>(nst, ceil_div(target, NB * ceil_div(M, 32 * wm)));
  }
  p.wm = wm;
  p.sps = (int)ceil_div(nst, S);
  p.S = (int)ceil_div(nst, p.sps);
  size_t o = LM_WS_BASE;
  p.off_ex = o;
  o += lm_round((size_t)M * 4);
  p.off_es = o;
  o += lm_round((size_t)NB * 4);
  p.off_x = o;
  o += lm_round((size_t)lm_rows16(M) * (size_t)p.Kp * 4);  // fp32 x', or f16 hi + lo, in whole row tiles
  p.off_s = o;  // [K][N]: room for a block-major copy of the scales when the caller has none
  if (!nk) o += lm_round((size_t)NB * (size_t)K * 4);
  p.off_p = o;
  if (p.S > 1) o += lm_round((size_t)p.S * (size_t)M * (size_t)N * 4);
  p.bytes = o;
  return p;
}

template <int FMT, int WM, bool NK, bool TILED>
void lm_launch_t(const LmPlan& p, hipStream_t st, const float* xs, const _Float16* xh, const _Float16* xl,
                 const float* sc, int sc_kbm, const int* ex, const int* es, const uint8_t* w, int64_t M, int64_t K,
                 int64_t N, const float* bias, float* out, float* part) {
  const dim3 grid((unsigned)(N / 128), (unsigned)ceil_div(M, 32 * WM), (unsigned)p.S);
  hipLaunchKernelGGL((k_linear_mfma<FMT, WM, NK, TILED>), grid, dim3(LM_THREADS), 0, st, xs, xh, xl, sc, sc_kbm, ex,
                     es, w, (int)M, K, p.Kp, N, p.sps, bias, out, p.S > 1 ? part : nullptr);
}

template <int FMT, bool NK, bool TILED = false>
void lm_launch_w(const LmPlan& p, hipStream_t st, const float* xs, const _Float16* xh, const _Float16* xl,
                 const float* sc, int sc_kbm, const int* ex, const int* es, const uint8_t* w, int64_t M, int64_t K,
                 int64_t N, const float* bias, float* out, float* part) {
  constexpr int MW = lm_max_wm(NK, lm_bits(FMT));
  switch (p.wm) {
    case 8:
      lm_launch_t<FMT, MW < 8 ? MW : 8, NK, TILED>(p, st, xs, xh, xl, sc, sc_kbm, ex, es, w, M, K, N, bias, out, part);
      break;
    case 4:
      lm_launch_t<FMT, MW < 4 ? MW : 4, NK, TILED>(p, st, xs, xh, xl, sc, sc_kbm, ex, es, w, M, K, N, bias, out, part);
      break;
    case 2: lm_launch_t<FMT, 2, NK, TILED>(p, st, xs, xh, xl, sc, sc_kbm, ex, es, w, M, K, N, bias, out, part); break;
    default: lm_launch_t<FMT, 1, NK, TILED>(p, st, xs, xh, xl, sc, sc_kbm, ex, es, w, M, K, N, bias, out, part); break;
  }
}

// rows of x (and, with sT, the NB column-block exponents of a [K][N] weight)
template <typename T, bool SPLIT>
void lm_prep_rows_t(const T* x, int64_t M, int64_t K, int64_t Kp, float* xs, _Float16* xh, _Float16* xl, int* ex,
                    const float* sT, int64_t NB, int* es, hipStream_t st) {
  const dim3 grid((unsigned)(M + (sT ? NB : 0)));
  if (aligned16(x) && (K * (int64_t)sizeof(T)) % 16 == 0)
    hipLaunchKernelGGL((k_linear_mfma_prep_rows<T, SPLIT, true>), grid, dim3(256), 0, st, x, M, K, Kp, xs, xh, xl, ex,
                       sT, es);
  else
    hipLaunchKernelGGL((k_linear_mfma_prep_rows<T, SPLIT, false>), grid, dim3(256), 0, st, x, M, K, Kp, xs, xh, xl,
                       ex, sT, es);
}

template <bool SPLIT>
void lm_prep_rows(const void* x, int x_type, int64_t M, int64_t K, int64_t Kp, float* xs, _Float16* xh, _Float16* xl,
                  int* ex, const float* sT, int64_t NB, int* es, hipStream_t st) {
  if (x_type == MXK_IN_F32) lm_prep_rows_t<float, SPLIT>((const float*)x, M, K, Kp, xs, xh, xl, ex, sT, NB, es, st);
  else if (x_type == MXK_IN_F16)
    lm_prep_rows_t<__half, SPLIT>((const __half*)x, M, K, Kp, xs, xh, xl, ex, sT, NB, es, st);
  else lm_prep_rows_t<hip_bfloat16, SPLIT>((const hip_bfloat16*)x, M, K, Kp, xs, xh, xl, ex, sT, NB, es, st);
}

bool lm_common_ok(int64_t M, int64_t K, int64_t N, int kind, int bits, int block, int x_type, const float* out) {
  if (lm_format(kind, bits) == 0 || block != 128) return false;
  if (M < 1 || K < 1 || N < 128 || N % 128 != 0 || M >= (int64_t(1) << 31)) return false;
  if (x_type != MXK_IN_F32 && x_type != MXK_IN_F16 && x_type != MXK_IN_BF16) return false;
  if (!aligned16(out)) return false;
  const int64_t Kp = ceil_div(K, LM_STAGE) * LM_STAGE, lim = int64_t(1) << 31;
  // 32-bit buffer offsets: codes (with the padded stage rows), one row tile of x', the scales
  if ((Kp + LM_STAGE) * N * bits / 8 >= lim || 256 * Kp * 4 >= lim || (N / 128) * Kp * 4 >= lim) return false;
  if (ceil_div(M, 32) >= 65536 || M + N / 128 >= (int64_t(1) << 31)) return false;
  return true;
}

}  // namespace

// ---------------------------------------------------------------- internal entry points
// Bytes of workspace the MFMA path needs for this product (0 when it does
// not take the shape); the first LM_WS_BASE bytes are left untouched.
size_t linear_mfma_workspace(int64_t M, int64_t K, int64_t N, int bits, int block, bool nk) {
  if ((bits != 1 && bits != 2 && bits != 4 && bits != 8) || block != 128 || M < 1 || K < 1 || N < 128 || N % 128 != 0) return 0;
  if (nk && K % 128 != 0) return 0;
  return lm_plan(M, K, N, nk, bits).bytes;
}

// [K][N] weight (mx_linear).  Returns MXK_EUNSUPPORTED, with nothing
// launched, for shapes it does not take.
int linear_mfma_kn(const void* x, int x_type, int64_t M, int64_t K, const void* w_packed, const float* w_scales,
                   const float* w_scales_t, int64_t N, int kind, int bits, int block, const float* bias, float* out,
                   void* workspace, size_t workspace_nbytes, hipStream_t st) {
  if (!lm_common_ok(M, K, N, kind, bits, block, x_type, out)) return MXK_EUNSUPPORTED;
  if ((reinterpret_cast<uintptr_t>(w_packed) & (bits == 8 ? 7u : bits == 4 ? 3u : bits == 2 ? 1u : 0u)) != 0)
    return MXK_EUNSUPPORTED;
  const LmPlan p = lm_plan(M, K, N, false, bits);
  if (!workspace || workspace_nbytes < p.bytes)
    return fail(MXK_EINVAL, "linear_wq: needs a workspace of mxk_linear_workspace() bytes");
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  int* ex = reinterpret_cast<int*>(ws + p.off_ex);
  int* es = reinterpret_cast<int*>(ws + p.off_es);
  float* xs = reinterpret_cast<float*>(ws + p.off_x);
  float* sc = reinterpret_cast<float*>(ws + p.off_s);
  float* part = reinterpret_cast<float*>(ws + p.off_p);
  const int64_t NB = N / 128;
  const float* sT = w_scales_t;
  if (!sT) {
    hipLaunchKernelGGL(k_linear_mfma_scales_t, dim3((unsigned)ceil_div(K * NB, 256)), dim3(256), 0, st, w_scales, K,
                       NB, sc);
    sT = sc;
  }
  lm_prep_rows<false>(x, x_type, M, K, p.Kp, xs, nullptr, nullptr, ex, sT, NB, es, st);
  const uint8_t* w = reinterpret_cast<const uint8_t*>(w_packed);
  const int fmt = lm_format(kind, bits);
  switch (fmt) {
#define MXK_LMK(F) \
  case F: lm_launch_w<F, false>(p, st, xs, nullptr, nullptr, sT, 1, ex, es, w, M, K, N, bias, out, part); break;
    MXK_LMK(LM_I1)
    MXK_LMK(LM_I2)
    MXK_LMK(LM_I4)
    MXK_LMK(LM_I8)
    MXK_LMK(LM_F4)
    MXK_LMK(LM_F8)
#undef MXK_LMK
  }
  if (p.S > 1)
    hipLaunchKernelGGL(k_linear_mfma_reduce, dim3((unsigned)ceil_div(M * N / 4, 256)), dim3(256), 0, st, part, p.S,
                       M, N, ex, es, bias, lm_post(fmt), out);
  return check_launch("linear_wq(mfma)");
}

// [K][N] int4 weight in the tiled layout (block-major scales required)
int linear_mfma_kn_tiled(const void* x, int x_type, int64_t M, int64_t K, const void* w_tiled,
                         const float* w_scales_t, int64_t N, int kind, const float* bias, float* out,
                         void* workspace, size_t workspace_nbytes, hipStream_t st) {
  if (!lm_common_ok(M, K, N, kind, 4, 128, x_type, out) || K % 32 != 0) return MXK_EUNSUPPORTED;
  if (!aligned16(w_tiled) || !w_scales_t) return MXK_EUNSUPPORTED;
  const LmPlan p = lm_plan(M, K, N, false, 4);
  if (!workspace || workspace_nbytes < p.bytes)
    return fail(MXK_EINVAL, "linear_wq_tiled: needs a workspace of mxk_linear_workspace() bytes");
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  int* ex = reinterpret_cast<int*>(ws + p.off_ex);
  int* es = reinterpret_cast<int*>(ws + p.off_es);
  float* xs = reinterpret_cast<float*>(ws + p.off_x);
  float* part = reinterpret_cast<float*>(ws + p.off_p);
  lm_prep_rows<false>(x, x_type, M, K, p.Kp, xs, nullptr, nullptr, ex, w_scales_t, N / 128, es, st);
  const uint8_t* wt = reinterpret_cast<const uint8_t*>(w_tiled);
  const int fmt = lm_format(kind, 4);
  if (fmt == LM_F4)
    lm_launch_w<LM_F4, false, true>(p, st, xs, nullptr, nullptr, w_scales_t, 1, ex, es, wt, M, K, N, bias, out, part);
  else
    lm_launch_w<LM_I4, false, true>(p, st, xs, nullptr, nullptr, w_scales_t, 1, ex, es, wt, M, K, N, bias, out, part);
  if (p.S > 1)
    hipLaunchKernelGGL(k_linear_mfma_reduce, dim3((unsigned)ceil_div(M * N / 4, 256)), dim3(256), 0, st, part, p.S,
                       M, N, ex, es, bias, lm_post(fmt), out);
  return check_launch("linear_wq_tiled(mfma)");
}

// [N][K] weight (mx_dynamic_linear, input gradients).  `w_scales_t` is the
// K-block-major copy [K/128][N] when given, else the scales [N][K/128].
int linear_mfma_nk(const void* x, int x_type, int64_t M, int64_t K, const void* w_packed, const float* w_scales,
                   const float* w_scales_t, int64_t N, int kind, int bits, int block, const float* bias, float* out,
                   void* workspace, size_t workspace_nbytes, hipStream_t st) {
  if (!lm_common_ok(M, K, N, kind, bits, block, x_type, out) || K % 128 != 0) return MXK_EUNSUPPORTED;
  if (!aligned16(w_packed)) return MXK_EUNSUPPORTED;
  if (N * K * bits / 8 >= (int64_t(1) << 31) || N * (K / 128) * 4 >= (int64_t(1) << 31)) return MXK_EUNSUPPORTED;
  const LmPlan p = lm_plan(M, K, N, true, bits);
  if (!workspace || workspace_nbytes < p.bytes)
    return fail(MXK_EINVAL, "linear_wq_nt: needs a workspace of mxk_linear_nt_workspace() bytes");
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  int* ex = reinterpret_cast<int*>(ws + p.off_ex);
  _Float16* xh = reinterpret_cast<_Float16*>(ws + p.off_x);
  _Float16* xl = xh + (size_t)lm_rows16(M) * (size_t)p.Kp;
  float* part = reinterpret_cast<float*>(ws + p.off_p);
  lm_prep_rows<true>(x, x_type, M, K, p.Kp, nullptr, xh, xl, ex, nullptr, 0, nullptr, st);
  const float* sc = w_scales_t ? w_scales_t : w_scales;
  const int kbm = w_scales_t ? 1 : 0;
  const uint8_t* w = reinterpret_cast<const uint8_t*>(w_packed);
  const int fmt = lm_format(kind, bits);
  switch (fmt) {
#define MXK_LMN(F) \
  case F: lm_launch_w<F, true>(p, st, nullptr, xh, xl, sc, kbm, ex, nullptr, w, M, K, N, bias, out, part); break;
    MXK_LMN(LM_I1)
    MXK_LMN(LM_I2)
    MXK_LMN(LM_I4)
    MXK_LMN(LM_I8)
    MXK_LMN(LM_F4)
    MXK_LMN(LM_F8)
#undef MXK_LMN
  }
  if (p.S > 1)
    hipLaunchKernelGGL(k_linear_mfma_reduce, dim3((unsigned)ceil_div(M * N / 4, 256)), dim3(256), 0, st, part, p.S,
                       M, N, ex, nullptr, bias, lm_post(fmt), out);
  return check_launch("linear_wq_nt(mfma)");
}

int linear_mfma_nk_tiled(const void* x, int x_type, int64_t M, int64_t K, const void* w_tiled,
                         const float* w_scales_t, int64_t N, const float* bias, float* out, void* workspace,
                         size_t workspace_nbytes, hipStream_t st) {
  if (!lm_common_ok(M, K, N, MXK_KIND_INT, 4, 128, x_type, out) || K % 128 != 0) return MXK_EUNSUPPORTED;
  if (!aligned16(w_tiled) || !w_scales_t) return MXK_EUNSUPPORTED;
  if (N * K / 2 >= (int64_t(1) << 31) || N * (K / 128) * 4 >= (int64_t(1) << 31)) return MXK_EUNSUPPORTED;
  const LmPlan p = lm_plan(M, K, N, true, 4);
  if (!workspace || workspace_nbytes < p.bytes)
    return fail(MXK_EINVAL, "linear_wq_nt_tiled: needs a workspace of mxk_linear_nt_workspace() bytes");
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  int* ex = reinterpret_cast<int*>(ws + p.off_ex);
  _Float16* xh = reinterpret_cast<_Float16*>(ws + p.off_x);
  _Float16* xl = xh + (size_t)lm_rows16(M) * (size_t)p.Kp;
  float* part = reinterpret_cast<float*>(ws + p.off_p);
  lm_prep_rows<true>(x, x_type, M, K, p.Kp, nullptr, xh, xl, ex, nullptr, 0, nullptr, st);
  lm_launch_w<LM_I4, true, true>(p, st, nullptr, xh, xl, w_scales_t, 1, ex, nullptr,
                                 reinterpret_cast<const uint8_t*>(w_tiled), M, K, N, bias, out, part);
  if (p.S > 1)
    hipLaunchKernelGGL(k_linear_mfma_reduce, dim3((unsigned)ceil_div(M * N / 4, 256)), dim3(256), 0, st, part, p.S,
                       M, N, ex, nullptr, bias, 1.0f, out);
  return check_launch("linear_wq_nt_tiled(mfma)");
}

}  // namespace mxk
