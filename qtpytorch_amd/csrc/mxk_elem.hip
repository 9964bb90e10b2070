// Quantized element-wise arithmetic for gfx950: the CPU branches of
// _dispatch_qadd / _dispatch_qsub / _dispatch_qmul (mxtorch.py:5321-5497)
// around _qscale_add / _qscale_mul (mxtorch.py:1186-1296), and
// mx_tensor.__neg__ (mxtorch.py:6177-6193).
//
// Both operands' codes are unpacked with a's width and sign-extended (float
// dtypes' grid indices included, as bit_packer.unpack_auto does), codes past
// n read as 0 (the reference pads the unpacked codes), per block of `block`:
//
//   add/sub (b's codes negated for sub), max_int = 2^(bits-1) - 1:
//     if max(sa,sb) / max(min(sa,sb), 1e-30) <= 2:        integer path
//        sc = max(sa,sb); c = rne(a*RN(sa/sc)) + rne(b*RN(sb/sc));
//        if max|c| > max_int: sc *= 2 and recompute; code = clamp(c)
//     else:                                              float path
//        s = RN(a*sa) + RN(b*sb); sc = RN(max(max|s|, 1e-12) / max_int);
//        code = rne(clamp(RN(s / sc)))
//   mul: code = rne(clamp(RN(RN(a*b) / max_int))), sc = RN(RN(sa*sb)*max_int)
//
// and the nb*block codes are packed with the output width (pack_auto masks
// each code to that width).  neg: code = clamp(-c, +-max_int) over the n
// codes (all stored bytes for 8-bit codes), scales unchanged.
#include "mxk_internal.h"

namespace mxk {

enum ElemOp : int { E_ADD = 0, E_SUB = 1, E_MUL = 2, E_NEG = 3 };

// Code g of a buffer packed with BITS (bytes for 1, 2, 4, 8; int32 words of
// floor(32/BITS) fields otherwise), sign-extended; 0 past nbytes.
template <int BITS>
__device__ __forceinline__ int32_t load_code(const uint8_t* __restrict__ p, int64_t nbytes, int64_t g) {
  uint32_t v;
  int sh;
  if constexpr (BITS == 1 || BITS == 2 || BITS == 4 || BITS == 8) {
    const int64_t bit = g * BITS;
    const int64_t byte = bit >> 3;
    v = byte < nbytes ? (uint32_t)p[byte] : 0u;
    sh = (int)(bit & 7);
  } else {
    constexpr int FPW = 32 / BITS;
    const int64_t w = g / FPW;
    sh = (int)(g % FPW) * BITS;
    v = (w * 4 + 4 <= nbytes) ? reinterpret_cast<const uint32_t*>(p)[w] : 0u;
  }
  return (int32_t)(v << (32 - BITS - sh)) >> (32 - BITS);
}

// One wave per block of `block` <= 256 elements, lane l holding elements
// l, l+64, ... (E = ceil(block/64) of them); grid-stride over blocks.
// OB > 0: the block's codes go through LDS and each lane packs 32-bit output
// words (block*OB % 32 == 0); OB == 0: int32 codes to `codes_out` (packed by
// k_pack_codes).
template <int OP, int BITS, int OB>
__global__ __launch_bounds__(256) void k_qelem(const uint8_t* __restrict__ a, int64_t a_nbytes,
                                               const float* __restrict__ sa_, const uint8_t* __restrict__ b,
                                               int64_t b_nbytes, const float* __restrict__ sb_, int64_t n, int64_t nb,
                                               int block, uint32_t* __restrict__ out_words,
                                               int32_t* __restrict__ codes_out, float* __restrict__ out_scales) {
  __shared__ int32_t s[4][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int E = (block + 63) >> 6;
  const float qf = (float)((1 << (BITS - 1)) - 1);
  for (int64_t blk = (int64_t)blockIdx.x * 4 + wave; blk < nb; blk += (int64_t)gridDim.x * 4) {
    const float sa = sa_[blk], sb = sb_[blk];
    float ac[4], bc[4], cv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ac[i] = bc[i] = cv[i] = 0.0f;
      if (i < E && lane + 64 * i < block) {
        const int64_t g = blk * block + lane + 64 * i;
        if (g < n) {
          ac[i] = (float)load_code<BITS>(a, a_nbytes, g);
          const int32_t bq = load_code<BITS>(b, b_nbytes, g);
          bc[i] = (float)(OP == E_SUB ? -bq : bq);
        }
      }
    }
    float scale;
    if constexpr (OP == E_MUL) {
#pragma unroll
      for (int i = 0; i < 4; ++i) cv[i] = rne(fminf(fmaxf((ac[i] * bc[i]) / qf, -qf), qf));
      scale = (sa * sb) * qf;
    } else {
      const float hi = fmaxf(sa, sb);
      const float ratio = hi / fmaxf(fminf(sa, sb), 1e-30f);
      if (ratio <= 2.0f) {
        float sc = hi;
        float ra = sa / sc, rb = sb / sc, m = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          cv[i] = rne(ac[i] * ra) + rne(bc[i] * rb);
          m = fmaxf(m, __builtin_fabsf(cv[i]));
        }
        m = group_max<64>(m);
        if (m > qf) {
          sc = sc * 2.0f;
          ra = sa / sc;
          rb = sb / sc;
#pragma unroll
          for (int i = 0; i < 4; ++i) cv[i] = rne(ac[i] * ra) + rne(bc[i] * rb);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) cv[i] = fminf(fmaxf(cv[i], -qf), qf);
        scale = sc;
      } else {
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          cv[i] = ac[i] * sa + bc[i] * sb;
          m = fmaxf(m, __builtin_fabsf(cv[i]));
        }
        m = group_max<64>(m);
        const float sc = fmaxf(m, MXK_AMIN) / qf;
#pragma unroll
        for (int i = 0; i < 4; ++i) cv[i] = rne(fminf(fmaxf(cv[i] / sc, -qf), qf));
        scale = sc;
      }
    }
    if (lane == 0) out_scales[blk] = scale;
    if constexpr (OB == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (i < E && lane + 64 * i < block) codes_out[blk * block + lane + 64 * i] = (int32_t)cv[i];
    } else {
      constexpr int CPW = 32 / OB;
      constexpr uint32_t MASK = OB == 32 ? 0xFFFFFFFFu : ((1u << OB) - 1u);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (i < E && lane + 64 * i < block) s[wave][lane + 64 * i] = (int32_t)cv[i];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int W = block * OB / 32;
      for (int w = lane; w < W; w += 64) {
        uint32_t word = 0u;
#pragma unroll
        for (int f = 0; f < CPW; ++f) word |= ((uint32_t)s[wave][w * CPW + f] & MASK) << (f * OB);
        out_words[blk * W + w] = word;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
}

// Fast path for byte-packed operands (BITS in {2, 4, 8}) and outputs
// OB in {2, 4, 8, 16} with block = E * LPB (64, 128, 256): each lane owns E
// (8 or 16) consecutive codes of one block (one 2..16-byte buffer load per
// operand, loads past the buffer return 0), LPB lanes share a block, and the
// lane packs its E result codes into one 2..16-byte store.  Buffers < 4 GiB.
template <int NBYTES>
__device__ __forceinline__ uint64_t load_packed(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  if constexpr (NBYTES == 2) return (uint64_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
  else if constexpr (NBYTES == 4) return (uint64_t)(uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
  else {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
    return (uint64_t)(uint32_t)v[0] | ((uint64_t)(uint32_t)v[1] << 32);
  }
}

// A lane's packed codes (NBYTES <= 16) as 64-bit words, low codes first.
// A 16-byte load that would cross the buffer's end (nbytes) is made as two
// 8-byte loads, so that the bytes below the end are read as for 8 codes per lane.
template <int NBYTES>
__device__ __forceinline__ void load_codes(__amdgpu_buffer_rsrc_t r, uint32_t off, int64_t nbytes,
                                           uint64_t (&w)[(NBYTES + 7) / 8]) {
  if constexpr (NBYTES == 16) {
    if ((int64_t)off + 16 <= nbytes) {
      const u32x4 v = buf_load_b128(r, off, 0u);
      w[0] = (uint64_t)v[0] | ((uint64_t)v[1] << 32);
      w[1] = (uint64_t)v[2] | ((uint64_t)v[3] << 32);
    } else {
      w[0] = load_packed<8>(r, off);
      w[1] = load_packed<8>(r, off + 8u);
    }
  } else {
    w[0] = load_packed<NBYTES>(r, off);
  }
}

// RN(a / b) by Markstein's correction with y = RN(1/b): correctly rounded
// unless 0 < |a| < 2^-96 (the callers state why that cannot change their
// result), and a zero quotient may come out with either sign (callers that
// round it to an integer code code both zeros the same).
__device__ __forceinline__ float markstein(float a, float b, float y) {
  const float q0 = a * y;
  return __builtin_fmaf(__builtin_fmaf(-q0, b, a), y, q0);
}

// Bit pattern whose low bits are rne(clamp(q, -qf, qf)) in two's
// complement: the float adder rounds t + 1.5 * 2^23 (|t| <= qf <= 2^15) to
// an integer with ties to even, leaving 2^22 + 2^23 + rne(t) in the
// significand.
__device__ __forceinline__ uint32_t rne_clamped_bits(float q, float qf) {
  return __float_as_uint(__builtin_amdgcn_fmed3f(q, -qf, qf) + 12582912.0f);
}

// A lane's E codes of BITS in {2, 4, 8} bits (little-endian fields of w,
// low codes first) as floats of code * 2^(8 - BITS): each word's fields of
// one sub-position are moved to the tops of its bytes by one shift and one
// mask, then each byte converts as a sign-extended byte (v_cvt_f32_i32 with
// an SDWA byte select): ~1.2 VALU per code against ~5 for a 64-bit shift,
// a field extract and a conversion.  The caller scales its factors by
// 2^(BITS - 8), which keeps every product exact.
template <int BITS, int E, int NW>
__device__ __forceinline__ void codes_scaled(const uint64_t (&w)[NW], float (&c)[E]) {
  constexpr int PB = 8 / BITS, CW = 32 / BITS;  // fields per byte, codes per 32-bit word
  constexpr uint32_t TOP = BITS == 8 ? 0xFFFFFFFFu : (BITS == 4 ? 0xF0F0F0F0u : 0xC0C0C0C0u);
#pragma unroll
  for (int h = 0; h < (E + CW - 1) / CW; ++h) {
    const uint32_t x = (uint32_t)(w[h >> 1] >> (32 * (h & 1)));
#pragma unroll
    for (int p = 0; p < PB; ++p) {
      const uint32_t t = (x << (8 - BITS * (p + 1))) & TOP;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (h * CW + j * PB + p < E) c[h * CW + j * PB + p] = (float)(int8_t)(t >> (8 * j));
    }
  }
}

template <int OP, int BITS, int OB, int LPB, int E>
__global__ __launch_bounds__(256) void k_qelem_fast(const uint8_t* __restrict__ a, int64_t a_nbytes,
                                                    const float* __restrict__ sa_, const uint8_t* __restrict__ b,
                                                    int64_t b_nbytes, const float* __restrict__ sb_, int64_t n,
                                                    int64_t nb, uint8_t* __restrict__ out, int64_t out_nbytes,
                                                    float* __restrict__ out_scales) {
  constexpr int B = E * LPB, GPW = 64 / LPB, GPB = 4 * GPW;
  static_assert(E * BITS <= 128, "codes of a lane in one load of up to 16 bytes");
  constexpr int NW = (E * BITS + 63) / 64;  // 64-bit words of a lane's codes
  constexpr int INB = E * BITS / 8, ONB = E * OB / 8;
  constexpr uint32_t OMASK = (1u << OB) - 1u;
  const float qf = (float)((1 << (BITS - 1)) - 1);
  const float qinv_c = 1.0f / qf;  // RN(1/q)
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(a, (uint32_t)a_nbytes);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(b, (uint32_t)b_nbytes);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane / LPB, li = lane % LPB;
  for (int64_t b0 = (int64_t)blockIdx.x * GPB; b0 < nb; b0 += (int64_t)gridDim.x * GPB) {
    const int64_t blk = b0 + wave * GPW + g;
    const bool live = blk < nb;
    const int64_t e0 = blk * B + (int64_t)li * E;
    uint64_t wa[NW], wb[NW];
    load_codes<INB>(ra, (uint32_t)(live ? e0 * BITS / 8 : 0), a_nbytes, wa);
    load_codes<INB>(rb, (uint32_t)(live ? e0 * BITS / 8 : 0), b_nbytes, wb);
    const float sa = live ? sa_[blk] : 1.0f, sb = live ? sb_[blk] : 1.0f;
    // codes at or past n (and every code of a dead lane) read as 0: one mask
    // per lane instead of a bounds select per element
    const int64_t rem = live ? n - e0 : 0;
    if (rem < E) {
      const int kb = rem <= 0 ? 0 : (int)rem * BITS;  // bits kept, < E * BITS
#pragma unroll
      for (int k = 0; k < NW; ++k) {
        const int kk = kb - 64 * k;
        const uint64_t keep = kk <= 0 ? 0ull : (kk >= 64 ? ~0ull : ((1ull << kk) - 1ull));
        wa[k] &= keep;
        wb[k] &= keep;
      }
    }
    // codes times 2^(8 - BITS) (codes_scaled); factors that multiply them
    // are scaled by CS = 2^(BITS - 8): exact for every factor >= 2^-100 (a
    // scale below that takes the codes back to their values instead)
    constexpr float CS = BITS == 8 ? 1.0f : (BITS == 4 ? 0.0625f : 0.015625f);
    float ac[E], bc[E], cv[E];
    uint32_t cu[E];  // code bits (the low OB bits are the two's complement code)
    codes_scaled<BITS, E, NW>(wa, ac);
    codes_scaled<BITS, E, NW>(wb, bc);
    if constexpr (OP == E_SUB) {
#pragma unroll
      for (int i = 0; i < E; ++i) bc[i] = -bc[i];
    }
    float scale;
    if constexpr (OP == E_MUL) {
      // RN(prod / max_int) by Markstein's correction with y = RN(1/max_int):
      // the products are 0 or at least 1 in magnitude; the scaled codes'
      // product over max_int * 2^(16 - 2 BITS) is the same quotient
      constexpr float CS2 = CS * CS;
      const float qs = qf / CS2, qinv = (1.0f / qf) * CS2;
#pragma unroll
      for (int i = 0; i < E; ++i) cu[i] = rne_clamped_bits(markstein(ac[i] * bc[i], qs, qinv), qf);
      scale = (sa * sb) * qf;
    } else {
      const float hi = fmaxf(sa, sb);
      // RN(hi / lo) <= 2 exactly when hi / lo <= 2 + 2^-23 (the midpoint
      // above 2 rounds to even, to 2): hi - 2 lo <= 2^-23 lo, where the FMA
      // difference is exact near the boundary (hi and 2 lo within a factor
      // of 2) and 2^-23 lo is exact (lo >= 1e-30); non-finite scales take
      // the division's branches (an infinite hi or NaN difference: float
      // form).  Two VALU in place of a division.
      const float lo_ = fmaxf(fminf(sa, sb), 1e-30f);
      const bool use_int = __builtin_fmaf(-2.0f, lo_, hi) <= 0x1p-23f * lo_;  // uniform over the block's lanes
      float sc = hi;
      float ra_ = 1.0f, rb_ = 1.0f, m = 0.0f;
      float f = CS;  // the factor the codes' products carry
      if (BITS != 8 && __builtin_expect(!(fminf(sa, sb) >= 0x1p-100f), 0)) {
#pragma unroll
        for (int i = 0; i < E; ++i) {
          ac[i] *= CS;
          bc[i] *= CS;
        }
        f = 1.0f;
      }
      // one form per block (the lanes of a block agree on use_int)
      if (use_int) {
        ra_ = sa / sc;
        rb_ = sb / sc;
        const float fa = ra_ * f, fb = rb_ * f;
#pragma unroll
        for (int i = 0; i < E; ++i) cv[i] = rne(ac[i] * fa) + rne(bc[i] * fb);
      } else {
        const float fa = sa * f, fb = sb * f;
#pragma unroll
        for (int i = 0; i < E; ++i) cv[i] = ac[i] * fa + bc[i] * fb;
      }
#pragma unroll
      for (int i = 0; i < E; ++i) m = fmaxf(m, __builtin_fabsf(cv[i]));
      m = group_max<LPB>(m);
      if (use_int) {
        if (m > qf) {
          sc = sc * 2.0f;
          ra_ = sa / sc;
          rb_ = sb / sc;
          const float fa = ra_ * f, fb = rb_ * f;
#pragma unroll
          for (int i = 0; i < E; ++i) cv[i] = rne(ac[i] * fa) + rne(bc[i] * fb);
        }
      } else {
        // RN(max / q) by Markstein's correction with RN(1/q): the dividend
        // is at least fl32(1e-12), so the quotient is correctly rounded
        sc = markstein(fmaxf(m, MXK_AMIN), qf, qinv_c);
        // RN(sum / sc) by Markstein's correction for every element, without
        // div_rn_all's small-dividend vote: sc >= 1e-12 / 127 > 2^-47, so a
        // dividend below 2^-96 has |quotient| < 2^-49 on either path and
        // rounds to code 0 below
        const float y = 1.0f / sc;
#pragma unroll
        for (int i = 0; i < E; ++i) cv[i] = markstein(cv[i], sc, y);
      }
      // both forms end in one tail: the integer sums are already integers,
      // so clamp + round is their clamp (the integer form used to run its
      // own clamp and conversion, in every wave: the compiler did not
      // branch around it)
#pragma unroll
      for (int i = 0; i < E; ++i) cu[i] = rne_clamped_bits(cv[i], qf);
      scale = sc;
    }
    uint32_t w[(ONB + 3) / 4];
#pragma unroll
    for (int q = 0; q < (ONB + 3) / 4; ++q) w[q] = 0u;
#pragma unroll
    for (int i = 0; i < E; ++i) w[(i * OB) >> 5] |= (cu[i] & OMASK) << ((i * OB) & 31);
    if (live) {
      store_bytes<ONB>(out, e0 * OB / 8, out_nbytes, w);
      if (li == 0) out_scales[blk] = scale;
    }
  }
}

// Negation: output unit u (a byte for OB in {1,2,4,8}, else an int32 word)
// of `count` codes, code = clamp(-c, +-max_int), packed with OB = BITS.
template <int BITS>
__global__ __launch_bounds__(256) void k_qneg(const uint8_t* __restrict__ a, int64_t a_nbytes, int64_t count,
                                              uint8_t* __restrict__ out, int64_t out_units) {
  constexpr bool BYTES = BITS == 1 || BITS == 2 || BITS == 4 || BITS == 8;
  constexpr int CPU = BYTES ? 8 / BITS : 32 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  const int32_t qi = (1 << (BITS - 1)) - 1;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < out_units;
       u += (int64_t)gridDim.x * blockDim.x) {
    uint32_t unit = 0u;
#pragma unroll
    for (int f = 0; f < CPU; ++f) {
      const int64_t g = u * CPU + f;
      if (g < count) {
        const int32_t c = -load_code<BITS>(a, a_nbytes, g);
        unit |= ((uint32_t)min(max(c, -qi), qi) & MASK) << (f * BITS);
      }
    }
    if constexpr (BYTES) out[u] = (uint8_t)unit;
    else reinterpret_cast<uint32_t*>(out)[u] = unit;
  }
}

// pack_auto of int32 codes with width OB (mxtorch.py:882-955): output unit u
// is a byte (OB in {1,2,4,8}) or an int32 word of floor(32/OB) fields.
template <int OB>
__global__ __launch_bounds__(256) void k_pack_codes(const int32_t* __restrict__ codes, int64_t count,
                                                    uint8_t* __restrict__ out, int64_t out_units) {
  constexpr bool BYTES = OB == 1 || OB == 2 || OB == 4 || OB == 8;
  constexpr int CPU = BYTES ? 8 / OB : 32 / OB;
  constexpr uint32_t MASK = OB == 32 ? 0xFFFFFFFFu : ((1u << OB) - 1u);
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < out_units;
       u += (int64_t)gridDim.x * blockDim.x) {
    uint32_t unit = 0u;
#pragma unroll
    for (int f = 0; f < CPU; ++f) {
      const int64_t g = u * CPU + f;
      if (g < count) unit |= ((uint32_t)codes[g] & MASK) << (f * OB);
    }
    if constexpr (BYTES) out[u] = (uint8_t)unit;
    else reinterpret_cast<uint32_t*>(out)[u] = unit;
  }
}

static bool valid_bits(int b) { return (b >= 1 && b <= 8) || b == 16; }
static bool byte_bits(int b) { return b == 1 || b == 2 || b == 4 || b == 8; }

template <int OB>
static void launch_pack(const int32_t* codes, int64_t count, void* out, int64_t out_units, hipStream_t st) {
  const dim3 g((unsigned)std::min<int64_t>(ceil_div(out_units, 256), (int64_t)num_cus() * 16));
  hipLaunchKernelGGL((k_pack_codes<OB>), g, dim3(256), 0, st, codes, count, (uint8_t*)out, out_units);
}

template <int OP, int BITS, int OB>
static void launch_elem(const void* a, int64_t an, const float* sa, const void* b, int64_t bn, const float* sb,
                        int64_t n, int64_t nb, int block, void* out, int32_t* codes, float* cs, hipStream_t st) {
  const dim3 g((unsigned)std::min<int64_t>(ceil_div(nb, 4), (int64_t)num_cus() * 16));
  hipLaunchKernelGGL((k_qelem<OP, BITS, OB>), g, dim3(256), 0, st, (const uint8_t*)a, an, sa, (const uint8_t*)b, bn,
                     sb, n, nb, block, (uint32_t*)out, codes, cs);
}

template <int OP, int BITS>
static int dispatch_out(int out_bits, bool fused, const void* a, int64_t an, const float* sa, const void* b,
                        int64_t bn, const float* sb, int64_t n, int64_t nb, int block, void* out, int64_t out_units,
                        int32_t* ws, float* cs, hipStream_t st) {
  if (fused) {
    switch (out_bits) {
      case 1: launch_elem<OP, BITS, 1>(a, an, sa, b, bn, sb, n, nb, block, out, nullptr, cs, st); break;
      case 2: launch_elem<OP, BITS, 2>(a, an, sa, b, bn, sb, n, nb, block, out, nullptr, cs, st); break;
      case 4: launch_elem<OP, BITS, 4>(a, an, sa, b, bn, sb, n, nb, block, out, nullptr, cs, st); break;
      case 8: launch_elem<OP, BITS, 8>(a, an, sa, b, bn, sb, n, nb, block, out, nullptr, cs, st); break;
      default: launch_elem<OP, BITS, 16>(a, an, sa, b, bn, sb, n, nb, block, out, nullptr, cs, st); break;
    }
    return check_launch("qelementwise");
  }
  launch_elem<OP, BITS, 0>(a, an, sa, b, bn, sb, n, nb, block, nullptr, ws, cs, st);
  const int64_t count = nb * block;
  switch (out_bits) {
    case 1: launch_pack<1>(ws, count, out, out_units, st); break;
    case 2: launch_pack<2>(ws, count, out, out_units, st); break;
    case 3: launch_pack<3>(ws, count, out, out_units, st); break;
    case 4: launch_pack<4>(ws, count, out, out_units, st); break;
    case 5: launch_pack<5>(ws, count, out, out_units, st); break;
    case 6: launch_pack<6>(ws, count, out, out_units, st); break;
    case 7: launch_pack<7>(ws, count, out, out_units, st); break;
    case 8: launch_pack<8>(ws, count, out, out_units, st); break;
    default: launch_pack<16>(ws, count, out, out_units, st); break;
  }
  return check_launch("qelementwise(pack)");
}

template <int OP>
static int dispatch_bits(int bits, int out_bits, bool fused, const void* a, int64_t an, const float* sa,
                         const void* b, int64_t bn, const float* sb, int64_t n, int64_t nb, int block, void* out,
                         int64_t out_units, int32_t* ws, float* cs, hipStream_t st) {
#define MXK_EB(B) \
  case B: return dispatch_out<OP, B>(out_bits, fused, a, an, sa, b, bn, sb, n, nb, block, out, out_units, ws, cs, st);
  switch (bits) {
    MXK_EB(2) MXK_EB(3) MXK_EB(4) MXK_EB(5) MXK_EB(6) MXK_EB(7) MXK_EB(8) MXK_EB(16)
    default: return fail(MXK_EUNSUPPORTED, "qelementwise: operand width must be 2..8 or 16");
  }
#undef MXK_EB
}

static bool fused_ok(int block, int out_bits) {
  return block <= 256 && (byte_bits(out_bits) || out_bits == 16) && (block * out_bits) % 32 == 0;
}

template <int OP, int BITS, int OB, int LPB, int E>
static void launch_fast_t(const void* a, int64_t an, const float* sa, const void* b, int64_t bn, const float* sb,
                          int64_t n, int64_t nb, void* out, int64_t onb, float* cs, hipStream_t st) {
  constexpr int GPB = 4 * (64 / LPB);
  // workgroups per CU (0: one per pass, no grid-stride cap), measured at
  // 2^28 codes with identical outputs: the int8 multiply streams best
  // uncapped (0.65 -> 0.77 of 8 TB/s), the add and the 4-bit multiply at 64
  constexpr int CAP = (OP == E_MUL && BITS == 8) ? 0 : 64;
  const int64_t units = ceil_div(nb, GPB);
  const dim3 g((unsigned)(CAP == 0 ? units : std::min<int64_t>(units, (int64_t)num_cus() * CAP)));
  hipLaunchKernelGGL((k_qelem_fast<OP, BITS, OB, LPB, E>), g, dim3(256), 0, st, (const uint8_t*)a, an, sa,
                     (const uint8_t*)b, bn, sb, n, nb, (uint8_t*)out, onb, cs);
}

// Codes per lane: 16 when a lane's codes of each operand and its packed
// result each fit 16 bytes (more bytes in flight and the per-block work over
// more codes), else 8.
template <int OP, int BITS, int OB>
static void launch_fast_b(int block, const void* a, int64_t an, const float* sa, const void* b, int64_t bn,
                          const float* sb, int64_t n, int64_t nb, void* out, int64_t onb, float* cs, hipStream_t st) {
  constexpr int E = (16 * BITS <= 128 && 16 * OB <= 128) ? 16 : 8;
  if (block == 64) launch_fast_t<OP, BITS, OB, 64 / E, E>(a, an, sa, b, bn, sb, n, nb, out, onb, cs, st);
  else if (block == 128) launch_fast_t<OP, BITS, OB, 128 / E, E>(a, an, sa, b, bn, sb, n, nb, out, onb, cs, st);
  else launch_fast_t<OP, BITS, OB, 256 / E, E>(a, an, sa, b, bn, sb, n, nb, out, onb, cs, st);
}

template <int OP, int BITS>
static void launch_fast_o(int block, int ob, const void* a, int64_t an, const float* sa, const void* b, int64_t bn,
                          const float* sb, int64_t n, int64_t nb, void* out, int64_t onb, float* cs, hipStream_t st) {
  if (ob == 2) launch_fast_b<OP, BITS, 2>(block, a, an, sa, b, bn, sb, n, nb, out, onb, cs, st);
  else if (ob == 4) launch_fast_b<OP, BITS, 4>(block, a, an, sa, b, bn, sb, n, nb, out, onb, cs, st);
  else if (ob == 8) launch_fast_b<OP, BITS, 8>(block, a, an, sa, b, bn, sb, n, nb, out, onb, cs, st);
  else launch_fast_b<OP, BITS, 16>(block, a, an, sa, b, bn, sb, n, nb, out, onb, cs, st);
}

template <int OP>
static int launch_fast(int block, int bits, int ob, const void* a, int64_t an, const float* sa, const void* b,
                       int64_t bn, const float* sb, int64_t n, int64_t nb, void* out, int64_t onb, float* cs,
                       hipStream_t st) {
  if (bits == 2) launch_fast_o<OP, 2>(block, ob, a, an, sa, b, bn, sb, n, nb, out, onb, cs, st);
  else if (bits == 4) launch_fast_o<OP, 4>(block, ob, a, an, sa, b, bn, sb, n, nb, out, onb, cs, st);
  else launch_fast_o<OP, 8>(block, ob, a, an, sa, b, bn, sb, n, nb, out, onb, cs, st);
  return check_launch("qelementwise(fast)");
}

}  // namespace mxk

using namespace mxk;

extern "C" {

size_t mxk_qelementwise_workspace(int op, int64_t n, int64_t nb, int block, int bits, int out_bits) {
  (void)n;
  (void)bits;
  if (op == E_NEG || nb <= 0 || block <= 0 || fused_ok(block, out_bits)) return 0;
  return (size_t)nb * (size_t)block * sizeof(int32_t);
}

int mxk_qelementwise(int op, const void* a_packed, int64_t a_nbytes, const float* a_scales, const void* b_packed,
                     int64_t b_nbytes, const float* b_scales, int64_t n, int64_t nb, int block, int bits,
                     int out_bits, void* c_packed, int64_t c_nbytes, float* c_scales, void* workspace,
                     size_t workspace_nbytes, void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (op < E_ADD || op > E_NEG) return fail(MXK_EINVAL, "qelementwise: op must be 0 (add), 1 (sub), 2 (mul), 3 (neg)");
  if (n <= 0 || block <= 0) return fail(MXK_EINVAL, "qelementwise: sizes must be positive");
  if (!valid_bits(bits) || !valid_bits(out_bits)) return fail(MXK_EUNSUPPORTED, "qelementwise: widths 1..8 or 16");
  if (!a_packed || !c_packed || a_nbytes < 0) return fail(MXK_EINVAL, "qelementwise: null operand");
  if ((reinterpret_cast<uintptr_t>(a_packed) & 3u) || (reinterpret_cast<uintptr_t>(c_packed) & 3u) ||
      (b_packed && (reinterpret_cast<uintptr_t>(b_packed) & 3u)))
    return fail(MXK_EINVAL, "qelementwise: packed buffers must be 4-byte aligned");
  if (op == E_NEG) {
    // 8-bit codes: every stored byte (the reference negates the int8 tensor);
    // other widths: the n codes, repacked with the same width
    if (out_bits != bits) return fail(MXK_EINVAL, "qelementwise: neg keeps the width");
    const int64_t count = bits == 8 ? a_nbytes : n;
    const int64_t units = byte_bits(bits) ? mxk_packed_nbytes(bits, count) : mxk_packed_nbytes(bits, count) / 4;
    if (c_nbytes < mxk_packed_nbytes(bits, count)) return fail(MXK_EINVAL, "qelementwise: output too small");
    const dim3 g((unsigned)std::max<int64_t>(1, std::min<int64_t>(ceil_div(units, 256), (int64_t)num_cus() * 16)));
    const uint8_t* a = (const uint8_t*)a_packed;
    uint8_t* c = (uint8_t*)c_packed;
#define MXK_NB(B) \
    case B: hipLaunchKernelGGL((k_qneg<B>), g, dim3(256), 0, st, a, a_nbytes, count, c, units); break;
    switch (bits) {
      MXK_NB(1) MXK_NB(2) MXK_NB(3) MXK_NB(4) MXK_NB(5) MXK_NB(6) MXK_NB(7) MXK_NB(8) MXK_NB(16)
      default: break;
    }
#undef MXK_NB
    return check_launch("qelementwise(neg)");
  }
  if (!b_packed || !a_scales || !b_scales || !c_scales || b_nbytes < 0) return fail(MXK_EINVAL, "qelementwise: null operand");
  if (nb * block < n) return fail(MXK_EINVAL, "qelementwise: nb * block < n");
  if (block > 256) return fail(MXK_EUNSUPPORTED, "qelementwise: block must be at most 256");
  if (bits == 1) return fail(MXK_EUNSUPPORTED, "qelementwise: 1-bit operands (max_int = 0) are not supported");
  const int64_t count = nb * block;
  const int64_t pbytes = mxk_packed_nbytes(out_bits, count);
  if (c_nbytes < pbytes) return fail(MXK_EINVAL, "qelementwise: output too small");
  // the fast kernels load every lane's codes whole (8 or 16 bytes), so both
  // operands must hold the codes of all nb*block elements; buffers that stop
  // at n codes (GEMM outputs, mxtorch.py:5570) take the byte-checked kernels
  const bool whole = a_nbytes >= count * bits / 8 && b_nbytes >= count * bits / 8;
  if (whole && (block == 64 || block == 128 || block == 256) && (bits == 2 || bits == 4 || bits == 8) &&
      (out_bits == 2 || out_bits == 4 || out_bits == 8 || out_bits == 16) && a_nbytes < ((int64_t)1 << 32) &&
      b_nbytes < ((int64_t)1 << 32) && count * bits / 8 < ((int64_t)1 << 32) &&
      (reinterpret_cast<uintptr_t>(c_packed) & 15u) == 0) {
    if (op == E_ADD) return launch_fast<E_ADD>(block, bits, out_bits, a_packed, a_nbytes, a_scales, b_packed, b_nbytes,
                                               b_scales, n, nb, c_packed, pbytes, c_scales, st);
    if (op == E_SUB) return launch_fast<E_SUB>(block, bits, out_bits, a_packed, a_nbytes, a_scales, b_packed, b_nbytes,
                                               b_scales, n, nb, c_packed, pbytes, c_scales, st);
    return launch_fast<E_MUL>(block, bits, out_bits, a_packed, a_nbytes, a_scales, b_packed, b_nbytes, b_scales, n,
                              nb, c_packed, pbytes, c_scales, st);
  }
  const bool fused = fused_ok(block, out_bits);
  const int64_t units = byte_bits(out_bits) ? pbytes : pbytes / 4;
  int32_t* ws = reinterpret_cast<int32_t*>(workspace);
  if (!fused && (!ws || workspace_nbytes < (size_t)count * sizeof(int32_t)))
    return fail(MXK_EINVAL, "qelementwise: workspace too small");
  if (op == E_ADD)
    return dispatch_bits<E_ADD>(bits, out_bits, fused, a_packed, a_nbytes, a_scales, b_packed, b_nbytes, b_scales, n,
                                nb, block, c_packed, units, ws, c_scales, st);
  if (op == E_SUB)
    return dispatch_bits<E_SUB>(bits, out_bits, fused, a_packed, a_nbytes, a_scales, b_packed, b_nbytes, b_scales, n,
                                nb, block, c_packed, units, ws, c_scales, st);
  return dispatch_bits<E_MUL>(bits, out_bits, fused, a_packed, a_nbytes, a_scales, b_packed, b_nbytes, b_scales, n,
                              nb, block, c_packed, units, ws, c_scales, st);
}

}  // extern "C"
