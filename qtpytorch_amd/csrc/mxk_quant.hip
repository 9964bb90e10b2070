// Block-absmax quantize / dequantize with bit packing, for gfx950.
//
// Semantics follow the reference's CPU path (mxtorch.py):
//   int base   _quant_int    mxtorch.py:1426-1463  r=RN(1/a'), inv=RN(r*q), s=RN(1/inv),
//                                                  code=rne(clamp(RN(x*inv),-q,q))
//   int1       _quant_int    mxtorch.py:1442-1454  s=a', code = x>=0 ? 0 : -1
//   'v'        quantize      mxtorch.py:1739-1752  s=RN(a'/q), code=rne(clamp(RN(x/s)))
//   float4/8   _quant_float  mxtorch.py:1465-1528  s=a', y=RN(x/s), idx=#{mids < y}
//   'h'        quantize      mxtorch.py:1720-1736  rotate (mxtorch.py:2866-2889) then base
//   dequant    _dequant      mxtorch.py:1530-1597
// where a' = max(absmax(block), fl32(1e-12)).
//
// Layout of work: a "group" of LPB consecutive lanes owns one block of
// B = E*LPB elements; each lane holds E elements as 16-byte chunks (half a
// block apart when there are two, so that each load instruction covers
// whole lines), the block absmax is a DPP / ds_swizzle reduction across
// the group, and each lane packs its codes into E*bits/8 bytes that it
// stores directly.  A 256-thread workgroup walks steps of blocks
// grid-stride (k_quant_fast describes the steps).
#include "mxk_internal.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <type_traits>
#include <vector>

namespace mxk {

// ---------------------------------------------------------------- errors
static thread_local std::string g_err;
void set_error(const std::string& msg) { g_err = msg; }
int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}
int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MXK_ELAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  return MXK_OK;
}

int num_cus() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lk(mu);
  if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    cache[dev] = cus;
  }
  return cache[dev];
}

// ---------------------------------------------------------------- fast quantize
// A workgroup's step count for the grid-stride loops over steps of GPB
// blocks: the workgroup whose first block is b makes q_all + (b < r_all)
// steps in all, and q_whole + (b <= r_whole) steps that end at or below
// both n and n_store.
struct QuantSteps {
  int64_t q_all, r_all, q_whole, r_whole;
};
static QuantSteps quant_steps(int grid, int gpb, int block, int64_t n, int64_t nb, int64_t n_store) {
  const int64_t rstride = (int64_t)grid * gpb;
  QuantSteps s;
  s.q_all = nb / rstride;
  s.r_all = nb % rstride;
  // step s0 is whole when s0 + gpb <= floor(min(n, n_store) / block)
  const int64_t last = std::min(n, n_store) / block - gpb;
  s.q_whole = last < 0 ? 0 : last / rstride;
  s.r_whole = last < 0 ? -1 : last % rstride;
  return s;
}

template <typename T, int E, int LPB, int MODE, int BITS>
__global__ __launch_bounds__(256) void k_quant_fast(const T* __restrict__ x, int64_t n, int64_t nb,
                                                    uint8_t* __restrict__ packed, int64_t packed_nbytes,
                                                    int64_t n_store, float* __restrict__ scales, float qf,
                                                    QuantSteps st) {
  constexpr int B = E * LPB;
  constexpr int GPW = 64 / LPB;
  constexpr int GPB = 4 * GPW;
  // A lane's E elements are Q chunks of CH consecutive elements (one
  // 16-byte load each), chunk q at offset q * B / Q in the block, so that
  // every load instruction of a wave covers whole lines.  1-bit codes of a
  // fp32 chunk fill half a byte: lanes 2i and 2i+1 swap nibbles (DPP) and
  // the even lane stores the byte.  (16-bit inputs used to keep one
  // consecutive run of 32 bytes per lane, half of each line per load
  // instruction: config 5 int4d 117 -> 108 us split, int8dv 136 -> 132.)
  constexpr int PER16 = 16 / (int)sizeof(T);
  constexpr bool NIB = sizeof(T) == 4 && BITS == 1 && E / PER16 > 1;
  constexpr bool SPLIT = E / PER16 > 1 && ((PER16 * BITS) % 8 == 0 || NIB);
  constexpr int Q = SPLIT ? E / PER16 : 1;
  constexpr int CH = E / Q;
  constexpr int NW = (CH * BITS + 31) / 32;
  constexpr int NB = NIB ? 1 : CH * BITS / 8;
  constexpr uint32_t MASK = BITS == 32 ? 0xFFFFFFFFu : ((1u << BITS) - 1u);
  const float* sP = fp_mids<MODE == Q_FP ? BITS : 4>();  // read only by the non-finite path
  __shared__ int2 sK[fp_keys_n<MODE, BITS>()];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane / LPB, li = lane % LPB;
  const int64_t rstride = (int64_t)gridDim.x * GPB;
  // A step is the workgroup's GPB consecutive blocks; the workgroup's steps
  // are grid-stride.  The steps that end at or below both n and n_store
  // ("whole": every step but those reaching the end of the data) read and
  // write through buffer resources based at the step, at the lane's fixed
  // offset: no per-lane range checks and no 64-bit lane addresses.  Their
  // loop is unrolled twice over two register sets, so that the next step's
  // loads are in flight while this one is encoded without copying
  // registers.  The remaining steps check each lane.  Step counts come from
  // the host as quotients and remainders so that the loop tests are scalar.
  // (With the signed key tables: float4d at 2^28 220 -> 198 us, float8d 243
  // -> 229 us, fp16 int8dv 149 -> 136 us.)
  const int64_t b_first = (int64_t)blockIdx.x * GPB;
  const int steps = (int)(st.q_all + (b_first < st.r_all ? 1 : 0));
  const int wholes = (int)(st.q_whole + (b_first <= st.r_whole ? 1 : 0));
  const int lo = (wave * GPW + g) * B + li * CH;  // the lane's first element in a step
  auto load_whole_step = [&](int t, float (&v)[Q][CH]) {
    const int64_t s0 = b_first + (int64_t)t * rstride;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(x + s0 * B, (uint32_t)(GPB * B * sizeof(T)));
#pragma unroll
    for (int q = 0; q < Q; ++q) buf_load_elems<T, CH>(r, (uint32_t)((lo + q * (B / Q)) * sizeof(T)), v[q]);
  };
  auto encode_step = [&](auto whole_c, int t, float (&v)[Q][CH]) {
    constexpr bool WHOLE = decltype(whole_c)::value;
    const int64_t s0 = b_first + (int64_t)t * rstride;
    const int64_t blk = s0 + wave * GPW + g;
    uint32_t mb = 0u;
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
      for (int i = 0; i < CH; ++i) mb = max(mb, mag_bits(v[q][i]));
    const float ap = amax_clamped(group_max_u<LPB>(mb));
    const BlockParams bp = block_params<MODE>(ap, qf);
    // a NaN or an infinity in the block: its codes take encode_nonfinite
    const bool nf = MODE != Q_INT1 && !finite_scale(bp.s);
    // the 'v' rule from 16-bit input divides a lane's values after one wave
    // vote (fp16 int8dv 0.66 -> 0.71 of 8 TB/s; per-element checks elsewhere)
    constexpr bool VOTE = MODE == Q_VEC && sizeof(T) == 2;
    if constexpr (VOTE) {
      if (!nf) {
#pragma unroll
        for (int q = 0; q < Q; ++q) div_rn_all<CH>(v[q], bp.s, bp.mul);
      }
    }
    // float codes: the quotients RN(v / s) for the whole step after one
    // wave vote on subnormal values (a class test and a scalar OR per
    // element, where div_rn branches per element).  Markstein's correction
    // is exact for |v| >= 2^-96; between 2^-126 and 2^-96 the quotient is
    // below 2^-56 (s >= 1e-12), where the bucket reads only whether it is
    // above 2^-150, which the correction gets right for normal v; for a
    // subnormal v its residual is rounded and the hardware divide is used.
    constexpr bool FPVOTE = MODE == Q_FP;
    if constexpr (FPVOTE) {
      if (!nf) {
        uint64_t sub = 0ull;
#pragma unroll
        for (int q = 0; q < Q; ++q)
#pragma unroll
          for (int i = 0; i < CH; ++i) sub |= __ballot(__builtin_amdgcn_classf(v[q][i], 0x90));
        if (__builtin_expect(sub != 0ull, 0)) {
#pragma unroll
          for (int q = 0; q < Q; ++q)
#pragma unroll
            for (int i = 0; i < CH; ++i) v[q][i] = v[q][i] / bp.s;
        } else {
#pragma unroll
          for (int q = 0; q < Q; ++q)
#pragma unroll
            for (int i = 0; i < CH; ++i) {
              const float q0 = v[q][i] * bp.mul;
              v[q][i] = __builtin_fmaf(__builtin_fmaf(-q0, bp.s, v[q][i]), bp.mul, q0);
            }
        }
      }
    }
    __amdgpu_buffer_rsrc_t rp;
    if constexpr (WHOLE) rp = make_rsrc(packed + s0 * (B * BITS / 8), (uint32_t)(GPB * B * BITS / 8));
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int64_t idx = blk * B + q * (B / Q) + (int64_t)li * CH;
      uint32_t w[NW];
#pragma unroll
      for (int k = 0; k < NW; ++k) w[k] = 0u;
      if (__builtin_expect(nf, 0)) {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
          const uint32_t f = (uint32_t)encode_nonfinite<MODE, BITS>(v[q][i], bp, qf, sP) & MASK;
          w[(i * BITS) >> 5] |= f << ((i * BITS) & 31);
        }
      } else {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
          // float codes come out of the table in [0, 2^BITS) and need no mask
          int c;
          if constexpr (FPVOTE) c = bucket_signed<BITS>(v[q][i], sK);
          else c = VOTE ? encode_vec_q(v[q][i], qf) : encode_keyed<MODE, BITS>(v[q][i], bp, qf, sP, sK);
          const uint32_t f = MODE == Q_FP ? (uint32_t)c : (uint32_t)c & MASK;
          w[(i * BITS) >> 5] |= f << ((i * BITS) & 31);
        }
      }
      if (!WHOLE && idx + CH > n_store) clear_tail<NW, BITS>(w, n_store - idx);
      if constexpr (NIB) {
        const uint32_t other = (uint32_t)__builtin_amdgcn_mov_dpp((int)w[0], 0xB1, 0xF, 0xF, true);
        w[0] = (w[0] & 0xFu) | ((other & 0xFu) << 4);
        if ((li & 1) == 0) {
          if constexpr (WHOLE) buf_store<1>(rp, (uint32_t)((lo + q * (B / Q)) / 8), w);
          else if (blk < nb) store_bytes<1>(packed, idx / 8, packed_nbytes, w);
        }
      } else {
        if constexpr (WHOLE) buf_store<NB>(rp, (uint32_t)((lo + q * (B / Q)) * BITS / 8), w);
        else if (blk < nb) store_bytes<NB>(packed, idx * BITS / 8, packed_nbytes, w);
      }
    }
    if constexpr (WHOLE) {
      if (li == 0) {
        const uint32_t sb = __float_as_uint(bp.s);
        buf_store<4>(make_rsrc(scales + s0, (uint32_t)(GPB * 4)), (uint32_t)((wave * GPW + g) * 4), &sb);
      }
    } else {
      if (li == 0 && blk < nb) scales[blk] = bp.s;
    }
  };
  float va[Q][CH], vb[Q][CH];
  int t = 0;
  // the first step's loads are in flight while the float key table is copied
  if (wholes > 0) load_whole_step(0, va);
  if constexpr (MODE == Q_FP) load_fp_keys<BITS>(sK);
  for (; t + 1 < wholes; t += 2) {
    load_whole_step(t + 1, vb);
    encode_step(std::true_type(), t, va);
    if (t + 2 < wholes) load_whole_step(t + 2, va);
    encode_step(std::true_type(), t + 1, vb);
  }
  if (t < wholes) {
    encode_step(std::true_type(), t, va);
    ++t;
  }
  for (; t < steps; ++t) {
    const int64_t blk = b_first + (int64_t)t * rstride + wave * GPW + g;
#pragma unroll
    for (int q = 0; q < Q; ++q) load_elems<T, CH>(x, blk * B + q * (B / Q) + (int64_t)li * CH, n, va[q]);
    encode_step(std::false_type(), t, va);
  }
}

// ---------------------------------------------------------------- long blocks
// Blocks of 264..8192 elements (a multiple of 8): one NT-thread workgroup
// per block, grid-stride.  Thread t holds chunks t, t+NT, ... of 8
// consecutive elements in registers (x is read once), the block absmax is
// a wave maximum then an NT/64-way LDS maximum, and each chunk packs into
// BITS bytes stored directly (consecutive threads, consecutive bytes).
template <typename T, int MODE, int BITS, int R, int NT>
__global__ __launch_bounds__(NT) void k_quant_rows(const T* __restrict__ x, int64_t n, int64_t nb, int block,
                                                    uint8_t* __restrict__ packed, int64_t packed_nbytes,
                                                    int64_t n_store, float* __restrict__ scales, float qf) {
  constexpr int NW = (8 * BITS + 31) / 32;
  constexpr uint32_t MASK = BITS == 32 ? 0xFFFFFFFFu : ((1u << BITS) - 1u);
  constexpr int H = MODE == Q_FP ? (1 << (BITS - 1)) : 1;
  __shared__ float sP[H + 1];
  __shared__ uint32_t s_max[NT / 64];
  if constexpr (MODE == Q_FP && BITS != 4) build_tables<BITS>(sP, nullptr);  // FP4 buckets by constants
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int chunks = block / 8;
  for (int64_t blk = blockIdx.x; blk < nb; blk += gridDim.x) {
    float v[R][8];
    uint32_t m = 0u;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = threadIdx.x + NT * r;
      if (c < chunks) {
        load_elems<T, 8>(x, blk * block + 8 * (int64_t)c, n, v[r]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[r][e] = 0.0f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) m = max(m, mag_bits(v[r][e]));
    }
    m = group_max_u<64>(m);
    if (lane == 0) s_max[wave] = m;
    __syncthreads();
    uint32_t am = s_max[0];
#pragma unroll
    for (int q = 1; q < NT / 64; ++q) am = max(am, s_max[q]);
    const float ap = amax_clamped(am);
    const BlockParams bp = block_params<MODE>(ap, qf);
    const bool nf = MODE != Q_INT1 && !finite_scale(bp.s);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = threadIdx.x + NT * r;
      if (c >= chunks) continue;
      const int64_t idx = blk * block + 8 * (int64_t)c;
      uint32_t w[NW];
#pragma unroll
      for (int k = 0; k < NW; ++k) w[k] = 0u;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t f = (uint32_t)(nf ? encode_nonfinite<MODE, BITS>(v[r][e], bp, qf, sP)
                                         : encode<MODE, BITS>(v[r][e], bp, qf, sP)) & MASK;
        w[(e * BITS) >> 5] |= f << ((e * BITS) & 31);
      }
      if (idx + 8 > n_store) clear_tail<NW, BITS>(w, n_store - idx);
      store_bytes<BITS>(packed, idx * BITS / 8, packed_nbytes, w);
    }
    if (threadIdx.x == 0) scales[blk] = bp.s;
    __syncthreads();  // s_max is rewritten by the next block
  }
}

// ---------------------------------------------------------------- generic quantize
// Any block size and any supported width: pass 1 reduces one block per wave
// and stores the scale and the multiplier, pass 2 writes one packed byte
// (bits in {1,2,4,8}) or one int32 word (bits in {3,5,6,7,16}) per thread.
template <typename T, int MODE>
__global__ __launch_bounds__(256) void k_block_params(const T* __restrict__ x, int64_t n, int64_t nb,
                                                      int block, float qf, float* __restrict__ scales,
                                                      float2* __restrict__ params) {
  const int lane = threadIdx.x & 63;
  const int64_t wave0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t blk = wave0; blk < nb; blk += nwaves) {
    uint32_t m = 0u;
    for (int i = lane; i < block; i += 64) {
      int64_t j = blk * block + i;
      if (j < n) m = max(m, mag_bits(ElemT<T>::cvt(x[j])));
    }
    const float ap = amax_clamped(group_max_u<64>(m));
    const BlockParams bp = block_params<MODE>(ap, qf);
    if (lane == 0) {
      scales[blk] = bp.s;
      params[blk] = make_float2(bp.s, bp.mul);
    }
  }
}

template <typename T, int MODE, int BITS>
__global__ __launch_bounds__(256) void k_pack_generic(const T* __restrict__ x, int64_t n, int block,
                                                      float qf, const float2* __restrict__ params,
                                                      int bits, int64_t n_store, uint8_t* __restrict__ packed,
                                                      int64_t packed_nbytes) {
  constexpr int H = MODE == Q_FP ? (1 << (BITS - 1)) : 1;
  __shared__ float sP[H + 1];
  if constexpr (MODE == Q_FP && BITS != 4) build_tables<BITS>(sP, nullptr);  // FP4 buckets by constants
  const bool words = !(bits == 1 || bits == 2 || bits == 4 || bits == 8);
  const int per = words ? 32 / bits : 8 / bits;
  const int64_t units = words ? packed_nbytes / 4 : packed_nbytes;
  const uint32_t mask = (bits >= 32) ? 0xFFFFFFFFu : ((1u << bits) - 1u);
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < units;
       u += (int64_t)gridDim.x * blockDim.x) {
    uint32_t word = 0u;
    for (int f = 0; f < per; ++f) {
      int64_t j = u * per + f;
      if (j >= n_store) break;
      float v = j < n ? ElemT<T>::cvt(x[j]) : 0.0f;
      float2 p = params[j / block];
      BlockParams bp{p.x, p.y};
      const bool nf = MODE != Q_INT1 && !finite_scale(bp.s);
      uint32_t code = (uint32_t)(nf ? encode_nonfinite<MODE, BITS>(v, bp, qf, sP) : encode<MODE, BITS>(v, bp, qf, sP)) & mask;
      word |= code << (f * bits);
    }
    if (words) reinterpret_cast<uint32_t*>(packed)[u] = word;
    else packed[u] = (uint8_t)word;
  }
}

// ---------------------------------------------------------------- Hadamard
// Randomized Walsh-Hadamard over rows of d elements zero-padded to
// n = next_pow2(d) (hadamard_rotation.rotate, mxtorch.py:2866-2889, and
// _fast_hadamard_transform, mxtorch.py:2811-2832): forward multiplies by the
// sign vector, runs butterflies (u,v)->(u+v,u-v) at half-widths n/2 ... 1,
// then divides by fl32(sqrt(n)); inverse (unrotate, mxtorch.py:2891-2904)
// runs the butterflies, divides, then multiplies by the signs.  Every
// butterfly is an independent IEEE add/sub, so any schedule that keeps the
// level order reproduces the reference bit for bit.
//
// Fused block-128 paths: rows of 128 = one quantization block, a group of 8
// lanes owns a row, 16 elements per lane.  Quantize: the row is loaded in
// line layout (each load instruction of the group covers whole 128-byte
// lines), levels 64..8 run in registers after an LDS transpose (lane holds
// positions li + 8j), levels 4..1 after a second transpose (lane holds 16
// consecutive positions).  Dequantize: the codes of positions li + 8j are
// read directly (1-4 bit codes: every lane of a row loads the row's words;
// 8-bit codes: one 16-byte load per lane and an LDS byte exchange), levels
// 64..8 run in registers, one LDS transpose gives the line layout of the
// stores, level 4 pairs neighbouring lanes (DPP) and levels 2, 1 run in
// registers.
template <int STRIDE_LO, int COUNT>
__device__ __forceinline__ void butterflies(float (&v)[16]) {
  // pairs (j, j + STRIDE_LO) inside groups of 2*STRIDE_LO, over 16 registers
#pragma unroll
  for (int base = 0; base < 16; base += 2 * STRIDE_LO)
#pragma unroll
    for (int j = 0; j < STRIDE_LO; ++j) {
      float u = v[base + j], w = v[base + j + STRIDE_LO];
      v[base + j] = u + w;
      v[base + j + STRIDE_LO] = u - w;
    }
}

// LDS exchange among lanes of one wave (each 8-lane group owns its row of
// LDS): a wave's LDS operations execute in issue order, so ordering the
// compiler is enough; no s_barrier and no wait for the wave's global memory
// operations still in flight.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Forward rotation of one row without the division.  In (fwht128_stage):
// line layout, v[PER16 * q + k] at position 8 * PER16 * q + PER16 * li + k
// (PER16 elements of the input type per 16 bytes).  Out (fwht128_rest):
// natural layout, v[i] at position li * 16 + i.  Bit j of smask is the sign of position li + 8j; the signs
// flip sign bits (exact) before level 64.  row: 128(+pad) floats of LDS.
// fwht128_stage writes the row (line layout) to LDS; fwht128_rest reads it
// back transposed and runs the levels.  Between the two the caller may
// reuse the registers of the input (the next row's loads).
template <int PER16>
__device__ __forceinline__ void fwht128_stage(const float (&v)[16], float* __restrict__ row, int li) {
#pragma unroll
  for (int q = 0; q < 16 / PER16; ++q)
#pragma unroll
    for (int h = 0; h < PER16 / 4; ++h)
      *reinterpret_cast<float4*>(row + 8 * PER16 * q + PER16 * li + 4 * h) =
          make_float4(v[PER16 * q + 4 * h], v[PER16 * q + 4 * h + 1], v[PER16 * q + 4 * h + 2], v[PER16 * q + 4 * h + 3]);
}

__device__ __forceinline__ void fwht128_rest(float (&v)[16], float* __restrict__ row, int li, uint32_t smask) {
  wave_lds_sync();
#pragma unroll
  for (int j = 0; j < 16; ++j) v[j] = row[li + 8 * j];
  // positions li + 8j: level 64 pairs j<->j+8, 32: j<->j+4, 16: j<->j+2, 8: j<->j+1
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float u = __uint_as_float(__float_as_uint(v[j]) ^ ((smask << (31 - j)) & 0x80000000u));
    const float w = __uint_as_float(__float_as_uint(v[j + 8]) ^ ((smask << (23 - j)) & 0x80000000u));
    v[j] = u + w;
    v[j + 8] = u - w;
  }
  butterflies<4, 1>(v);
  butterflies<2, 1>(v);
  butterflies<1, 1>(v);
  wave_lds_sync();
#pragma unroll
  for (int j = 0; j < 16; ++j) row[li + 8 * j] = v[j];
  wave_lds_sync();
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float4 t = *reinterpret_cast<const float4*>(row + li * 16 + 4 * q);
    v[4 * q] = t.x; v[4 * q + 1] = t.y; v[4 * q + 2] = t.z; v[4 * q + 3] = t.w;
  }
  // natural positions li*16 + i: level 4 pairs i<->i+4 (groups of 8), 2, 1
  butterflies<4, 1>(v);
  butterflies<2, 1>(v);
  butterflies<1, 1>(v);
}

// Row of 128 elements in line layout: load q of lane li is the 16 bytes at
// element 8 * PER16 * q + PER16 * li, so the 8 lanes of a row cover whole
// 128-byte lines with each load instruction.
template <typename T>
__device__ __forceinline__ void load_line(const T* __restrict__ x, int64_t row0, int li, int64_t n, float (&v)[16]) {
  constexpr int PER16 = 16 / (int)sizeof(T);
#pragma unroll
  for (int q = 0; q < 16 / PER16; ++q) {
    const int64_t j0 = row0 + 8 * PER16 * q + PER16 * li;
    if (j0 + PER16 <= n) {
      u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x + j0));
      const T* t = reinterpret_cast<const T*>(&w);
#pragma unroll
      for (int k = 0; k < PER16; ++k) v[PER16 * q + k] = ElemT<T>::cvt(t[k]);
    } else {
#pragma unroll
      for (int k = 0; k < PER16; ++k) v[PER16 * q + k] = (j0 + k < n) ? ElemT<T>::cvt(x[j0 + k]) : 0.0f;
    }
  }
}

#define MXK_ROWPAD 132  // 128 + 4 floats: keeps float4 alignment, skews banks per row

template <typename T, int MODE, int BITS>
__global__ __launch_bounds__(256) void k_quant_had128(const T* __restrict__ x, int64_t n, int64_t nb,
                                                      const float* __restrict__ signs,
                                                      uint8_t* __restrict__ packed, int64_t packed_nbytes,
                                                      int64_t n_store, float* __restrict__ scales, float qf,
                                                      QuantSteps st) {
  constexpr int E = 16, LPB = 8, GPW = 8, GPB = 32;
  constexpr int NW = (E * BITS + 31) / 32;
  constexpr int NB = E * BITS / 8;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  constexpr int P16 = 16 / (int)sizeof(T);
  const float* sP = fp_mids<MODE == Q_FP ? BITS : 4>();  // read only by the non-finite path
  __shared__ __attribute__((aligned(16))) float srow[GPB * MXK_ROWPAD];
  __shared__ int2 sK[fp_keys_n<MODE, BITS>()];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane / LPB, li = lane % LPB;
  float* row = srow + (wave * GPW + g) * MXK_ROWPAD;
  const float rdiv = 11.3137083f;           // fl32(sqrt(128))
  const float rinv = 1.0f / 11.3137083f;
  const int64_t rstride = (int64_t)gridDim.x * GPB;
  // Steps of GPB rows as in k_quant_fast: the whole ones load and store
  // through buffer resources based at the step; the next row is loaded into
  // the registers this row leaves once it is staged in LDS (no copy).
  const int64_t b_first = (int64_t)blockIdx.x * GPB;
  const int steps = (int)(st.q_all + (b_first < st.r_all ? 1 : 0));
  const int wholes = (int)(st.q_whole + (b_first <= st.r_whole ? 1 : 0));
  const int r0 = (wave * GPW + g) * 128;  // the row's first element in a step
  auto load_whole_step = [&](int t, float (&v)[E]) {
    const int64_t s0 = b_first + (int64_t)t * rstride;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(x + s0 * 128, (uint32_t)(GPB * 128 * sizeof(T)));
#pragma unroll
    for (int q = 0; q < 16 / P16; ++q) {
      const u32x4 w = buf_load_b128_nt(r, (uint32_t)((r0 + 8 * P16 * q + P16 * li) * sizeof(T)), 0);
      const T* tv = reinterpret_cast<const T*>(&w);
#pragma unroll
      for (int k = 0; k < P16; ++k) v[P16 * q + k] = ElemT<T>::cvt(tv[k]);
    }
  };
  // The division by d of every element: the Markstein quotient, unless some
  // lane holds a nonzero value below 2^-96 (one wave-wide vote, below) and
  // the codes read the quotient's low bits: 1-bit codes its sign, float
  // codes whether it is above 2^-150.  Integer codes of 2+ bits need no
  // vote: the block scale comes from the maximum before the division (a
  // correctly rounded division is monotone, so max RN(|v|/d) = RN(max |v| /
  // d)), and below 2^-96 a quotient (< 2^-99) times the largest multiplier
  // (q / 1e-12 < 2^55) or over the smallest 'v' scale (1e-12 / q > 2^-55)
  // is below 2^-44 on either path: code 0.
  constexpr bool VOTE = MODE == Q_INT1 || MODE == Q_FP;
  auto encode_step = [&](auto whole_c, int t, float (&v)[E]) {
    constexpr bool WHOLE = decltype(whole_c)::value;
    const int64_t s0 = b_first + (int64_t)t * rstride;
    const int64_t blk = s0 + wave * GPW + g;
    const int64_t idx = blk * 128 + (int64_t)li * E;
    // one pass over the magnitudes gives the block maximum and (VOTE) the
    // wave's smallest nonzero magnitude: (bits << 1) - 1 orders the nonzero
    // magnitudes and sends both zeros to 0xFFFFFFFF, so its minimum is below
    // 2 * bits(2^-96) - 1 exactly when some lane holds 0 < |v| < 2^-96.
    uint32_t mxb = 0u;
    uint32_t mnb = 0xFFFFFFFFu;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      mxb = max(mxb, mag_bits(v[i]));
      if constexpr (VOTE) mnb = min(mnb, (__float_as_uint(v[i]) << 1) - 1u);
    }
    const float gmx = __uint_as_float(group_max_u<LPB>(mxb));
    float am;
    if (VOTE && __builtin_expect(__ballot(mnb < 2u * 0x0F800000u - 1u) != 0ull, 0)) {
#pragma unroll
      for (int i = 0; i < E; ++i) v[i] = v[i] / rdiv;
      am = gmx / rdiv;
    } else {
      // Markstein quotient; a zero comes out +0 whatever its sign, which
      // encodes like -0 in every mode (code 0, or the bucket of y <= 0)
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const float q0 = v[i] * rinv;
        v[i] = __builtin_fmaf(__builtin_fmaf(-q0, rdiv, v[i]), rinv, q0);
      }
      am = finite_scale(gmx) ? div_rn(gmx, rdiv, rinv) : gmx;  // inf / d = inf, NaN / d = NaN
    }
    const float ap = amax_clamped(mag_bits(am));
    const BlockParams bp = block_params<MODE>(ap, qf);
    const bool nf = MODE != Q_INT1 && !finite_scale(bp.s);
    uint32_t w[NW];
#pragma unroll
    for (int k = 0; k < NW; ++k) w[k] = 0u;
    if (__builtin_expect(nf, 0)) {
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const uint32_t f = (uint32_t)encode_nonfinite<MODE, BITS>(v[i], bp, qf, sP) & MASK;
        w[(i * BITS) >> 5] |= f << ((i * BITS) & 31);
      }
    } else {
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const uint32_t f = (uint32_t)encode_keyed<MODE, BITS>(v[i], bp, qf, sP, sK) & MASK;
        w[(i * BITS) >> 5] |= f << ((i * BITS) & 31);
      }
    }
    if constexpr (WHOLE) {
      buf_store<NB>(make_rsrc(packed + s0 * (128 * BITS / 8), (uint32_t)(GPB * 128 * BITS / 8)),
                    (uint32_t)((r0 + li * E) * BITS / 8), w);
      if (li == 0) {
        const uint32_t sb = __float_as_uint(bp.s);
        buf_store<4>(make_rsrc(scales + s0, (uint32_t)(GPB * 4)), (uint32_t)((wave * GPW + g) * 4), &sb);
      }
    } else {
      if (idx + E > n_store) clear_tail<NW, BITS>(w, n_store - idx);
      if (blk < nb) {
        store_bytes<NB>(packed, idx * BITS / 8, packed_nbytes, w);
        if (li == 0) scales[blk] = bp.s;
      }
    }
  };
  float vn[E], v[E];
  int t = 0;
  if (wholes > 0) load_whole_step(0, vn);
  uint32_t smask = 0u;  // bit j: the sign of position li + 8j is negative
#pragma unroll
  for (int j = 0; j < E; ++j) smask |= (signs[li + 8 * j] < 0.0f ? 1u : 0u) << j;
  if constexpr (MODE == Q_FP) load_fp_keys<BITS>(sK);
  for (; t < wholes; ++t) {
    fwht128_stage<P16>(vn, row, li);
    if (t + 1 < wholes) load_whole_step(t + 1, vn);
    asm volatile("" : "+v"(smask));  // keeps the sign words out of loop-invariant registers
    fwht128_rest(v, row, li, smask);
    encode_step(std::true_type(), t, v);
  }
  for (; t < steps; ++t) {
    load_line<T>(x, (b_first + (int64_t)t * rstride + wave * GPW + g) * 128, li, n, vn);
    fwht128_stage<P16>(vn, row, li);
    asm volatile("" : "+v"(smask));
    fwht128_rest(v, row, li, smask);
    encode_step(std::false_type(), t, v);
  }
}

// Generic rotation: one workgroup per row, n = next_pow2(d) <= 8192 in LDS.
// FWD: out[r, :d] = (WHT(pad(x[r]) * signs) / sqrt(n))[:d]
// INV: out[r, :d] = (WHT(pad(x[r])) / sqrt(n) * signs)[:d]
template <typename T, bool FWD>
__global__ __launch_bounds__(256) void k_fwht_rows(const T* in, float* out,
                                                   int64_t rows, int64_t d, int n, int logn,
                                                   const float* __restrict__ signs, float rdiv, float rinv) {
  extern __shared__ float sh[];
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      float v = i < d ? ElemT<T>::cvt(in[r * d + i]) : 0.0f;
      if (FWD) v = v * signs[i];
      sh[i] = v;
    }
    __syncthreads();
    for (int lvl = logn - 1; lvl >= 0; --lvl) {
      const int h = 1 << lvl;
      for (int p = threadIdx.x; p < n / 2; p += blockDim.x) {
        int i = ((p >> lvl) << (lvl + 1)) | (p & (h - 1));
        float u = sh[i], w = sh[i + h];
        sh[i] = u + w;
        sh[i + h] = u - w;
      }
      __syncthreads();
    }
    for (int i = threadIdx.x; i < d; i += blockDim.x) {
      float v = div_rn(sh[i], rdiv, rinv);
      if (!FWD) v = v * signs[i];
      out[r * d + i] = v;
    }
    __syncthreads();
  }
}

// Large rotations (n > 8192): the input is first staged into a padded
// [rows, n] float buffer (with signs for FWD), the levels n/2 ... 8192 run
// as global passes, and the last 13 levels plus the division run in LDS.
template <typename T, bool FWD>
__global__ void k_fwht_stage(const T* __restrict__ in, float* __restrict__ buf, int64_t rows, int64_t d,
                             int64_t n, const float* __restrict__ signs) {
  int64_t total = rows * n;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = t / n, i = t % n;
    float v = i < d ? ElemT<T>::cvt(in[r * d + i]) : 0.0f;
    if (FWD) v = v * signs[i];
    buf[t] = v;
  }
}

__global__ void k_fwht_level(float* __restrict__ buf, int64_t rows, int64_t n, int64_t h) {
  int64_t pairs = rows * (n / 2);
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < pairs; t += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = t / (n / 2), p = t % (n / 2);
    int64_t i = (p / h) * (2 * h) + (p % h);
    float* row = buf + r * n;
    float u = row[i], w = row[i + h];
    row[i] = u + w;
    row[i + h] = u - w;
  }
}

// last 13 levels of each 8192-element segment, then division, signs, crop
template <bool FWD>
__global__ __launch_bounds__(256) void k_fwht_tail(const float* __restrict__ buf, float* __restrict__ out,
                                                   int64_t rows, int64_t d, int64_t n,
                                                   const float* __restrict__ signs, float rdiv, float rinv) {
  constexpr int S = 8192;
  extern __shared__ float sh[];
  const int64_t segs = rows * (n / S);
  for (int64_t sgi = blockIdx.x; sgi < segs; sgi += gridDim.x) {
    const int64_t r = sgi / (n / S), off = (sgi % (n / S)) * S;
    const float* src = buf + r * n + off;
    for (int i = threadIdx.x; i < S; i += blockDim.x) sh[i] = src[i];
    __syncthreads();
    for (int lvl = 12; lvl >= 0; --lvl) {
      const int h = 1 << lvl;
      for (int p = threadIdx.x; p < S / 2; p += blockDim.x) {
        int i = ((p >> lvl) << (lvl + 1)) | (p & (h - 1));
        float u = sh[i], w = sh[i + h];
        sh[i] = u + w;
        sh[i + h] = u - w;
      }
      __syncthreads();
    }
    for (int i = threadIdx.x; i < S; i += blockDim.x) {
      int64_t col = off + i;
      if (col < d) {
        float v = div_rn(sh[i], rdiv, rinv);
        if (!FWD) v = v * signs[col];
        out[r * d + col] = v;
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- dequantize
// One lane per 4 outputs.  Fields are read from the packed buffer (only
// bytes below packed_nbytes), sign-extended, and decoded as
//   int: RN(code * s)   int1: code==0 ? s : -s   float: RN(G[idx] * s).
template <int MODE, int BITS>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ packed, int64_t packed_nbytes,
                                                 const float* __restrict__ scales, int64_t nb, int64_t n,
                                                 int block, float* __restrict__ out) {
  constexpr int H = MODE == Q_FP ? (1 << (BITS - 1)) : 1;
  __shared__ float sG[2 * H];
  if constexpr (MODE == Q_FP) build_tables<BITS>(nullptr, sG);
  constexpr bool WORDS = !(BITS == 1 || BITS == 2 || BITS == 4 || BITS == 8);
  constexpr int PER = WORDS ? 32 / BITS : 8 / BITS;
  constexpr uint32_t MASK = BITS >= 32 ? 0xFFFFFFFFu : ((1u << BITS) - 1u);
  const int64_t quads = (n + 3) / 4;
  for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < quads; q += (int64_t)gridDim.x * blockDim.x) {
    float r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t j = q * 4 + i;
      uint32_t f = 0u;
      const int64_t unit = j / PER;
      const int sh = (int)(j % PER) * BITS;
      if (WORDS) {
        if (unit * 4 + 3 < packed_nbytes) f = (reinterpret_cast<const uint32_t*>(packed)[unit] >> sh) & MASK;
      } else {
        if (unit < packed_nbytes) f = ((uint32_t)packed[unit] >> sh) & MASK;
      }
      const int64_t b = j / block;
      const float s = (j < n && b < nb) ? scales[b] : 0.0f;
      float val;
      if constexpr (MODE == Q_INT1) {
        val = f == 0u ? s : -s;
      } else if constexpr (MODE == Q_FP) {
        val = sG[f] * s;
      } else {
        int32_t c = BITS >= 32 ? (int32_t)f : ((int32_t)(f << (32 - BITS)) >> (32 - BITS));
        val = (float)c * s;
      }
      r[i] = val;
    }
    const int64_t j0 = q * 4;
    if (j0 + 4 <= n && ((reinterpret_cast<uintptr_t>(out) & 15u) == 0)) {
      *reinterpret_cast<float4*>(out + j0) = make_float4(r[0], r[1], r[2], r[3]);
    } else {
      for (int i = 0; i < 4; ++i)
        if (j0 + i < n) out[j0 + i] = r[i];
    }
  }
}

// Fast dequantize for bits 1/2/4/8 with blocks that are a multiple of 4: a
// lane decodes slots of 4 consecutive outputs (one 1-4 byte load of its
// codes, one scale) and writes each slot with one 16-byte store, so each
// store instruction of a wave covers 1 KiB of contiguous output.  A thread
// takes U slots a grid-stride apart per iteration, loads first.  Slots that
// cross the end of the data or of the packed buffer take the element path.
template <int MODE, int BITS>
__global__ __launch_bounds__(256) void k_dequant_fast(const uint8_t* __restrict__ packed, int64_t packed_nbytes,
                                                      const float* __restrict__ scales, int64_t nb, int64_t n,
                                                      int block, float* __restrict__ out, DivU32 slots_per_block,
                                                      bool div32) {
  constexpr int U = 4;
  constexpr int H = MODE == Q_FP ? (1 << (BITS - 1)) : 1;
  // int codes of up to 4 bits decode through a table of their values as
  // floats (the same float(code) * s): measured faster than the bit-field
  // extract and conversion; a 256-entry table for int8 codes was slower.
  // FP4 codes read the sorted grid, made by the compiler and copied in
  // (float4d dequantize 182 -> 176-181 us against building it per
  // workgroup); FP8 values are computed (fp8_grid_value): its 256-entry
  // grid in LDS measured 220 -> 276-280 us, the random codes' LDS reads
  // conflicting on the banks
  constexpr bool ITAB = (MODE == Q_INT && BITS <= 4) || MODE == Q_INT1;
  constexpr bool GTAB = MODE == Q_FP && BITS == 4;
  constexpr int TS = ITAB ? (1 << BITS) : 2 * H;
  __shared__ float sG[TS];
  if constexpr (GTAB) load_fp_grid<BITS>(sG);
  if constexpr (ITAB) {
    // int1: code 0 -> +s, 1 -> -s (mxtorch.py:1553-1557), i.e. (+-1) * s exactly
    for (int c = threadIdx.x; c < TS; c += blockDim.x)
      sG[c] = MODE == Q_INT1 ? (c == 0 ? 1.0f : -1.0f)
                             : (float)((int32_t)((uint32_t)c << (32 - BITS)) >> (32 - BITS));
    __syncthreads();
  }
  const int64_t slots = (n + 3) / 4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t s0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; s0 < slots; s0 += U * stride) {
    uint32_t w[U];
    float sc[U];
    bool full[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t sl = s0 + u * stride;
      const int64_t j0 = sl * 4;
      const int64_t last_byte = (j0 + 3) * BITS / 8;  // last byte holding this slot's codes
      full[u] = sl < slots && j0 + 4 <= n && last_byte < packed_nbytes;
      w[u] = 0u;
      if (full[u]) {
        if constexpr (BITS == 8) w[u] = *reinterpret_cast<const uint32_t*>(packed + j0);
        else if constexpr (BITS == 4) w[u] = *reinterpret_cast<const uint16_t*>(packed + j0 / 2);
        else if constexpr (BITS == 2) w[u] = packed[j0 / 4];
        else w[u] = (uint32_t)packed[j0 / 8] >> (j0 & 4);
      }
      // the slot's block: slot / (block / 4) (all 4 of its outputs share it),
      // by multiplication when slot indices fit 32 bits (dequantize at 2^28:
      // int4d 180 -> 174 us, float8d 218 -> 212 us)
      const int64_t b = div32 ? (int64_t)divu32((uint32_t)sl, slots_per_block) : j0 / block;
      sc[u] = (sl < slots && b < nb) ? scales[b] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t sl = s0 + u * stride;
      if (sl >= slots) break;
      const int64_t j0 = sl * 4;
      if (full[u]) {
        f32x4v v;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (ITAB || GTAB) v[i] = sG[(w[u] >> (i * BITS)) & ((1u << BITS) - 1u)] * sc[u];
          else v[i] = decode_field<MODE, BITS>(w[u], i * BITS, sc[u], sG);
        }
        __builtin_nontemporal_store(v, reinterpret_cast<f32x4v*>(out + j0));
      } else {
        for (int i = 0; i < 4; ++i) {
          const int64_t j = j0 + i;
          if (j >= n) break;
          const int64_t unit = j / (8 / BITS);
          const uint32_t f = unit < packed_nbytes ? (uint32_t)packed[unit] : 0u;
          const float sj = (j / block) < nb ? scales[j / block] : 0.0f;
          out[j] = decode_field<MODE, BITS>(f, (int)(j % (8 / BITS)) * BITS, sj, sG);
        }
      }
    }
  }
}

// Fused dequantize + inverse rotation for 'h' dtypes with rows of 128 =
// blocks of 128 (unrotate, mxtorch.py:2891-2904, over the rows quantize
// rotated): out = (WHT(RN(code*s)) / fl32(sqrt 128)) * signs.  The same
// butterflies in the same level order as k_quant_had128; the lane layouts
// are the dequantize ones described above k_quant_had128.
template <int MODE, int BITS>
__global__ __launch_bounds__(256) void k_dequant_had128(const uint8_t* __restrict__ packed, int64_t packed_nbytes,
                                                        const float* __restrict__ scales, int64_t nb,
                                                        const float* __restrict__ signs, float* __restrict__ out) {
  constexpr int E = 16, LPB = 8, GPW = 8, GPB = 32;
  constexpr int RB = 16 * BITS;  // code bytes per row
  constexpr int NWR = RB / 4;    // code words per row
  constexpr int H = MODE == Q_FP ? (1 << (BITS - 1)) : 1;
  __shared__ float sG[2 * H];
  __shared__ __attribute__((aligned(16))) float srow[GPB * MXK_ROWPAD];
  // FP8 grid values from the table here (the arithmetic decode costs ~14
  // VALU per code, a quarter of this kernel's work per element)
  if constexpr (MODE == Q_FP) build_tables<BITS>(nullptr, sG);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane / LPB, li = lane % LPB;
  float* row = srow + (wave * GPW + g) * MXK_ROWPAD;
  float sgl[E];  // signs of the line layout: slot 4q + k is position 32q + 4li + k
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int k = 0; k < 4; ++k) sgl[4 * q + k] = signs[32 * q + 4 * li + k];
  const float pm = (li & 1) ? -1.0f : 1.0f;
  const float rdiv = 11.3137083f;  // fl32(sqrt(128))
  const float rinv = 1.0f / 11.3137083f;
  const int64_t iters = (nb + (int64_t)gridDim.x * GPB - 1) / ((int64_t)gridDim.x * GPB);
  for (int64_t it = 0; it < iters; ++it) {
    const int64_t blk = (it * gridDim.x + blockIdx.x) * GPB + wave * GPW + g;
    const int64_t u0 = blk * RB;
    const bool live = blk < nb;
    const float s = live ? scales[blk] : 0.0f;
    // v[j]: the value of position li + 8j
    float v[E];
    if constexpr (BITS == 8) {
      // lane li loads bytes 16 li .. 16 li + 15 of the row (the row's 8 lanes
      // cover its line with one load instruction), orders them so that
      // halfword h holds bytes h and h + 8, and puts them in its LDS row;
      // lane li then reads halfword li of each lane c: the codes of
      // positions 16c + li and 16c + 8 + li, i.e. j = 2c and 2c + 1
      u32x4 t = {0u, 0u, 0u, 0u};
      if (live && u0 + RB <= packed_nbytes) {
        t = *reinterpret_cast<const u32x4*>(packed + u0 + 16 * li);
      } else if (live) {
        for (int c = 0; c < 16; ++c)
          if (u0 + 16 * li + c < packed_nbytes) t[c >> 2] |= (uint32_t)packed[u0 + 16 * li + c] << (8 * (c & 3));
      }
      u32x4 e;
      e[0] = __builtin_amdgcn_perm(t[2], t[0], 0x05010400u);
      e[1] = __builtin_amdgcn_perm(t[2], t[0], 0x07030602u);
      e[2] = __builtin_amdgcn_perm(t[3], t[1], 0x05010400u);
      e[3] = __builtin_amdgcn_perm(t[3], t[1], 0x07030602u);
      *reinterpret_cast<u32x4*>(row + 4 * li) = e;
      wave_lds_sync();
      const uint16_t* rh = reinterpret_cast<const uint16_t*>(row);
      uint32_t hw[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) hw[c] = rh[8 * c + li];
      wave_lds_sync();
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        if constexpr (MODE == Q_FP) {
          v[2 * c] = sG[hw[c] & 0xFFu] * s;
          v[2 * c + 1] = sG[(hw[c] >> 8) & 0xFFu] * s;
        } else {
          v[2 * c] = decode_field<MODE, BITS>(hw[c], 0, s, sG);
          v[2 * c + 1] = decode_field<MODE, BITS>(hw[c], 8, s, sG);
        }
      }
    } else {
      // word (8j * BITS) / 32 of the row holds position li + 8j; every lane
      // of a row loads the row's words (the same addresses for its 8 lanes)
      uint32_t w[NWR];
#pragma unroll
      for (int k = 0; k < NWR; ++k) w[k] = 0u;
      if (live && u0 + RB <= packed_nbytes) {
#pragma unroll
        for (int k = 0; k < NWR / 4; ++k) {
          const u32x4 t = *reinterpret_cast<const u32x4*>(packed + u0 + 16 * k);
          w[4 * k] = t[0]; w[4 * k + 1] = t[1]; w[4 * k + 2] = t[2]; w[4 * k + 3] = t[3];
        }
      } else if (live) {
#pragma unroll
        for (int k = 0; k < NWR; ++k)
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (u0 + 4 * k + c < packed_nbytes) w[k] |= (uint32_t)packed[u0 + 4 * k + c] << (8 * c);
      }
#pragma unroll
      for (int j = 0; j < E; ++j)
        v[j] = decode_field<MODE, BITS>(w[(8 * j * BITS) >> 5], ((li * BITS) & 31) + ((8 * j * BITS) & 31), s, sG);
    }
    // levels 64, 32, 16, 8: pairs j<->j+8, j+4, j+2, j+1
    butterflies<8, 1>(v);
    butterflies<4, 1>(v);
    butterflies<2, 1>(v);
    butterflies<1, 1>(v);
#pragma unroll
    for (int j = 0; j < E; ++j) row[li + 8 * j] = v[j];
    wave_lds_sync();
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 t = *reinterpret_cast<const float4*>(row + 32 * q + 4 * li);
      v[4 * q] = t.x; v[4 * q + 1] = t.y; v[4 * q + 2] = t.z; v[4 * q + 3] = t.w;
    }
    wave_lds_sync();
    // level 4 pairs lanes li and li^1 at the same slot: the even lane holds u,
    // the odd lane w; u + w = fma(u, 1, w) and u - w = fma(w, -1, u)
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const float p = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v[i]), 0xB1, 0xF, 0xF, true));
      v[i] = __builtin_fmaf(v[i], pm, p);
    }
    // levels 2, 1 inside each slot group of 4
    butterflies<2, 1>(v);
    butterflies<1, 1>(v);
    div_rn_all<E>(v, rdiv, rinv);
    if (live) {
      float* dst = out + blk * 128 + 4 * li;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        __builtin_nontemporal_store(f32x4v{v[4 * q] * sgl[4 * q], v[4 * q + 1] * sgl[4 * q + 1],
                                           v[4 * q + 2] * sgl[4 * q + 2], v[4 * q + 3] * sgl[4 * q + 3]},
                                    reinterpret_cast<f32x4v*>(dst + 32 * q));
    }
  }
}

// ---------------------------------------------------------------- host dispatch
static int grid_for(int64_t work_items, int per_block) {
  int64_t blocks = ceil_div(work_items, per_block);
  int64_t cap = (int64_t)num_cus() * 8;
  return (int)std::max<int64_t>(1, std::min<int64_t>(blocks, cap));
}

// Workgroups for a streaming kernel: one per `per_block` items, at most
// cap_per_cu per CU (0: no cap, every workgroup makes one pass of the
// grid-stride loop).  Measured at 2^28 elements (outputs identical at every
// setting): the light integer quantizers from fp32 stream best uncapped
// (int8d 0.69 -> 0.81 of 8 TB/s), kernels with per-workgroup setup (LDS
// tables) or heavy per-element work at 32-128 per CU.
static int grid_capped(int64_t work_items, int per_block, int cap_per_cu) {
  const int64_t blocks = std::max<int64_t>(1, ceil_div(work_items, per_block));
  if (cap_per_cu <= 0) return (int)std::min<int64_t>(blocks, (int64_t)0x7FFFFFFF);
  return (int)std::min<int64_t>(blocks, (int64_t)num_cus() * cap_per_cu);
}
// k_quant_fast: fp32 int codes uncapped; 16-bit int codes 128 (config 5
// int4d 117 us, 118 uncapped or at 256, 124 at 64); 'v' from 16-bit 64
// (config 5 int8dv 132-135 us against 137-139 at 32, 143 at 128); FP4 codes 384 (float4d at 2^28: 196 us against 212 at 128, 198
// at 256 and 512, 197 uncapped), FP8 codes 192 (float8d 228 us against 233
// at 128, 231 at 160, 238 at 256, 240 at 96); the rest 64.
template <typename T, int MODE, int BITS>
constexpr int quant_fast_cap() {
  return (sizeof(T) == 4 && (MODE == Q_INT || MODE == Q_INT1)) ? 0
         : (sizeof(T) == 2 && (MODE == Q_INT || MODE == Q_INT1)) ? 128
         : (sizeof(T) == 2 && MODE == Q_VEC) ? 64
         : MODE == Q_FP ? (BITS == 4 ? 384 : 192) : 64;
}
// k_dequant_fast: codes decoded without a table (int8, FP8) uncapped; the
// LDS-table widths (int 1-4 bits, FP4) 64.
template <int MODE, int BITS>
constexpr int dequant_fast_cap() {
  return (MODE == Q_INT || MODE == Q_FP) && BITS == 8 ? 0 : 64;
}

// mx_dtype.max_val (mxtorch.py:509-523): q for int widths (1 for int1),
// the format maximum for float widths.  Only the 'v' rule uses it for
// float dtypes.
static float qmax_for(int kind, int bits, int variant) {
  (void)variant;
  if (kind == MXK_KIND_FLOAT) return bits == 4 ? 6.0f : 448.0f;
  if (bits == 1) return 1.0f;
  return (float)((1u << (bits - 1)) - 1u);
}
// The quantizer rule: 'v' rounds to integers clamped at max_val for every
// kind, float dtypes included (mxtorch.py:1739-1752, codes packed as ints);
// otherwise float dtypes bucketize into the grid and int dtypes use
// _quant_int (int1: sign codes).
static int mode_for(int kind, int bits, int variant) {
  if (variant == MXK_VAR_VECTOR) return Q_VEC;
  if (kind == MXK_KIND_FLOAT) return Q_FP;
  if (bits == 1) return Q_INT1;
  return Q_INT;
}

template <typename T, int MODE, int BITS, int E>
static void launch_fast_b(const T* x, int64_t n, int64_t nb, int block, uint8_t* packed, int64_t pbytes,
                          int64_t n_store, float* scales, float qf, hipStream_t st, bool* done) {
  auto go = [&](auto lpb_tag) {
    constexpr int LPB = decltype(lpb_tag)::value;
    constexpr int GPB = 4 * (64 / LPB);
    const int grid = grid_capped(nb, GPB, quant_fast_cap<T, MODE, BITS>());
    const QuantSteps qs = quant_steps(grid, GPB, E * LPB, n, nb, n_store);
    hipLaunchKernelGGL((k_quant_fast<T, E, LPB, MODE, BITS>), dim3(grid), dim3(256), 0, st, x, n, nb, packed, pbytes,
                       n_store, scales, qf, qs);
    *done = true;
  };
  switch (block / E) {
    case 2: go(std::integral_constant<int, 2>()); break;
    case 4: go(std::integral_constant<int, 4>()); break;
    case 8: go(std::integral_constant<int, 8>()); break;
    case 16: go(std::integral_constant<int, 16>()); break;
    case 32: go(std::integral_constant<int, 32>()); break;
    case 64: go(std::integral_constant<int, 64>()); break;
    default: break;
  }
}

template <typename T, int MODE, int BITS, int E>
static bool try_fast_e(const T* x, int64_t n, int64_t nb, int block, uint8_t* packed, int64_t pbytes,
                       int64_t n_store, float* scales, float qf, hipStream_t st) {
  constexpr int PER16 = 16 / (int)sizeof(T);
  constexpr bool NIB = sizeof(T) == 4 && BITS == 1 && E / PER16 > 1;
  constexpr bool SPLIT = E / PER16 > 1 && ((PER16 * BITS) % 8 == 0 || NIB);
  constexpr int CH = SPLIT ? PER16 : E;
  constexpr int NB = NIB ? 1 : CH * BITS / 8;
  if (block % E != 0 || !is_pow2(block / E) || block / E > 64 || block / E < 2) return false;
  if (!aligned16(x) || ((CH * BITS) % 8 != 0 && !NIB) || NB > 16) return false;
  if ((reinterpret_cast<uintptr_t>(packed) % (uintptr_t)NB) != 0) return false;
  bool done = false;
  launch_fast_b<T, MODE, BITS, E>(x, n, nb, block, packed, pbytes, n_store, scales, qf, st, &done);
  return done;
}

// Elements per lane: two 16-byte loads (for fp32 half a block apart), which
// halves the per-element share of the block reduction and scale arithmetic;
// one load when the block is too small for two; 8 consecutive fp32 for 1-bit
// codes (one packed byte per lane); at most 16 packed bytes per lane.
template <typename T, int MODE, int BITS>
static bool try_fast(const T* x, int64_t n, int64_t nb, int block, uint8_t* packed, int64_t pbytes,
                     int64_t n_store, float* scales, float qf, hipStream_t st) {
  constexpr int PER16 = 16 / (int)sizeof(T);
  constexpr int E2x = (8 / BITS) > 2 * PER16 ? (8 / BITS) : 2 * PER16;
  constexpr int E2 = (sizeof(T) == 2 && E2x * BITS > 128) ? PER16 : E2x;
  constexpr int E1 = (8 / BITS) > PER16 ? (8 / BITS) : PER16;
  if (try_fast_e<T, MODE, BITS, E2>(x, n, nb, block, packed, pbytes, n_store, scales, qf, st)) return true;
  if constexpr (E1 != E2) return try_fast_e<T, MODE, BITS, E1>(x, n, nb, block, packed, pbytes, n_store, scales, qf, st);
  return false;
}

template <typename T, int MODE, int BITS>
static bool try_rows(const T* x, int64_t n, int64_t nb, int block, uint8_t* packed, int64_t pbytes,
                     int64_t n_store, float* scales, float qf, hipStream_t st) {
  if (block % 8 != 0 || block <= 256 || block > 8192 || !aligned16(x)) return false;
  if ((reinterpret_cast<uintptr_t>(packed) % (uintptr_t)(BITS >= 16 ? 16 : BITS)) != 0) return false;
  const int chunks = block / 8;
  const dim3 grid((unsigned)std::max<int64_t>(1, std::min<int64_t>(nb, (int64_t)num_cus() * 64)));
  // Blocks of more than 4096 elements take 512 threads of two chunks each:
  // per-token int8 of fp32 [8192, 8192] 58 us against 60 us with 256 x 4.
  if (chunks <= 256)
    hipLaunchKernelGGL((k_quant_rows<T, MODE, BITS, 1, 256>), grid, dim3(256), 0, st, x, n, nb, block, packed,
                       pbytes, n_store, scales, qf);
  else if (chunks <= 512)
    hipLaunchKernelGGL((k_quant_rows<T, MODE, BITS, 2, 256>), grid, dim3(256), 0, st, x, n, nb, block, packed,
                       pbytes, n_store, scales, qf);
  else
    hipLaunchKernelGGL((k_quant_rows<T, MODE, BITS, 2, 512>), grid, dim3(512), 0, st, x, n, nb, block, packed,
                       pbytes, n_store, scales, qf);
  return true;
}

template <typename T, int MODE, int BITS>
static int run_generic(const T* x, int64_t n, int64_t nb, int block, int bits, uint8_t* packed, int64_t pbytes,
                       int64_t n_store, float* scales, float qf, void* ws, size_t ws_bytes, hipStream_t st) {
  if (ws == nullptr || ws_bytes < (size_t)nb * sizeof(float2))
    return fail(MXK_EINVAL, "quantize: workspace too small for the generic path");
  float2* params = reinterpret_cast<float2*>(ws);
  hipLaunchKernelGGL((k_block_params<T, MODE>), dim3(grid_for(nb, 4)), dim3(256), 0, st, x, n, nb, block, qf, scales,
                     params);
  const bool words = !(bits == 1 || bits == 2 || bits == 4 || bits == 8);
  const int64_t units = words ? pbytes / 4 : pbytes;
  hipLaunchKernelGGL((k_pack_generic<T, MODE, BITS>), dim3(grid_for(units, 256)), dim3(256), 0, st, x, n, block, qf,
                     params, bits, n_store, packed, pbytes);
  return check_launch("quantize(generic)");
}

template <typename T>
static int quantize_t(const T* x, int64_t n, int kind, int bits, int variant, int block, uint8_t* packed,
                      int64_t pbytes, float* scales, int64_t n_store, void* ws, size_t ws_bytes, hipStream_t st) {
  const int64_t nb = ceil_div(n, block);
  const int mode = mode_for(kind, bits, variant);
  const float qf = qmax_for(kind, bits, variant);
#define MXK_TRY(MODE, BITS)                                                                               \
  if (mode == MODE && bits == BITS) {                                                                     \
    if (try_fast<T, MODE, BITS>(x, n, nb, block, packed, pbytes, n_store, scales, qf, st))               \
      return check_launch("quantize");                                                                    \
    if (try_rows<T, MODE, BITS>(x, n, nb, block, packed, pbytes, n_store, scales, qf, st))               \
      return check_launch("quantize(rows)");                                                              \
    return run_generic<T, MODE, BITS>(x, n, nb, block, bits, packed, pbytes, n_store, scales, qf, ws, ws_bytes, st); \
  }
  MXK_TRY(Q_INT, 2)
  MXK_TRY(Q_INT, 4)
  MXK_TRY(Q_INT, 8)
  MXK_TRY(Q_INT, 16)
  MXK_TRY(Q_INT1, 1)
  MXK_TRY(Q_VEC, 2)
  MXK_TRY(Q_VEC, 4)
  MXK_TRY(Q_VEC, 8)
  MXK_TRY(Q_VEC, 16)
  MXK_TRY(Q_FP, 4)
  MXK_TRY(Q_FP, 8)
#undef MXK_TRY
#define MXK_GEN(MODE, BITS) \
  if (mode == MODE && bits == BITS) return run_generic<T, MODE, BITS>(x, n, nb, block, bits, packed, pbytes, n_store, scales, qf, ws, ws_bytes, st);
  MXK_GEN(Q_INT, 3)
  MXK_GEN(Q_INT, 5)
  MXK_GEN(Q_INT, 6)
  MXK_GEN(Q_INT, 7)
  MXK_GEN(Q_VEC, 1)
  MXK_GEN(Q_VEC, 3)
  MXK_GEN(Q_VEC, 5)
  MXK_GEN(Q_VEC, 6)
  MXK_GEN(Q_VEC, 7)
#undef MXK_GEN
  return fail(MXK_EUNSUPPORTED, "quantize: unsupported kind/bits/variant combination");
}

template <typename T>
static bool try_had128(const T* x, int64_t n, int mode, int bits, const float* signs, uint8_t* packed,
                       int64_t pbytes, int64_t n_store, float* scales, float qf, hipStream_t st) {
  if (!aligned16(x)) return false;
  const int64_t nb = ceil_div(n, 128);
  // 256 workgroups per CU: int4dh at 2^28 193 us against 199 at 128, 210
  // at 64, 195 uncapped
  const int grid = grid_capped(nb, 32, 256);
  const QuantSteps qs = quant_steps(grid, 32, 128, n, nb, n_store);
#define MXK_HAD_CASE(MODE, BITS)                                                                               \
  if (mode == MODE && bits == BITS) {                                                                          \
    hipLaunchKernelGGL((k_quant_had128<T, MODE, BITS>), dim3(grid), dim3(256), 0, st, x, n, nb, signs, packed, \
                       pbytes, n_store, scales, qf, qs);                                                       \
    return true;                                                                                               \
  }
  MXK_HAD_CASE(Q_INT, 2)
  MXK_HAD_CASE(Q_INT, 4)
  MXK_HAD_CASE(Q_INT, 8)
  MXK_HAD_CASE(Q_INT1, 1)
  MXK_HAD_CASE(Q_FP, 4)
  MXK_HAD_CASE(Q_FP, 8)
#undef MXK_HAD_CASE
  return false;
}

// Rotate rows of d (padded to n) into a float buffer `rot` [rows, d].
template <typename T, bool FWD>
static int rotate_rows(const T* in, float* rot, int64_t rows, int64_t d, const float* signs, void* ws,
                       size_t ws_bytes, hipStream_t st) {
  const int64_t n = next_pow2(d);
  int logn = 0;
  while ((int64_t(1) << logn) < n) ++logn;
  const float rdiv = (float)std::sqrt((double)n);
  const float rinv = 1.0f / rdiv;
  if (n <= 8192) {
    const int grid = (int)std::min<int64_t>(rows, (int64_t)num_cus() * 8);
    hipLaunchKernelGGL((k_fwht_rows<T, FWD>), dim3(std::max(grid, 1)), dim3(256), n * sizeof(float), st, in, rot, rows,
                       d, (int)n, logn, signs, rdiv, rinv);
    return check_launch("rotate");
  }
  if (ws == nullptr || ws_bytes < (size_t)(rows * n) * sizeof(float))
    return fail(MXK_EINVAL, "rotation: workspace too small");
  float* buf = reinterpret_cast<float*>(ws);
  const int g = grid_for(rows * n, 256);
  hipLaunchKernelGGL((k_fwht_stage<T, FWD>), dim3(g), dim3(256), 0, st, in, buf, rows, d, n, signs);
  for (int64_t h = n / 2; h >= 8192; h /= 2)
    hipLaunchKernelGGL(k_fwht_level, dim3(grid_for(rows * n / 2, 256)), dim3(256), 0, st, buf, rows, n, h);
  const int gt = (int)std::min<int64_t>(rows * (n / 8192), (int64_t)num_cus() * 4);
  hipLaunchKernelGGL((k_fwht_tail<FWD>), dim3(gt), dim3(256), 8192 * sizeof(float), st, buf, rot, rows, d, n, signs,
                     rdiv, rinv);
  return check_launch("rotate(large)");
}

static size_t rot_ws_bytes(int64_t n, int64_t d) {
  // rotated copy [n] floats + staging [rows, next_pow2(d)] when next_pow2(d) > 8192
  const int64_t np = next_pow2(d);
  size_t bytes = (size_t)n * sizeof(float);
  if (np > 8192) bytes += (size_t)(n / d) * (size_t)np * sizeof(float);
  return bytes;
}

template <int MODE, int BITS>
static int launch_dequant(const void* packed, int64_t pbytes, const float* scales, int64_t nb, int64_t n, int block,
                          float* out, hipStream_t st) {
  if constexpr (BITS == 1 || BITS == 2 || BITS == 4 || BITS == 8) {
    if (block % 4 == 0 && (reinterpret_cast<uintptr_t>(packed) & 3u) == 0 &&
        (reinterpret_cast<uintptr_t>(out) & 15u) == 0) {
      const int64_t slots = ceil_div(n, 4);
      const int grid = grid_capped(slots, 256 * 4, dequant_fast_cap<MODE, BITS>());
      // every slot index a thread forms (sl + u * stride) stays below 2^32
      const bool div32 = slots + 4ll * grid * 256 < (1ll << 32);
      hipLaunchKernelGGL((k_dequant_fast<MODE, BITS>), dim3(grid), dim3(256), 0, st,
                         reinterpret_cast<const uint8_t*>(packed), pbytes, scales, nb, n, block, out,
                         make_divu32((uint32_t)(block / 4)), div32);
      return check_launch("dequantize");
    }
  }
  hipLaunchKernelGGL((k_dequant<MODE, BITS>), dim3(grid_for(ceil_div(n, 4), 256)), dim3(256), 0, st,
                     reinterpret_cast<const uint8_t*>(packed), pbytes, scales, nb, n, block, out);
  return check_launch("dequantize");
}

// 64 workgroups per CU at most (measured at 2^28 against 8, 16, 32, 128 and
// uncapped: int8dh 310 -> 285 us, int4dh 215 -> 200, outputs identical)
template <int MODE, int BITS>
static int launch_dequant_had128(const void* packed, int64_t pbytes, const float* scales, int64_t nb,
                                 const float* signs, float* out, hipStream_t st) {
  const int grid = grid_capped(nb, 32, 64);
  hipLaunchKernelGGL((k_dequant_had128<MODE, BITS>), dim3(grid), dim3(256), 0, st,
                     reinterpret_cast<const uint8_t*>(packed), pbytes, scales, nb, signs, out);
  return check_launch("dequantize(hadamard128)");
}

bool vec_rows_i32(const void* x, int x_type, int64_t rows, int64_t cols, int bits, int32_t* codes, float* scales,
                  hipStream_t st) {
  if ((reinterpret_cast<uintptr_t>(codes) & 15u) != 0) return false;
  const float qf = (float)((1u << (bits - 1)) - 1u);
  const int64_t n = rows * cols;
  if (cols > 8192) return false;
  uint8_t* pk = reinterpret_cast<uint8_t*>(codes);
  if (x_type == MXK_IN_F32)
    return try_rows<float, Q_VEC, 32>((const float*)x, n, rows, (int)cols, pk, n * 4, n, scales, qf, st);
  if (x_type == MXK_IN_F16)
    return try_rows<__half, Q_VEC, 32>((const __half*)x, n, rows, (int)cols, pk, n * 4, n, scales, qf, st);
  return try_rows<hip_bfloat16, Q_VEC, 32>((const hip_bfloat16*)x, n, rows, (int)cols, pk, n * 4, n, scales, qf, st);
}

int requant_vec_f32(const float* x, int64_t n, int bits, int block, void* packed, int64_t packed_nbytes,
                    float* scales, int64_t n_store, void* ws, size_t ws_bytes, hipStream_t st) {
  return quantize_t<float>(x, n, MXK_KIND_INT, bits, MXK_VAR_VECTOR, block, reinterpret_cast<uint8_t*>(packed),
                           packed_nbytes, scales, n_store, ws, ws_bytes, st);
}

}  // namespace mxk

using namespace mxk;

extern "C" {

int mxk_abi_version(void) { return MXK_ABI_VERSION; }

const char* mxk_last_error(void) { return g_err.c_str(); }

int64_t mxk_packed_nbytes(int bits, int64_t n_codes) {
  if (n_codes < 0 || bits <= 0 || bits > 16) return -1;
  if (bits == 1 || bits == 2 || bits == 4 || bits == 8) return ceil_div(n_codes, 8 / bits);
  return 4 * ceil_div(n_codes, 32 / bits);
}

int mxk_float_grid(int bits, float* grid, float* mids) {
  if (bits != 4 && bits != 8) return fail(MXK_EUNSUPPORTED, "float grid: bits must be 4 or 8");
  const int H = 1 << (bits - 1);
  std::vector<float> g(H);
  for (int c = 0; c < H; ++c) g[c] = fmt_value(bits, c) / fmt_max(bits);
  if (grid) {
    for (int c = 0; c < H; ++c) {
      grid[H + c] = g[c];
      grid[H - 1 - c] = -g[c];
    }
  }
  if (mids) {
    for (int j = 1; j < H; ++j) {
      float s = g[j - 1] + g[j];
      mids[H - 1 + j] = s * 0.5f;
      mids[H - 1 - j] = -(s * 0.5f);
    }
    mids[H - 1] = 0.0f;
  }
  return MXK_OK;
}

size_t mxk_quantize_workspace(int64_t n, int kind, int bits, int variant, int block, int64_t rot_dim) {
  (void)kind;
  (void)bits;
  if (n <= 0 || block <= 0) return 0;
  size_t bytes = (size_t)ceil_div(n, block) * sizeof(float2) + 256;
  if (variant == MXK_VAR_HADAMARD && rot_dim > 0) bytes += rot_ws_bytes(n, rot_dim) + 256;
  return bytes;
}

int mxk_quantize(const void* x, int x_type, int64_t n, int kind, int bits, int variant, int block,
                 const float* signs, int64_t rot_dim, void* packed, int64_t packed_nbytes, float* scales,
                 int64_t n_store, void* workspace, size_t workspace_nbytes, void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (n <= 0) return fail(MXK_EINVAL, "quantize: n must be positive");
  if (block <= 0) return fail(MXK_EINVAL, "quantize: block must be positive");
  if (!x || !packed || !scales) return fail(MXK_EINVAL, "quantize: null pointer");
  if (kind == MXK_KIND_FLOAT && bits != 4 && bits != 8)
    return fail(MXK_EUNSUPPORTED, "quantize: float kinds support bits 4 and 8");
  if (kind == MXK_KIND_INT && !((bits >= 1 && bits <= 8) || bits == 16))
    return fail(MXK_EUNSUPPORTED, "quantize: int kinds support bits 1..8 and 16");
  const int64_t nb = ceil_div(n, block);
  if (n_store < 0 || n_store > nb * block) return fail(MXK_EINVAL, "quantize: n_store out of range");
  if (packed_nbytes < mxk_packed_nbytes(bits, n_store)) return fail(MXK_EINVAL, "quantize: packed buffer too small");
  if (x_type != MXK_IN_F32 && x_type != MXK_IN_F16 && x_type != MXK_IN_BF16)
    return fail(MXK_EINVAL, "quantize: bad input type");
  uint8_t* pk = reinterpret_cast<uint8_t*>(packed);
  const int mode = mode_for(kind, bits, variant);
  const float qf = qmax_for(kind, bits, variant);

  if (variant == MXK_VAR_HADAMARD) {
    if (!signs || rot_dim <= 0 || n % rot_dim != 0)
      return fail(MXK_EINVAL, "quantize: hadamard needs signs and a rot_dim dividing n");
    if (rot_dim == 128 && block == 128) {
      bool ok = false;
      if (x_type == MXK_IN_F32) ok = try_had128<float>((const float*)x, n, mode, bits, signs, pk, packed_nbytes, n_store, scales, qf, st);
      else if (x_type == MXK_IN_F16) ok = try_had128<__half>((const __half*)x, n, mode, bits, signs, pk, packed_nbytes, n_store, scales, qf, st);
      else ok = try_had128<hip_bfloat16>((const hip_bfloat16*)x, n, mode, bits, signs, pk, packed_nbytes, n_store, scales, qf, st);
      if (ok) return check_launch("quantize(hadamard128)");
    }
    // rotate into the workspace, then quantize the float32 rotated copy
    const size_t need = mxk_quantize_workspace(n, kind, bits, variant, block, rot_dim);
    if (!workspace || workspace_nbytes < need) return fail(MXK_EINVAL, "quantize: workspace too small");
    uint8_t* wsb = reinterpret_cast<uint8_t*>(workspace);
    const size_t pbytes_params = ((size_t)nb * sizeof(float2) + 255) & ~(size_t)255;
    float* rot = reinterpret_cast<float*>(wsb + pbytes_params);
    void* stage = wsb + pbytes_params + (((size_t)n * sizeof(float) + 255) & ~(size_t)255);
    size_t stage_bytes = workspace_nbytes - (pbytes_params + (((size_t)n * sizeof(float) + 255) & ~(size_t)255));
    const int64_t rows = n / rot_dim;
    int rc;
    if (x_type == MXK_IN_F32) rc = rotate_rows<float, true>((const float*)x, rot, rows, rot_dim, signs, stage, stage_bytes, st);
    else if (x_type == MXK_IN_F16) rc = rotate_rows<__half, true>((const __half*)x, rot, rows, rot_dim, signs, stage, stage_bytes, st);
    else rc = rotate_rows<hip_bfloat16, true>((const hip_bfloat16*)x, rot, rows, rot_dim, signs, stage, stage_bytes, st);
    if (rc != MXK_OK) return rc;
    return quantize_t<float>(rot, n, kind, bits, MXK_VAR_BASE, block, pk, packed_nbytes, scales, n_store, wsb,
                             pbytes_params, st);
  }
  if (variant != MXK_VAR_BASE && variant != MXK_VAR_VECTOR) return fail(MXK_EUNSUPPORTED, "quantize: bad variant");
  (void)mode;
  (void)qf;
  if (x_type == MXK_IN_F32)
    return quantize_t<float>((const float*)x, n, kind, bits, variant, block, pk, packed_nbytes, scales, n_store,
                             workspace, workspace_nbytes, st);
  if (x_type == MXK_IN_F16)
    return quantize_t<__half>((const __half*)x, n, kind, bits, variant, block, pk, packed_nbytes, scales, n_store,
                              workspace, workspace_nbytes, st);
  return quantize_t<hip_bfloat16>((const hip_bfloat16*)x, n, kind, bits, variant, block, pk, packed_nbytes, scales,
                                  n_store, workspace, workspace_nbytes, st);
}

int mxk_dequantize(const void* packed, int64_t packed_nbytes, const float* scales, int64_t nb, int64_t n, int kind,
                   int bits, int variant, int block, const float* signs, int64_t rot_dim, float* out,
                   void* workspace, size_t workspace_nbytes, void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (n <= 0 || block <= 0 || nb <= 0) return fail(MXK_EINVAL, "dequantize: sizes must be positive");
  if (!packed || !scales || !out) return fail(MXK_EINVAL, "dequantize: null pointer");
  const int mode = mode_for(kind, bits, variant == MXK_VAR_VECTOR ? MXK_VAR_BASE : variant);
  if (variant == MXK_VAR_HADAMARD && rot_dim == 128 && block == 128 && n % 128 == 0 && nb == n / 128 && signs &&
      (reinterpret_cast<uintptr_t>(out) & 15u) == 0 && (reinterpret_cast<uintptr_t>(packed) & 15u) == 0) {
#define MXK_DH(MODE, BITS) \
    if (mode == MODE && bits == BITS) return launch_dequant_had128<MODE, BITS>(packed, packed_nbytes, scales, nb, signs, out, st);
    MXK_DH(Q_INT1, 1)
    MXK_DH(Q_INT, 2)
    MXK_DH(Q_INT, 4)
    MXK_DH(Q_INT, 8)
    MXK_DH(Q_FP, 4)
    MXK_DH(Q_FP, 8)
#undef MXK_DH
  }
  int rc = MXK_EUNSUPPORTED;
#define MXK_D(MODE, BITS) \
  else if (mode == MODE && bits == BITS) rc = launch_dequant<MODE, BITS>(packed, packed_nbytes, scales, nb, n, block, out, st);
  if (false) {
  }
  MXK_D(Q_INT1, 1)
  MXK_D(Q_INT, 2)
  MXK_D(Q_INT, 3)
  MXK_D(Q_INT, 4)
  MXK_D(Q_INT, 5)
  MXK_D(Q_INT, 6)
  MXK_D(Q_INT, 7)
  MXK_D(Q_INT, 8)
  MXK_D(Q_INT, 16)
  MXK_D(Q_FP, 4)
  MXK_D(Q_FP, 8)
  else return fail(MXK_EUNSUPPORTED, "dequantize: unsupported kind/bits");
#undef MXK_D
  if (rc != MXK_OK) return rc;
  if (variant == MXK_VAR_HADAMARD) {
    if (!signs || rot_dim <= 0 || n % rot_dim != 0)
      return fail(MXK_EINVAL, "dequantize: hadamard needs signs and a rot_dim dividing n");
    // in-place unrotation of out viewed as [n/rot_dim, rot_dim]
    const int64_t np = next_pow2(rot_dim);
    if (np <= 8192) return rotate_rows<float, false>(out, out, n / rot_dim, rot_dim, signs, nullptr, 0, st);
    if (!workspace || workspace_nbytes < (size_t)(n / rot_dim) * (size_t)np * sizeof(float))
      return fail(MXK_EINVAL, "dequantize: workspace too small for the large rotation");
    return rotate_rows<float, false>(out, out, n / rot_dim, rot_dim, signs, workspace, workspace_nbytes, st);
  }
  return MXK_OK;
}

size_t mxk_dequantize_workspace(int64_t n, int variant, int64_t rot_dim) {
  if (variant != MXK_VAR_HADAMARD || rot_dim <= 0) return 0;
  const int64_t np = next_pow2(rot_dim);
  if (np <= 8192) return 0;
  return (size_t)(n / rot_dim) * (size_t)np * sizeof(float);
}

}  // extern "C"
