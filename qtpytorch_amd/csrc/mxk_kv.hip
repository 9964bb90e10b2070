// KV-cache ring buffer for gfx950: the streaming form of kv_cache_quantizer
// (mxtorch.py:2998-3090).
//
// The reference keeps a Python list of per-step mx_tensors and, per step,
// runs k.float(), a reshape to [B*H, D], quantize(k_f, dt, D); for V (when
// asymmetric) v_min = row min, v_f - v_min, quantize(..., D), and keeps
// v_min as the zero point (mxtorch.py:3039-3067).  get() dequantizes every
// step, stacks them along time and adds the zero points back to V
// (mxtorch.py:3069-3086).
//
// Here the caller owns a ring of slots (codes, scales, zero points of one
// step each).  k_kv_append quantizes one step's K and V rows straight into
// their slot in one launch; k_kv_gather dequantizes a window of slots back
// to float32 [rows, T, D] in time order in one launch per tensor.  Both use
// the arithmetic of the block quantizer with block = D (one block per row).
#include "mxk_internal.h"

namespace mxk {

// One row of D = 8 * LPB elements per group of LPB lanes; rows [0, rows)
// are K's, rows [rows, 2 * rows) V's.  Every lane runs the reductions (the
// DPP lane exchanges read the whole group); tasks past the end recompute the
// last row and store nothing.
template <typename T, int LPB, int MODE, int BITS>
__global__ __launch_bounds__(256) void k_kv_append(const T* __restrict__ k, const T* __restrict__ v, int64_t rows,
                                                   int asym, uint8_t* __restrict__ kc, float* __restrict__ ks,
                                                   uint8_t* __restrict__ vc, float* __restrict__ vs,
                                                   float* __restrict__ zp, float qf) {
  constexpr int E = 8, D = E * LPB, GPW = 64 / LPB;
  constexpr int NB = E * BITS / 8;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  constexpr int H = MODE == Q_FP ? (1 << (BITS - 1)) : 1;
  __shared__ float sP[H + 1];
  if constexpr (MODE == Q_FP && BITS != 4) build_tables<BITS>(sP, nullptr);  // FP4 buckets by constants

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane / LPB, li = lane % LPB;
  const int64_t task = ((int64_t)blockIdx.x * 4 + wave) * GPW + g;
  const bool live = task < 2 * rows;
  const int64_t tk = live ? task : 2 * rows - 1;
  const bool is_v = tk >= rows;
  const int64_t r = is_v ? tk - rows : tk;
  float x[E];
  load_elems<T, E>(is_v ? v : k, r * D + (int64_t)li * E, rows * D, x);
  // V's row minimum (an exact comparison), subtracted in float32 as
  // v_f - v_min (mxtorch.py:3062-3063)
  float mn = x[0];
#pragma unroll
  for (int i = 1; i < E; ++i) mn = fminf(mn, x[i]);
  mn = -group_max<LPB>(-mn);
  const bool shift = is_v && asym;
  if (shift) {
#pragma unroll
    for (int i = 0; i < E; ++i) x[i] = x[i] - mn;
  }
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < E; ++i) m = fmaxf(m, __builtin_fabsf(x[i]));
  const float ap = fmaxf(group_max<LPB>(m), MXK_AMIN);
  const BlockParams bp = block_params<MODE>(ap, qf);
  uint32_t w[(NB + 3) / 4];
#pragma unroll
  for (int q = 0; q < (NB + 3) / 4; ++q) w[q] = 0u;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const uint32_t f = (uint32_t)encode<MODE, BITS>(x[i], bp, qf, sP) & MASK;
    w[(i * BITS) >> 5] |= f << ((i * BITS) & 31);
  }
  if (live) {
    uint8_t* dst = is_v ? vc : kc;
    store_bytes<NB>(dst, (r * D + (int64_t)li * E) * BITS / 8, rows * D * BITS / 8, w);
    if (li == 0) {
      (is_v ? vs : ks)[r] = bp.s;
      if (shift) zp[r] = mn;
    }
  }
}

// out[r][j][d] for r < rows, j < T, d < D: slot (start + j) mod cap, decoded
// as the dequantizer does (int: RN(c*s); int1: +-s; float: RN(G[c]*s)),
// plus the slot's zero point when zp is given (RN(dq + zp), mxtorch.py:3083).
// Tiles of KV_RT rows x KV_JT steps per block (row tiles on grid-x, step
// tiles on grid-y, both looped): each thread writes float4s (4 codes, read
// from the 32-bit word holding them); a tile reads KV_RT consecutive rows of
// each of its slots and writes KV_RT runs of KV_JT * D contiguous floats.
// D = 4 << LQ.  A thread issues the loads of all its IT items of a tile
// (code word, scale, zero point) before it decodes and stores any of them.
// rows * D * BITS < 2^35 and T < 2^31 (host-checked).
#define KV_RT 4
#define KV_JT 8
template <int MODE, int BITS, int LQ>
__global__ __launch_bounds__(256) void k_kv_gather(const uint8_t* __restrict__ codes, const float* __restrict__ scales,
                                                   const float* __restrict__ zp, int64_t rows, int64_t cap,
                                                   int64_t start, int64_t T, float* __restrict__ out) {
  constexpr int H = (MODE == Q_FP && BITS == 4) ? 16 : 1;
  constexpr int QPR = 1 << LQ;            // float4s per (row, step): 16, 32 or 64
  constexpr int LJQ = LQ + 3;             // log2(KV_JT * QPR)
  constexpr int IT = KV_RT * KV_JT * QPR / 256;
  constexpr int D = 4 * QPR;
  __shared__ float sG[H];
  if constexpr (MODE == Q_FP && BITS == 4) build_tables<4>(nullptr, sG);
  const int64_t slot_bytes = rows * (D * BITS / 8);
  const int64_t ntr = (rows + KV_RT - 1) / KV_RT, ntj = (T + KV_JT - 1) / KV_JT;
  for (int64_t tj = blockIdx.y; tj < ntj; tj += gridDim.y) {
    for (int64_t tr = blockIdx.x; tr < ntr; tr += gridDim.x) {
      uint32_t word[IT];
      float s[IT], z[IT];
      int64_t dst[IT];
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const uint32_t t = threadIdx.x + 256u * it;
        const uint32_t rr = t >> LJQ, jj = (t >> LQ) & (KV_JT - 1), q = t & (QPR - 1);
        const int64_t r = tr * KV_RT + rr, j = tj * KV_JT + jj;
        word[it] = 0u;
        s[it] = 0.0f;
        z[it] = 0.0f;
        dst[it] = -1;
        if (r < rows && j < T) {
          int64_t slot = start + j;
          if (slot >= cap) slot -= cap;
          const int64_t bit0 = ((int64_t)r * D + 4 * q) * BITS;
          word[it] = *reinterpret_cast<const uint32_t*>(codes + slot * slot_bytes + (bit0 >> 5) * 4);
          s[it] = scales[slot * rows + r];
          if (zp) z[it] = zp[slot * rows + r];
          dst[it] = ((r * T + j) << (LQ + 2)) + q * 4;
        }
      }
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        if (dst[it] < 0) continue;
        const int sh0 = (int)((((threadIdx.x + 256u * it) & (QPR - 1)) * 4 * BITS) & 31);
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = decode_field<MODE, BITS>(word[it], sh0 + e * BITS, s[it], sG);
        if (zp) {
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = o[e] + z[it];
        }
        __builtin_nontemporal_store(f32x4v{o[0], o[1], o[2], o[3]}, reinterpret_cast<f32x4v*>(out + dst[it]));
      }
    }
  }
}

// Quantizer rule, decode rule and max_val for the dtypes the kernels cover
// (the rules of mxk_quantize / mxk_dequantize): 'v' rounds to integers for
// every kind and decodes like the base dtype (mxtorch.py:1739-1752,
// 1573-1575); Hadamard dtypes and the int32-word widths are not covered.
static bool kv_mode(int kind, int bits, int variant, int& qmode, int& dmode, float& qf) {
  if (variant == MXK_VAR_HADAMARD) return false;
  const bool fl = kind == MXK_KIND_FLOAT;
  if (fl ? !(bits == 4 || bits == 8) : !(bits == 1 || bits == 2 || bits == 4 || bits == 8)) return false;
  if (variant == MXK_VAR_VECTOR && bits == 1) return false;
  qf = fl ? (bits == 4 ? 6.0f : 448.0f) : (bits == 1 ? 1.0f : (float)((1u << (bits - 1)) - 1u));
  dmode = fl ? Q_FP : (bits == 1 ? Q_INT1 : Q_INT);
  qmode = variant == MXK_VAR_VECTOR ? Q_VEC : dmode;
  return true;
}

template <typename T, int LPB>
static void launch_append_t(int mode, int bits, const void* k, const void* v, int64_t rows, int asym, void* kc,
                            float* ks, void* vc, float* vs, float* zp, float qf, hipStream_t st) {
  const int64_t per_block = 4 * (64 / LPB);
  const dim3 grid((unsigned)ceil_div(2 * rows, per_block));
  const T* kt = reinterpret_cast<const T*>(k);
  const T* vt = reinterpret_cast<const T*>(v);
  uint8_t* kb = reinterpret_cast<uint8_t*>(kc);
  uint8_t* vb = reinterpret_cast<uint8_t*>(vc);
#define MXK_KVA(MODE, BITS)                                                                                    \
  hipLaunchKernelGGL((k_kv_append<T, LPB, MODE, BITS>), grid, dim3(256), 0, st, kt, vt, rows, asym, kb, ks, vb, vs, \
                     zp, qf)
  if (mode == Q_FP) {
    if (bits == 4) MXK_KVA(Q_FP, 4);
    else MXK_KVA(Q_FP, 8);
  } else if (mode == Q_INT1) {
    MXK_KVA(Q_INT1, 1);
  } else if (mode == Q_VEC) {
    if (bits == 2) MXK_KVA(Q_VEC, 2);
    else if (bits == 4) MXK_KVA(Q_VEC, 4);
    else MXK_KVA(Q_VEC, 8);
  } else {
    if (bits == 2) MXK_KVA(Q_INT, 2);
    else if (bits == 4) MXK_KVA(Q_INT, 4);
    else MXK_KVA(Q_INT, 8);
  }
#undef MXK_KVA
}

template <typename T>
static int launch_append(int head_dim, int mode, int bits, const void* k, const void* v, int64_t rows, int asym,
                         void* kc, float* ks, void* vc, float* vs, float* zp, float qf, hipStream_t st) {
  if (head_dim == 64) launch_append_t<T, 8>(mode, bits, k, v, rows, asym, kc, ks, vc, vs, zp, qf, st);
  else if (head_dim == 128) launch_append_t<T, 16>(mode, bits, k, v, rows, asym, kc, ks, vc, vs, zp, qf, st);
  else launch_append_t<T, 32>(mode, bits, k, v, rows, asym, kc, ks, vc, vs, zp, qf, st);
  return check_launch("kv_append");
}

}  // namespace mxk

using namespace mxk;

extern "C" {

int mxk_kv_append(const void* k, const void* v, int x_type, int64_t rows, int head_dim, int kind, int bits,
                  int variant, int asymmetric_v, void* k_codes, float* k_scales, void* v_codes, float* v_scales,
                  float* v_zero_point, void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  int mode = 0, dmode = 0;
  float qf = 0.0f;
  if (rows <= 0) return fail(MXK_EINVAL, "kv_append: rows must be positive");
  if (!(head_dim == 64 || head_dim == 128 || head_dim == 256))
    return fail(MXK_EUNSUPPORTED, "kv_append: head_dim must be 64, 128 or 256");
  if (!kv_mode(kind, bits, variant, mode, dmode, qf))
    return fail(MXK_EUNSUPPORTED, "kv_append: int widths 1, 2, 4, 8 and float 4, 8 (base or 'v') only");
  if (!k || !v || !k_codes || !k_scales || !v_codes || !v_scales || (asymmetric_v && !v_zero_point))
    return fail(MXK_EINVAL, "kv_append: null pointer");
  if (!aligned16(k) || !aligned16(v)) return fail(MXK_EINVAL, "kv_append: k and v must be 16-byte aligned");
  if (rows * head_dim * bits / 8 >= ((int64_t)1 << 40)) return fail(MXK_EINVAL, "kv_append: slot too large");
  if (x_type == MXK_IN_F32)
    return launch_append<float>(head_dim, mode, bits, k, v, rows, asymmetric_v, k_codes, k_scales, v_codes,
                                v_scales, v_zero_point, qf, st);
  if (x_type == MXK_IN_F16)
    return launch_append<__half>(head_dim, mode, bits, k, v, rows, asymmetric_v, k_codes, k_scales, v_codes,
                                 v_scales, v_zero_point, qf, st);
  if (x_type == MXK_IN_BF16)
    return launch_append<hip_bfloat16>(head_dim, mode, bits, k, v, rows, asymmetric_v, k_codes, k_scales,
                                       v_codes, v_scales, v_zero_point, qf, st);
  return fail(MXK_EINVAL, "kv_append: unknown x_type");
}

int mxk_kv_gather(const void* codes, const float* scales, const float* zero_point, int64_t rows, int head_dim,
                  int kind, int bits, int variant, int64_t capacity, int64_t start, int64_t count, float* out,
                  void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  int qmode = 0, mode = 0;
  float qf = 0.0f;
  if (rows <= 0 || capacity <= 0 || count <= 0 || count > capacity || start < 0 || start >= capacity)
    return fail(MXK_EINVAL, "kv_gather: need rows > 0 and 0 <= start < capacity, 0 < count <= capacity");
  if (!(head_dim == 64 || head_dim == 128 || head_dim == 256))
    return fail(MXK_EUNSUPPORTED, "kv_gather: head_dim must be 64, 128 or 256");
  if (!kv_mode(kind, bits, variant, qmode, mode, qf))
    return fail(MXK_EUNSUPPORTED, "kv_gather: int widths 1, 2, 4, 8 and float 4, 8 (base or 'v') only");
  if (!codes || !scales || !out) return fail(MXK_EINVAL, "kv_gather: null pointer");
  if ((reinterpret_cast<uintptr_t>(codes) & 3u) != 0 || !aligned16(out))
    return fail(MXK_EINVAL, "kv_gather: codes must be 4-byte and out 16-byte aligned");
  if (rows * head_dim * bits >= ((int64_t)1 << 35) || capacity >= ((int64_t)1 << 31))
    return fail(MXK_EINVAL, "kv_gather: ring too large");
  const uint8_t* c = reinterpret_cast<const uint8_t*>(codes);
  const dim3 grid((unsigned)std::min<int64_t>(ceil_div(rows, KV_RT), 65535),
                  (unsigned)std::min<int64_t>(ceil_div(count, KV_JT), 65535));
#define MXK_KVG(MODE, BITS)                                                                                       \
  do {                                                                                                            \
    if (head_dim == 64)                                                                                           \
      hipLaunchKernelGGL((k_kv_gather<MODE, BITS, 4>), grid, dim3(256), 0, st, c, scales, zero_point, rows,     \
                         capacity, start, count, out);                                                            \
    else if (head_dim == 128)                                                                                     \
      hipLaunchKernelGGL((k_kv_gather<MODE, BITS, 5>), grid, dim3(256), 0, st, c, scales, zero_point, rows,     \
                         capacity, start, count, out);                                                            \
    else                                                                                                          \
      hipLaunchKernelGGL((k_kv_gather<MODE, BITS, 6>), grid, dim3(256), 0, st, c, scales, zero_point, rows,     \
                         capacity, start, count, out);                                                            \
  } while (0)
  if (mode == Q_FP) {
    if (bits == 4) MXK_KVG(Q_FP, 4);
    else MXK_KVG(Q_FP, 8);
  } else if (mode == Q_INT1) {
    MXK_KVG(Q_INT1, 1);
  } else {
    if (bits == 2) MXK_KVG(Q_INT, 2);
    else if (bits == 4) MXK_KVG(Q_INT, 4);
    else MXK_KVG(Q_INT, 8);
  }
#undef MXK_KVG
  return check_launch("kv_gather");
}

}  // extern "C"
