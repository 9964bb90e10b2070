/*
 * mxk.h — C ABI of libmxk.so, the MI355X (gfx950) kernels behind the
 * mxtorch quantize / dequantize / packed-GEMM hot path.
 *
 * The reference (mxtorch.py, a single Python module) has no FFI: its swap
 * points are Python functions.  Each entry point below names the reference
 * function it replaces (mxtorch.py:LINE).  The Python package qtpytorch_amd
 * binds these symbols with ctypes and keeps the reference's Python API
 * (mx_tensor.quantize / dequantize / @, mx_linear, to_mx, _QGemmSTE,
 * mx_matmul, kv_cache_quantizer) and its byte and scale layouts.
 *
 * Conventions
 *  - All pointers except `signs`' host copy are device pointers; the caller
 *    owns and allocates every buffer (outputs, optional workspaces).  The
 *    library never allocates device memory.
 *  - Every call is asynchronous on `stream` (a hipStream_t; NULL is the
 *    default stream).  Entry points are reentrant; calls that share a
 *    workspace must not overlap.
 *  - Return 0 on success or a negative mxk_status; mxk_last_error() gives a
 *    thread-local message.  No exceptions cross the ABI.
 *  - Layouts (mxtorch.py:870-985, 6044-6049): values are blocked over the
 *    row-major flattened tensor, zero-padded to nb = ceil(n/block) blocks.
 *    For bits in {1,2,4,8} codes are packed LSB-first into bytes (element j
 *    at byte j/(8/bits), bit (j%(8/bits))*bits); for bits in {3,5,6,7,16}
 *    into little-endian int32 words holding floor(32/bits) fields.  Int
 *    fields are two's complement; float fields are indices into the sorted
 *    grid.  Scales are float32 [nb].
 */
#ifndef MXK_H
#define MXK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MXK_ABI_VERSION 10

typedef enum {
  MXK_OK = 0,
  MXK_EINVAL = -22,       /* bad argument (shape, size, pointer, alignment) */
  MXK_EUNSUPPORTED = -95, /* combination this build does not implement     */
  MXK_ELAUNCH = -5        /* a HIP launch or runtime call failed            */
} mxk_status;

typedef enum { MXK_IN_F32 = 0, MXK_IN_F16 = 1, MXK_IN_BF16 = 2 } mxk_elem_type;
typedef enum { MXK_KIND_INT = 0, MXK_KIND_FLOAT = 1 } mxk_kind;
typedef enum {
  MXK_VAR_BASE = 0,     /* ""  : block absmax                              */
  MXK_VAR_HADAMARD = 1, /* "h" : randomized Walsh-Hadamard, then base      */
  MXK_VAR_VECTOR = 2    /* "v" : per-row absmax, true division             */
} mxk_variant;
typedef enum {
  MXK_DYN_PER_TOKEN = 0,   /* one scale per row of the last dimension        */
  MXK_DYN_PER_CHANNEL = 1, /* one scale per column of x.reshape(shape[0], -1) */
  MXK_DYN_PER_TENSOR = 2   /* one scale for the whole tensor                 */
} mxk_dyn_granularity;

/* Library version; equals MXK_ABI_VERSION. */
int mxk_abi_version(void);

/* Thread-local message describing the last failed call on this thread. */
const char* mxk_last_error(void);

/* Bytes of packed storage for n_codes codes of `bits` width: the length of
 * bit_packer.pack_auto's output (mxtorch.py:882-955) in bytes. */
int64_t mxk_packed_nbytes(int bits, int64_t n_codes);

/* Host-side copy of the sorted mini-float grid and its bucket midpoints for
 * float4d (bits=4) and float8d (bits=8): _get_minifloat_grid
 * (mxtorch.py:993-1054) and the mids of _quant_float (mxtorch.py:1523).
 * grid has 2^bits entries, mids 2^bits - 1.  Pure host code (no GPU). */
int mxk_float_grid(int bits, float* grid, float* mids);

/* Workspace bytes mxk_quantize needs for this problem (0 if none). */
size_t mxk_quantize_workspace(int64_t n, int kind, int bits, int variant, int block,
                              int64_t rot_dim);

/* quantize(x, dt, block) -> (packed, scales, n)  (mxtorch.py:1684-1763),
 * CPU semantics of _quant_int (mxtorch.py:1426-1463), _quant_float
 * (mxtorch.py:1465-1528), the 'v' branch (mxtorch.py:1739-1752) and the 'h'
 * branch (mxtorch.py:1720-1736, rotation mxtorch.py:2834-2889).
 *
 *  x         device input, n elements of x_type (row-major flattened).
 *  kind/bits int: bits in {1..8,16}; float: bits in {4,8}.
 *  variant   mxk_variant.  For MXK_VAR_HADAMARD, rot_dim is the rotated
 *            length d (the last dimension, or n for 1-D inputs), n must be a
 *            multiple of d, and `signs` holds next_pow2(d) device floats
 *            (+1/-1), the rotation's sign vector.  Otherwise signs=NULL,
 *            rot_dim=0.
 *  packed    output, packed_nbytes = mxk_packed_nbytes(bits, n_store).
 *  scales    output, ceil(n/block) floats.
 *  n_store   codes to store: ceil(n/block)*block for quantize (the
 *            reference packs the padded blocks), n for GEMM requantization
 *            (mxtorch.py:1384).
 */
int mxk_quantize(const void* x, int x_type, int64_t n, int kind, int bits, int variant,
                 int block, const float* signs, int64_t rot_dim, void* packed,
                 int64_t packed_nbytes, float* scales, int64_t n_store, void* workspace,
                 size_t workspace_nbytes, void* stream);

/* _dequant(packed, scales, dt, n, block) (mxtorch.py:1530-1597) -> out[n]
 * float32.  Reads only the first packed_nbytes bytes (GEMM outputs store n
 * codes, quantize stores the padded blocks).  For MXK_VAR_HADAMARD the
 * unrotation runs over rows of rot_dim elements (rot_dim = n reproduces the
 * reference's whole-tensor inverse, mxtorch.py:1582-1595); signs as for
 * mxk_quantize; a workspace of mxk_dequantize_workspace() bytes is needed
 * when next_pow2(rot_dim) > 8192. */
int mxk_dequantize(const void* packed, int64_t packed_nbytes, const float* scales, int64_t nb,
                   int64_t n, int kind, int bits, int variant, int block, const float* signs,
                   int64_t rot_dim, float* out, void* workspace, size_t workspace_nbytes,
                   void* stream);

/* Workspace bytes mxk_dequantize needs (0 if none). */
size_t mxk_dequantize_workspace(int64_t n, int variant, int64_t rot_dim);

/* Workspace bytes mxk_qgemm needs for packed operands that start on 16
 * bytes; out_bits = 0 when no packed output is requested.  With block 128,
 * K % 128 == 0 and N a multiple of 128, int8 x int8 -> 16-bit and int4 x int4
 * -> 8-bit packed outputs are requantized in the GEMM's epilogue and need no
 * M*N float32 buffer. */
size_t mxk_qgemm_workspace(int64_t M, int64_t K, int64_t N, int bits, int block, int out_bits);

/* Workspace bytes mxk_qgemm needs for packed operands at any alignment
 * (those not on 16 bytes are unpacked into the workspace first). */
size_t mxk_qgemm_workspace_any(int64_t M, int64_t K, int64_t N, int bits, int block, int out_bits);

/* Packed block-scaled GEMM: the CPU branch of _dispatch_qgemm
 * (mxtorch.py:5563-5573) around _qscale_matmul (mxtorch.py:1299-1385).
 *
 *  A [M,K] and B [K,N] are bits-packed codes (bits in {1,2,4,8}; both
 *  unpacked with this width and sign-extended, as the reference unpacks b
 *  with a's width, mxtorch.py:5564-5565).  KB = ceil(K/block).
 *  SA[m,kb] = a_scales[m*KB+kb] if a_nscales == M*KB, else 1.
 *  SB[kb,n] = b_scales[kb*N+n]  if b_nscales == KB*N, else 1 (the
 *  reference's reading of B's flat scales, mxtorch.py:1354).
 *  For kb ascending: P = exact int32 sum over the block,
 *  C = RN(C + RN(RN(P*SA)*SB)).
 *
 *  Optional outputs (NULL to skip, at least one required):
 *   c_f32    float32 [M,N], C before requantization;
 *   acc_i32  int32 [KB,M,N], the per-block integer products P;
 *   c_packed/c_scales  out_bits > 0: C requantized per `block` flat
 *            elements, s = RN(max(absmax,1e-12)/q), code = rne(clamp(RN(C/s)))
 *            (mxtorch.py:1372-1385), M*N codes packed (mxtorch.py:5570),
 *            scales [ceil(M*N/block)].
 */
int mxk_qgemm(const void* a_packed, const float* a_scales, int64_t a_nscales, const void* b_packed,
              const float* b_scales, int64_t b_nscales, int64_t M, int64_t K, int64_t N, int bits,
              int block, int out_bits, void* c_packed, int64_t c_packed_nbytes, float* c_scales,
              float* c_f32, int32_t* acc_i32, void* workspace, size_t workspace_nbytes,
              void* stream);

/* Workspace bytes mxk_linear_wq needs (0 if none).  The decode path
 * (1-, 2-, 4- and 8-bit codes, block 128, M <= 16, K % 32 == 0, N % 128 == 0) splits K
 * across workgroups; its workspace (a 64 KiB counter prefix, the partial
 * sums, then room for block-major scales when w_scales_t is NULL) must be
 * zero-filled before first use, and every call, of any shape, leaves the
 * counter prefix ready for the next one.  Calls sharing a workspace must
 * not overlap.  The size also covers mxk_linear_wq_tiled and the MFMA path
 * (1-, 2-, 4- and 8-bit codes, block 128, N % 128 == 0, any M): its row exponents,
 * x scaled by them (M * roundup(K, 256) floats), a block-major copy of the
 * scales when w_scales_t is NULL and any K-split partials, all after the
 * counter prefix, which it leaves alone. */
size_t mxk_linear_workspace(int64_t M, int64_t K, int64_t N, int bits, int block);

/* Block-major copy of a weight's scales for the decode path: w_scales_t[b][k]
 * = w_scales[k * (N/128) + b], i.e. [N/128][K] from the [K][N/128] layout
 * that quantize(weight.t()) stores (mxtorch.py:7447, 1684-1763).  block must
 * be 128 and N a multiple of 128.  No reference counterpart: the reference
 * dequantizes the whole weight instead (mxtorch.py:7454-7473).  Weights are
 * static, so callers make this copy once per weight. */
int mxk_linear_prepack_scales(const float* w_scales, int64_t K, int64_t N, int block, float* w_scales_t,
                              void* stream);

/* Weight-only linear, mx_linear.forward (mxtorch.py:7454-7473):
 * out[M,N] = x[M,K] (x_type, converted to float32) @ dequant(W) (+ bias[N]),
 * W = the packed codes/scales of quantize(weight.t()): [K,N] row-major,
 * blocks of `block` flat elements (mxtorch.py:7447).  The dequantized
 * weight RN(code*s) (mxtorch.py:1573-1575) is formed in registers only.
 * kind/bits as for mxk_quantize (base variant).  Float32 accumulation.
 * Int1, int2, int4, int8, FP4 and FP8 weights with x of at most 16 rows run the decode kernel;
 * the same weights (block 128, N % 128 == 0) with any other x run on f16 MFMAs, x * s as an f16 hi + lo pair against the exact
 * codes or grid values (each term within 2^-22 of x * RN(code * s), after a
 * power-of-two scaling of every row of x and every block of scales into
 * f16's range); other widths and shapes a scalar fallback.
 * w_scales_t: optional mxk_linear_prepack_scales() copy of w_scales, read
 * by the decode path and the MFMA path (NULL: they transpose into the
 * workspace). */
int mxk_linear_wq(const void* x, int x_type, int64_t M, int64_t K, const void* w_packed,
                  const float* w_scales, const float* w_scales_t, int64_t N, int kind, int bits,
                  int block, const float* bias, float* out, void* workspace,
                  size_t workspace_nbytes, void* stream);

/* mxk_linear_wq without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Same arguments and result as mxk_linear_wq; the decode path's split-K
 * workspace is a static 8 MiB device array of the library (one per GPU,
 * held until the process ends), so shapes that need more (for example
 * N = 16384, K = 8192) return MXK_EINVAL: pass w_scales_t or use
 * mxk_linear_wq.  Other shapes take the MFMA path when its buffers fit the
 * array and the scalar fallback otherwise.  The call allocates nothing; the first call on a device
 * clears the array's counters with a fill kernel on `stream`.  All calls on
 * one GPU share the array: calls that overlap on one GPU (other streams,
 * concurrent graph replays) race and must not be issued. */
int mxk_linear_wq_noalloc(const void* x, int x_type, int64_t M, int64_t K, const void* w_packed,
                          const float* w_scales, const float* w_scales_t, int64_t N, int kind, int bits, int block,
                          const float* bias, float* out, void* stream);

/* Tiled copy of a 4-bit weight (int4 or FP4 codes: the copy only moves
 * nibbles) for mxk_linear_wq_tiled: w_packed is the
 * [K][N] packing of quantize(weight.t()) (mxtorch.py:7447), bits 4, block
 * 128, K a multiple of 32, N of 128; w_tiled receives the same K*N/2 bytes
 * reordered so that the decode kernel reads each wave's rows as contiguous
 * 16-byte loads and builds its MFMA operands without byte permutes (2 KiB per
 * 128-column block and 32-row step).  No reference counterpart: the
 * reference dequantizes the whole weight instead (mxtorch.py:7454-7473).
 * Weights are static, so callers make this copy once per weight.
 * w_packed 4-byte aligned, w_tiled 16-byte aligned. */
int mxk_linear_prepack_weight(const void* w_packed, int64_t K, int64_t N, int bits, int block, void* w_tiled,
                              void* stream);

/* The inverse of mxk_linear_prepack_weight: w_packed receives the K*N/2
 * bytes of the [K][N] packing back from the tiled copy, so that a caller may
 * keep the tiled copy only and rebuild the packed codes when something else
 * needs them (dequantize, checkpoints).  No reference counterpart.  Same
 * arguments and alignment as mxk_linear_prepack_weight. */
int mxk_linear_unpack_weight(const void* w_tiled, int64_t K, int64_t N, int bits, int block, void* w_packed,
                             void* stream);

/* mx_linear.forward (mxtorch.py:7454-7473) for 4-bit weights (kind
 * MXK_KIND_INT: int4 codes, MXK_KIND_FLOAT: FP4 E2M1 codes), block 128, from
 * the prepacked copies: out[M,N] = x[M,K] @ dequant(W) (+ bias), the product
 * of mxk_linear_wq, float32 accumulation in another order.  w_tiled =
 * mxk_linear_prepack_weight(), w_scales_t = mxk_linear_prepack_scales().
 * K % 32 == 0, N % 128 == 0, 16-byte aligned w_tiled, w_scales_t, bias and
 * out.  M <= 16 with 16-byte aligned x runs the decode kernel, any other M
 * the MFMA path on the same tiled copy; other shapes return
 * MXK_EUNSUPPORTED (call mxk_linear_wq).  workspace: as for mxk_linear_wq
 * (mxk_linear_workspace() bytes, zero-filled before first use, left ready
 * for the next call; calls sharing it must not overlap). */
int mxk_linear_wq_tiled(const void* x, int x_type, int64_t M, int64_t K, const void* w_tiled,
                        const float* w_scales_t, int64_t N, int kind, const float* bias, float* out,
                        void* workspace, size_t workspace_nbytes, void* stream);

/* One step of kv_cache_quantizer.append_kv (mxtorch.py:3039-3067) written
 * into a caller-owned ring slot (the reference appends a new mx_tensor to a
 * Python list instead, mxtorch.py:3058-3065).
 *  k, v      device [rows, head_dim] of x_type (rows = B*H of the step), 16-byte aligned.
 *  K rows:   quantize(k_f, dt, head_dim): one block per row.
 *  V rows:   with asymmetric_v, zp = row min, quantize(v_f - zp, dt, head_dim)
 *            and v_zero_point[r] = zp (mxtorch.py:3060-3065); else as K.
 *  Outputs:  k_codes / v_codes   packed codes of the slot, rows*head_dim*bits/8 bytes;
 *            k_scales / v_scales float32 [rows]; v_zero_point float32 [rows]
 *            (unused when asymmetric_v = 0).
 *  Covers head_dim in {64, 128, 256}; int widths 1, 2, 4, 8 and float 4, 8,
 *  base or 'v' variant (MXK_EUNSUPPORTED otherwise: use mxk_quantize). */
int mxk_kv_append(const void* k, const void* v, int x_type, int64_t rows, int head_dim, int kind, int bits,
                  int variant, int asymmetric_v, void* k_codes, float* k_scales, void* v_codes, float* v_scales,
                  float* v_zero_point, void* stream);

/* kv_cache_quantizer.get for one tensor (mxtorch.py:3069-3086): out float32
 * [rows, count, head_dim] = the dequantized slots start, start+1, ... (mod
 * capacity) of a ring whose slot s holds codes at codes + s*rows*head_dim*bits/8,
 * scales at scales + s*rows and (V, asymmetric) zero points at
 * zero_point + s*rows, added after the dequantization (RN(dq + zp));
 * zero_point = NULL adds nothing.  Same dtype coverage as mxk_kv_append. */
int mxk_kv_gather(const void* codes, const float* scales, const float* zero_point, int64_t rows, int head_dim,
                  int kind, int bits, int variant, int64_t capacity, int64_t start, int64_t count, float* out,
                  void* stream);

/* Workspace bytes mxk_qelementwise needs (0 when the output is packed in
 * the same pass: block <= 256, out_bits in {1, 2, 4, 8, 16}, block*out_bits
 * a multiple of 32). */
size_t mxk_qelementwise_workspace(int op, int64_t n, int64_t nb, int block, int bits, int out_bits);

/* Quantized element-wise arithmetic on packed operands (no float element
 * values are formed beyond the reference's own):
 *  op 0 add, 1 sub: the CPU branches of _dispatch_qadd / _dispatch_qsub
 *       (mxtorch.py:5397-5401, 5425-5431) around _qscale_add
 *       (mxtorch.py:1186-1256);
 *  op 2 mul: _dispatch_qmul's CPU branch (mxtorch.py:5489-5497) around
 *       _qscale_mul (mxtorch.py:1259-1296);
 *  op 3 neg: mx_tensor.__neg__ (mxtorch.py:6177-6193), b and the scales
 *       unused (the caller copies a's scales).
 *  Both operands' first n codes are unpacked with `bits` (a's width,
 *  bits in {2..8, 16}; neg also 1) and sign-extended; codes past n are 0.
 *  Outputs: c_packed = the nb*block result codes packed with out_bits
 *  (mxk_packed_nbytes(out_bits, nb*block) bytes; neg: the n codes, or all
 *  a_nbytes codes for 8-bit operands, with the same width), c_scales [nb].
 *  block <= 256.  Packed buffers 4-byte aligned. */
int mxk_qelementwise(int op, const void* a_packed, int64_t a_nbytes, const float* a_scales, const void* b_packed,
                     int64_t b_nbytes, const float* b_scales, int64_t n, int64_t nb, int block, int bits,
                     int out_bits, void* c_packed, int64_t c_nbytes, float* c_scales, void* workspace,
                     size_t workspace_nbytes, void* stream);

/* Weight-only linear with the weight stored [N][K] (row n = output n):
 * out[M,N] = x[M,K] (x_type, as float32) @ dequant(W)^T (+ bias[N]), the
 * computation of mx_dynamic_linear.forward (mxtorch.py:8949-8962: the
 * dequantized quantize(weight) applied as tokens @ w_dq.t() + bias) and of
 * _MXLinearAutograd.backward (mxtorch.py:6729-6740: grad @ w_dq.t()).
 * W: packed codes of any width/kind of mxk_quantize (base variant), flat
 * blocks of `block` elements of the row-major [N][K] weight, w_nscales >=
 * ceil(N*K/block).  Float32 accumulation.  With int4 codes, block 128 and
 * M <= 16 the K sum is split over workgroups (workspace below), and that
 * path reads w_scales_t when given: the K-block-major copy [K/128][N] of the
 * scales (mxk_linear_prepack_scales(w_scales, N, K, 128, w_scales_t) of the
 * [N][K/128] layout), made once per weight.  NULL reads w_scales. */
int mxk_linear_wq_nt(const void* x, int x_type, int64_t M, int64_t K, const void* w_packed, int64_t w_nbytes,
                     const float* w_scales, int64_t w_nscales, const float* w_scales_t, int64_t N, int kind,
                     int bits, int block, const float* bias, float* out, void* workspace, size_t workspace_nbytes,
                     void* stream);

/* Workspace bytes mxk_linear_wq_nt needs (0 if none): the decode path (int4
 * base codes, block 128, M <= 16, K % 128 == 0, N % 16 == 0) splits K over
 * workgroups of 1024 rows of K; its workspace (a 64 KiB prefix of arrival
 * counters, then the partial sums) must be zero-filled before first use,
 * and every call leaves the counters zero again.  Calls sharing a workspace
 * must not overlap.  The size also covers the MFMA path (int4 / int8 codes,
 * block 128, K and N multiples of 128, any M): row exponents, x as f16 hi +
 * lo (M * roundup(K, 256) * 4 bytes) and any K-split partials after the
 * counter prefix. */
size_t mxk_linear_nt_workspace(int64_t M, int64_t K, int64_t N, int bits, int block);

/* Tiled copy of an int4 [N][K] weight for mxk_linear_wq_nt_tiled: w_packed
 * is the packing of quantize(weight) of mx_dynamic_linear
 * (mxtorch.py:8870-8968, flat blocks of 128 along K), bits 4, block 128, K
 * and N multiples of 128; w_tiled receives the same N*K/2 bytes reordered so
 * that each 16-row tile of a K block is 1 KiB contiguous and every MFMA
 * operand comes out of its words with masks (no byte permutes).  No
 * reference counterpart: the reference dequantizes the weight instead
 * (mxtorch.py:8949-8962).  Weights are static, so callers make this copy
 * once per weight.  w_packed and w_tiled 16-byte aligned. */
int mxk_linear_prepack_weight_nt(const void* w_packed, int64_t N, int64_t K, int bits, int block, void* w_tiled,
                                 void* stream);

/* The inverse of mxk_linear_prepack_weight_nt: w_packed receives the N*K/2
 * bytes of the [N][K] packing back from the tiled copy (a caller may keep
 * the tiled copy only).  No reference counterpart.  Same arguments and
 * alignment as mxk_linear_prepack_weight_nt. */
int mxk_linear_unpack_weight_nt(const void* w_tiled, int64_t N, int64_t K, int bits, int block, void* w_packed,
                                void* stream);

/* mx_dynamic_linear.forward (mxtorch.py:8949-8962) for int4 weights, block
 * 128, from the prepacked copies: out[M,N] = x[M,K] @ dequant(W)^T (+ bias),
 * the product of mxk_linear_wq_nt's decode path, float32 accumulation in
 * another order.  w_tiled = mxk_linear_prepack_weight_nt(), w_scales_t =
 * the K-block-major scales [K/128][N] (mxk_linear_prepack_scales(w_scales,
 * N, K, 128, w_scales_t)).  K and N multiples of 128, 16-byte aligned
 * w_tiled, w_scales_t, bias and out.  M <= 16 with 16-byte aligned x runs
 * the tiled decode kernel; any other M runs the MFMA kernel on the same
 * tiled copy (the product of mxk_linear_wq_nt's MFMA path), so a weight may
 * be held as its tiled copy only.  Shapes neither takes return
 * MXK_EUNSUPPORTED (call mxk_linear_wq_nt on the packed codes).  workspace:
 * as for mxk_linear_wq_nt (mxk_linear_nt_workspace() bytes, zero-filled
 * before first use, left ready for the next call; calls sharing it must not
 * overlap). */
int mxk_linear_wq_nt_tiled(const void* x, int x_type, int64_t M, int64_t K, const void* w_tiled,
                           const float* w_scales_t, int64_t N, const float* bias, float* out, void* workspace,
                           size_t workspace_nbytes, void* stream);

/* Workspace bytes mxk_linear_i8 needs (0 when the shapes are not covered). */
size_t mxk_linear_i8_workspace(int64_t M, int64_t K, int64_t N, int x_bits, int w_bits, int64_t x_block,
                               int64_t w_block);

/* fused_int8_linear (mxtorch.py:3910-3960) on int codes: the reference's
 * result is F.linear(x.dequantize(), weight.dequantize(), bias)
 * (mxtorch.py:3957-3960), i.e.
 *   out[m,n] = sum_k RN(xc[m,k]*sx) * RN(wc[n,k]*sw) + bias[n]
 * with x [M][K] and W [N][K] packed int codes (widths 2, 4 or 8, base
 * variant), sx = x_scales[(m*K+k)/x_block], sw = w_scales[(n*K+k)/w_block]
 * (per-token activations from dynamic_quantize have x_block = K).  Here the
 * exact integer product of each K chunk runs on int8 MFMA and the chunk is
 * scaled once: out = sum_chunks RN(RN(P*sx)*sw) (+ bias), float32,
 * within 1e-3 relative of the reference.  Needs 64 to divide K, x_block
 * and w_block (MXK_EUNSUPPORTED otherwise: dequantize x and use
 * mxk_linear_wq_nt).  8-bit operands are read in place (16-byte aligned). */
int mxk_linear_i8(const void* x_packed, int64_t x_nbytes, const float* x_scales, int64_t x_nscales, int64_t x_block,
                  int x_bits, const void* w_packed, int64_t w_nbytes, const float* w_scales, int64_t w_nscales,
                  int64_t w_block, int w_bits, int64_t M, int64_t K, int64_t N, const float* bias, float* out,
                  void* workspace, size_t workspace_nbytes, void* stream);

/* Workspace bytes mxk_dynamic_quantize needs. */
size_t mxk_dynamic_quantize_workspace(int64_t rows, int64_t cols, int granularity, int bits);

/* dynamic_quantize(x, dt, granularity) (mxtorch.py:2665-2731) on x viewed
 * as [rows][cols]: rows x cols = x.reshape(-1, shape[-1]) for per_token,
 * x.reshape(shape[0], -1) for per_channel, any split for per_tensor.
 *   s = RN(max(absmax, 1e-12) / max_int), max_int = 2^(bits-1)-1,
 *   code = rne(clamp(RN(x / s), -max_int, max_int)),
 * over a row (per_token: scales[rows]), a column (per_channel:
 * scales[cols]) or the tensor (per_tensor: scales[1]); codes packed with
 * pack_auto (mxtorch.py:976-985), packed_nbytes = mxk_packed_nbytes(bits,
 * rows*cols).  Widths 2..8 and 16 per token, 2, 4 and 8 otherwise. */
int mxk_dynamic_quantize(const void* x, int x_type, int64_t rows, int64_t cols, int granularity, int bits,
                         void* packed, int64_t packed_nbytes, float* scales, void* workspace,
                         size_t workspace_nbytes, void* stream);

/* vector_quantize(x, dtype, axis) (mxtorch.py:2946-2987) on x [rows][cols]:
 * one scale per row (axis = 1) or per column (axis = 0),
 *   s = RN(max(absmax, 1e-12) / max_int),  max_int = 2^(bits-1)-1,
 *   codes = rne(clamp(RN(x / s), -max_int, max_int))  as int32 [rows][cols]
 * (the reference rounds before clamping; with an integer max_int the two
 * orders agree), scales float32 [rows] or [cols].  Widths 2..16.  No
 * workspace: the absmax accumulates in `scales`. */
int mxk_vector_quantize(const void* x, int x_type, int64_t rows, int64_t cols, int axis, int bits, int32_t* codes,
                        float* scales, void* stream);

/* vector_dequantize(codes, scales, axis) (mxtorch.py:2989-2994):
 * out[r][c] = RN(codes[r][c] * s), s = scales[r] (axis = 1) or scales[c]. */
int mxk_vector_dequantize(const int32_t* codes, const float* scales, int64_t rows, int64_t cols, int axis, float* out,
                          void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MXK_H */
