/*
 * ntops_amd.h -- C ABI of the MI355X (gfx950) operator library behind
 * ntops_amd.torch.<op>.
 *
 * Every entry point takes raw device pointers, element counts and element
 * strides (int64, in elements, never bytes), scalar arguments as plain C
 * values, and the HIP stream to launch on (a hipStream_t passed as void*;
 * NULL is the null stream).  Nothing here allocates device memory, nothing
 * synchronises, and no C++ exception crosses the boundary: each call returns
 * NTOPS_OK or an error code, and ntops_last_error() returns the message of the
 * calling thread's most recent failure.  Launches are asynchronous and stream
 * ordered, exactly like the Triton launches they replace.
 *
 * Reference interface replaced by each entry point (paths relative to the
 * mygitljf/ntops source tree):
 *   ntops_unary       <- src/ntops/torch/{silu,gelu,exp,bitwise_not}.py:7-17,
 *                        {relu,sigmoid,tanh,neg,abs,rsqrt,sin,cos}.py:7-17
 *                        (kernels/<op>.py application)
 *   ntops_binary      <- src/ntops/torch/{add,mul,bitwise_and,bitwise_or}.py:7-15,
 *                        {sub,div,pow}.py:7-15
 *   ntops_binary_cvt  <- no ntops counterpart (ntops requires equal dtypes):
 *                        torch's promotion of mixed operand dtypes to fp32
 *                        (cast, then the op) fused into the elementwise pass
 *   ntops_compare     <- src/ntops/torch/{eq,ne,gt,ge,lt,le}.py:7-15
 *   ntops_classify    <- src/ntops/torch/{isinf,isnan}.py:7-14
 *   ntops_clamp       <- src/ntops/torch/clamp.py:7-15
 *   ntops_cast        <- no ntops counterpart; the dtype promotion / layout
 *                        copy that torch's TensorIterator performs before the
 *                        elementwise kernels (kept native so no op falls back
 *                        to torch for data movement)
 *   ntops_rms_norm    <- src/ntops/torch/rms_norm.py:9-31, kernels/rms_norm.py:10-20
 *   ntops_layer_norm  <- src/ntops/torch/layer_norm.py:9-33, kernels/layer_norm.py:11-31
 *   ntops_softmax     <- src/ntops/torch/softmax.py:7-16, kernels/softmax.py:9-29
 *   ntops_rope        <- src/ntops/torch/rotary_position_embedding.py:7-29,
 *                        kernels/rotary_position_embedding.py:6-47
 *   ntops_sdpa        <- src/ntops/torch/scaled_dot_product_attention.py:10-108,
 *                        kernels/scaled_dot_product_attention.py:154-201
 *   ntops_gemm        <- src/ntops/torch/{mm,bmm,addmm}.py:7-18,
 *                        kernels/mm.py:54-65, kernels/bmm.py:8-43,
 *                        kernels/addmm.py:64-67
 *   ntops_gemm_ws     <- the same interface as ntops_gemm, plus a caller-owned
 *                        workspace that lets products whose tiles do not fill
 *                        the chip split K (no ntops counterpart: Triton's
 *                        autotuner picks smaller tiles instead)
 *   ntops_gemm_workspace <- no ntops counterpart; sizes that workspace
 *   ntops_conv2d      <- src/ntops/torch/conv2d.py:8-53, kernels/conv2d.py:12-104
 *   ntops_add_rms_norm <- no ntops counterpart: the composition
 *                        rms_norm(x + residual) (torch/add.py:7-15 then
 *                        torch/rms_norm.py:9-31) fused into one pass that also
 *                        returns the new residual
 *   ntops_rope_qk     <- no ntops counterpart: two calls of
 *                        torch/rotary_position_embedding.py:7-29 (q and k with
 *                        the same tables) in one launch
 *   ntops_im2col      <- src/ntops/torch/im2col.py:44-135, kernels/im2col.py:10-80
 *   ntops_conv2d_workspace <- no ntops counterpart (Triton tiles the unfolded
 *                        input on the fly); sizes the caller-owned buffer that
 *                        the GEMM path of ntops_conv2d unfolds into
 */
#ifndef NTOPS_AMD_H
#define NTOPS_AMD_H

#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define NTOPS_API __attribute__((visibility("default")))
#else
#define NTOPS_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* ---- element types ---------------------------------------------------- */
enum ntops_dtype {
  NTOPS_F32 = 0,
  NTOPS_F16 = 1,
  NTOPS_BF16 = 2,
  NTOPS_F64 = 3,
  NTOPS_BOOL = 4,
  NTOPS_U8 = 5,
  NTOPS_I8 = 6,
  NTOPS_I16 = 7,
  NTOPS_I32 = 8,
  NTOPS_I64 = 9
};

/* ---- status codes ----------------------------------------------------- */
enum ntops_status {
  NTOPS_OK = 0,
  NTOPS_ERR_INVALID = 1,     /* bad shape / stride / pointer / argument   */
  NTOPS_ERR_UNSUPPORTED = 2, /* valid request this library does not serve */
  NTOPS_ERR_HIP = 3          /* the HIP runtime reported an error         */
};

/* Maximum tensor rank accepted by the strided entry points (after adjacent
 * dimensions that are contiguous in every operand have been merged). */
#define NTOPS_MAX_DIMS 8

/* ---- library ----------------------------------------------------------- */
NTOPS_API int ntops_abi_version(void);
/* Message of this thread's most recent failed call ("" if none). */
NTOPS_API const char* ntops_last_error(void);
/* Name of the kernel that this thread's most recent GEMM-family, attention
 * or im2col call launched (e.g. "gemm_mfma 256x256 s4 A:K B:N even"), ""
 * before the first.
 * No ntops counterpart (Triton picks its kernel inside ninetoothed.make); it
 * lets callers and tests check which path served a call. */
NTOPS_API const char* ntops_last_kernel(void);

/* ---- elementwise ------------------------------------------------------ */
enum ntops_unary_op {
  NTOPS_UNARY_SILU = 1,      /* x / (1 + exp(-x))                 silu.py:10  */
  NTOPS_UNARY_GELU = 2,      /* x * 0.5 * (1 + erf(x / sqrt 2))   gelu.py:11  */
  NTOPS_UNARY_GELU_TANH = 3, /* 0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3)))
                                                                  gelu.py:14-26 */
  NTOPS_UNARY_EXP = 4,       /* exp(x)                            exp.py:10   */
  NTOPS_UNARY_BITWISE_NOT = 5, /* ~x; logical not for bool  bitwise_not.py:9-14 */
  NTOPS_UNARY_RELU = 6,      /* max(0, x), NaN kept               relu.py:9   */
  NTOPS_UNARY_SIGMOID = 7,   /* 1 / (1 + exp(-x))                 sigmoid.py:10 */
  NTOPS_UNARY_TANH = 8,      /* tanh(x)                           tanh.py:10-13 */
  NTOPS_UNARY_NEG = 9,       /* -x (two's complement wrap)        neg.py:9    */
  NTOPS_UNARY_ABS = 10,      /* |x|                               abs.py:10   */
  NTOPS_UNARY_RSQRT = 11,    /* 1 / sqrt(x), each op IEEE         rsqrt.py:10 */
  NTOPS_UNARY_SIN = 12,      /* sin(x)                            sin.py:10   */
  NTOPS_UNARY_COS = 13       /* cos(x)                            cos.py:10   */
};

/* y = op(x) over an ndim-dimensional index space `shape`.  x and y have the
 * same dtype; SILU/GELU/EXP/SIGMOID/TANH/RSQRT/SIN/COS accept F32/F16/BF16/F64
 * (16-bit types compute in fp32 and round once), RELU/NEG/ABS accept the
 * floating and the signed/unsigned integer types, BITWISE_NOT accepts
 * BOOL/U8/I8/I16/I32/I64.  y may alias x exactly (in-place). */
NTOPS_API int ntops_unary(int op, int dtype, int ndim, const int64_t* shape,
                const void* x, const int64_t* x_strides,
                void* y, const int64_t* y_strides, void* stream);

enum ntops_binary_op {
  NTOPS_BINARY_ADD = 1,         /* a + alpha * b              add.py:10 */
  NTOPS_BINARY_MUL = 2,         /* a * b                      mul.py:9  */
  NTOPS_BINARY_BITWISE_AND = 3, /* a & b               bitwise_and.py:9 */
  NTOPS_BINARY_BITWISE_OR = 4,  /* a | b                bitwise_or.py:9 */
  NTOPS_BINARY_SUB = 5,         /* a - alpha * b              sub.py:10 */
  NTOPS_BINARY_DIV = 6,         /* a / b (floating only)      div.py:10 */
  NTOPS_BINARY_DIV_TRUNC = 7,   /* trunc(a / b)               div.py:14 */
  NTOPS_BINARY_DIV_FLOOR = 8,   /* floor(a / b), Python's floor division
                                                              div.py:18 */
  NTOPS_BINARY_POW = 9          /* a ** b                     pow.py:10 */
};

/* out = op(a, b) over `shape`.  a, b and out share `dtype` (the caller has
 * already applied type promotion).  Broadcasting is expressed by stride 0.
 * When b is NULL, b is the scalar (b_f for floating dtypes, b_i for integer
 * and bool dtypes).  alpha (ADD, SUB) follows the same split; it is rounded
 * to `dtype` before use, as torch's CPU kernel does.  A scalar b of ADD/SUB
 * and of POW is rounded to `dtype`; of MUL/DIV* it stays in fp32 (fp64 for
 * F64) opmath -- torch's CPU conventions.  DIV_TRUNC / DIV_FLOOR on integer
 * dtypes give 0 where b == 0 (torch's CPU kernel raises instead).  POW on
 * integer dtypes uses torch's rule for negative exponents (1 for base 1,
 * +-1 for base -1, else 0). */
NTOPS_API int ntops_binary(int op, int dtype, int ndim, const int64_t* shape,
                 const void* a, const int64_t* a_strides,
                 const void* b, const int64_t* b_strides,
                 double b_f, int64_t b_i, double alpha_f, int64_t alpha_i,
                 void* out, const int64_t* out_strides, void* stream);

/* out (F32) = op(a, b) over n dense elements whose operand dtypes differ
 * from the fp32 result (a_dtype, b_dtype in {F32, F16, BF16, I32}; dtype
 * must be F32): each operand is converted to fp32 on load and the fp32 op
 * of ntops_binary applied, so the result equals casting both first and
 * calling ntops_binary on F32 -- in one pass.  op in {ADD, SUB, MUL, DIV};
 * alpha_f as for ntops_binary.  a, b and out must be 16-byte aligned. */
NTOPS_API int ntops_binary_cvt(int op, int a_dtype, int b_dtype, int dtype, int64_t n,
                 const void* a, const void* b, double alpha_f, void* out, void* stream);

enum ntops_compare_op {
  NTOPS_CMP_EQ = 1, /* a == b   eq.py:9 */
  NTOPS_CMP_NE = 2, /* a != b   ne.py:9 */
  NTOPS_CMP_GT = 3, /* a >  b   gt.py:9 */
  NTOPS_CMP_GE = 4, /* a >= b   ge.py:9 */
  NTOPS_CMP_LT = 5, /* a <  b   lt.py:9 */
  NTOPS_CMP_LE = 6  /* a <= b   le.py:9 */
};

/* out (BOOL) = op(a, b) over `shape`; a and b share `dtype` (any dtype),
 * broadcasting by stride 0.  When b is NULL it is the scalar b_f / b_i,
 * first rounded to `dtype` (the comparison runs in the common dtype, as in
 * torch).  NaN compares unequal to everything. */
NTOPS_API int ntops_compare(int op, int dtype, int ndim, const int64_t* shape,
                  const void* a, const int64_t* a_strides,
                  const void* b, const int64_t* b_strides,
                  double b_f, int64_t b_i,
                  void* out, const int64_t* out_strides, void* stream);

enum ntops_classify_op {
  NTOPS_CLASSIFY_ISINF = 1, /* x == +inf or x == -inf   isinf.py:9-11 */
  NTOPS_CLASSIFY_ISNAN = 2  /* x != x                   isnan.py:9    */
};

/* out (BOOL) = op(x) over `shape`; x of any dtype (integer and bool inputs
 * give false everywhere). */
NTOPS_API int ntops_classify(int op, int dtype, int ndim, const int64_t* shape,
                   const void* x, const int64_t* x_strides,
                   void* out, const int64_t* out_strides, void* stream);

/* out = min(max(x, lo), hi) over `shape` (clamp.py:9).  lo / hi are each
 * absent (has_lo / has_hi = 0), a tensor (lo / hi non-NULL, strides with 0
 * for broadcast) or the scalar lo_f / lo_i (hi_f / hi_i), rounded to
 * `dtype`.  Floating: a NaN in x, then in lo, then in hi, is the result
 * (torch's rule); lo > hi gives hi.  dtype: any but BOOL. */
NTOPS_API int ntops_clamp(int dtype, int ndim, const int64_t* shape,
                const void* x, const int64_t* x_strides,
                const void* lo, const int64_t* lo_strides, double lo_f, int64_t lo_i, int has_lo,
                const void* hi, const int64_t* hi_strides, double hi_f, int64_t hi_i, int has_hi,
                void* out, const int64_t* out_strides, void* stream);

/* y = (dst_dtype) x, elementwise, any strides (stride 0 allowed on x). */
NTOPS_API int ntops_cast(int src_dtype, int dst_dtype, int ndim, const int64_t* shape,
               const void* x, const int64_t* x_strides,
               void* y, const int64_t* y_strides, void* stream);

/* ---- row reductions --------------------------------------------------- */
/* y[r, :] = x[r, :] * rsqrt(mean(x[r, :]^2) + eps) * w[r, :]   (fp32
 * accumulate, one rounding to dtype).  x and y are rows x cols with unit
 * column stride and the given row strides; w (may be NULL = ones) holds rows
 * of cols contiguous elements of w_dtype (dtype or F32) w_row_stride apart --
 * 0 for one weight row shared by every row (the usual case; a non-zero
 * stride, a weight that differs per row, runs a slower looped kernel).
 * Any width and row offset: when x and y rows sit at the same offset within
 * 16 bytes the row is read once (register-resident, split into head /
 * 16-byte packs / tail, or staged in VGPRs + LDS up to 146944 16-bit /
 * 73472 fp32 elements); other layouts and wider rows run looped kernels.
 * dtype in {F32, F16, BF16}. */
NTOPS_API int ntops_rms_norm(int dtype, int64_t rows, int64_t cols,
                   const void* x, int64_t x_row_stride,
                   const void* w, int64_t w_row_stride, int w_dtype, double eps,
                   void* y, int64_t y_row_stride, void* stream);

/* y[r, :] = (x - mean) * rsqrt(var + eps) * w[r, :] + b[r, :], biased
 * variance, fp32 moments.  w and b may each be NULL (ones / zeros); both
 * have rows wb_row_stride apart, 0 when shared by every row (as for
 * ntops_rms_norm). */
NTOPS_API int ntops_layer_norm(int dtype, int64_t rows, int64_t cols,
                     const void* x, int64_t x_row_stride,
                     const void* w, const void* b, int64_t wb_row_stride, int wb_dtype, double eps,
                     void* y, int64_t y_row_stride, void* stream);

/* Softmax over the middle axis of an (outer, dim_size, inner) view.
 * x_strides / y_strides are the three strides of that view.  The input is
 * first converted to out_dtype (as torch does for the dtype= argument), then
 * max/sum are accumulated in fp32 (fp64 when out_dtype is F64).  A row that
 * is entirely -inf produces NaN. */
NTOPS_API int ntops_softmax(int in_dtype, int out_dtype,
                  int64_t outer, int64_t dim_size, int64_t inner,
                  const void* x, const int64_t* x_strides,
                  void* y, const int64_t* y_strides, void* stream);

/* ---- rotary position embedding ---------------------------------------- */
/* x, y: (B, S, H, D) with the given 4 strides; y may alias x.  sin/cos:
 * (S, table_cols) tables with row stride table_row_stride and unit column
 * stride; table_cols is D/2 (one angle per pair, as ntops expects) or D
 * (one value per element, the rotate_half convention).  interleaved != 0
 * rotates pairs (2i, 2i+1); otherwise pairs (i, i + D/2).  Every product and
 * sum is rounded to dtype, matching torch eager evaluation of
 * x*cos + rotate_half(x)*sin.  dtype in {F32, F16, BF16}; D even, <= 1024. */
NTOPS_API int ntops_rope(int dtype, int64_t B, int64_t S, int64_t H, int64_t D,
               const void* x, const int64_t* x_strides,
               const void* sin_table, const void* cos_table,
               int64_t table_row_stride, int64_t table_cols, int interleaved,
               void* y, const int64_t* y_strides, void* stream);

/* ---- GEMM family ------------------------------------------------------ */
/* For each batch index: out = alpha * (A @ B) + beta * C
 *   A: M x K, B: K x N, out: M x N, all with 3 strides (batch, row, col).
 *   C may be NULL (or beta == 0: C is not read); its 3 strides may contain
 *   zeros to broadcast (e.g. a bias row: {0, 0, 1}).
 * dtype in {BF16, F16, F32} for A, B, C and out.  Products accumulate in
 * fp32 and round to dtype once.  bf16/fp16 run on MFMA matrix cores; fp32
 * runs IEEE fp32 (no reduced-precision input path exists on gfx950). */
NTOPS_API int ntops_gemm(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K,
               const void* A, const int64_t* a_strides,
               const void* B, const int64_t* b_strides,
               const void* C, const int64_t* c_strides,
               double alpha, double beta,
               void* out, const int64_t* out_strides, void* stream);

/* ntops_gemm with a caller-owned workspace (16-byte aligned device memory;
 * NULL or too small: the product runs as ntops_gemm).  Products whose
 * 128 x 128 tiles do not fill the GPU and whose K is long enough (bf16 /
 * fp16: batch 1; fp32: any batch) split K over up to 16 slices: fp32 partial
 * products into the workspace, then their sum in slice order, so the result
 * is deterministic (it differs from ntops_gemm's only by the fp32 summation
 * order). */
NTOPS_API int ntops_gemm_ws(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K,
               const void* A, const int64_t* a_strides,
               const void* B, const int64_t* b_strides,
               const void* C, const int64_t* c_strides,
               double alpha, double beta,
               void* out, const int64_t* out_strides,
               void* workspace, int64_t workspace_bytes, void* stream);

/* Bytes of workspace ntops_gemm_ws uses for this problem on the current
 * device (0: it would not split K). */
NTOPS_API int64_t ntops_gemm_workspace(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K);

/* ---- attention ---------------------------------------------------------- */
/* out = softmax(q k^T * scale + mask) v for q (B, Hq, Sq, D), k and v
 * (B, Hkv, Skv, D), out (B, Hq, Sq, D); each tensor is described by its 4
 * element strides.  Query head h attends key / value head h / (Hq / Hkv)
 * (GQA; Hq % Hkv == 0).  mask (may be NULL) is broadcast by its 4 strides
 * (0 = broadcast) over (B, Hq, Sq, Skv): mask_dtype BOOL (true = attend) or
 * F32 / F16 / BF16 (added to the scaled scores).  causal: 0 none, 1
 * upper-left (key j visible to query i when j <= i), 2 lower-right
 * (j <= i + Skv - Sq); mask and causal are exclusive.  dtype in {F32, F16,
 * BF16}; fp32 accumulation, the probabilities rounded to dtype for the
 * product with v (16-bit dtypes).  A row with every key masked yields 0.
 * D <= 256; 16-bit data with D a multiple of 8 up to 128 and unit-stride
 * rows runs on the matrix cores, anything else on a generic fp32 kernel. */
NTOPS_API int ntops_sdpa(int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Skv,
               int64_t D, const void* q, const int64_t* q_strides,
               const void* k, const int64_t* k_strides,
               const void* v, const int64_t* v_strides,
               const void* mask, int mask_dtype, const int64_t* mask_strides,
               int causal, double scale,
               void* out, const int64_t* out_strides, void* stream);

/* ---- fused variants ------------------------------------------------------- */
/* residual_out = x + residual (rounded to dtype) and y = rms_norm(residual_out)
 * over rows x cols with the conventions of ntops_rms_norm (weight of dtype or
 * F32, may be NULL; fp32 accumulation; one rounding).  Element for element
 * equal to ntops_binary(ADD) followed by ntops_rms_norm, in one pass (reads
 * x and residual once, writes residual_out and y once) when the four
 * operands' rows sit at one offset within 16 bytes and fit the one-pass
 * kernels; otherwise it runs exactly those two calls.  y may alias x and
 * residual_out may alias residual; y and residual_out must differ. */
NTOPS_API int ntops_add_rms_norm(int dtype, int64_t rows, int64_t cols,
               const void* x, int64_t x_row_stride,
               const void* residual, int64_t residual_row_stride,
               const void* w, int64_t w_row_stride, int w_dtype, double eps,
               void* y, int64_t y_row_stride,
               void* residual_out, int64_t residual_out_row_stride, void* stream);

/* ntops_rope on q (B, S, Hq, D) and k (B, S, Hk, D) with the same sin / cos
 * tables in one launch (either head count may be 0); results equal two
 * ntops_rope calls.  In-place per tensor is allowed with equal strides. */
NTOPS_API int ntops_rope_qk(int dtype, int64_t B, int64_t S, int64_t Hq, int64_t Hk, int64_t D,
               const void* q, const int64_t* q_strides,
               const void* k, const int64_t* k_strides,
               const void* sin_table, const void* cos_table,
               int64_t table_row_stride, int64_t table_cols, int interleaved,
               void* q_out, const int64_t* q_out_strides,
               void* k_out, const int64_t* k_out_strides, void* stream);

/* ---- convolution -------------------------------------------------------- */
/* out (N, K, P, Q) = conv2d(x (N, C, H, W), w (K, C, R, S)) + bias (K),
 * groups == 1: out[n,k,p,q] = bias[k] + sum_{c,r,s} x[n, c, p*stride_h -
 * pad_h + r*dil_h, q*stride_w - pad_w + s*dil_w] * w[k,c,r,s], zero outside
 * the image (pad_h / pad_w are the top / left padding; P and Q are given, so
 * asymmetric padding is expressed by the output size).  Each tensor is
 * described by its 4 element strides; bias may be NULL (bias_stride is its
 * element stride).  fp32 accumulation, one rounding to dtype (BF16, F16,
 * F32).  workspace (device memory of workspace_bytes, 16-byte aligned, may
 * be NULL) lets large problems run as a matrix-core GEMM over a rearranged
 * copy of the input (padded channels-last images, shifted planes or the
 * unfold), in chunks of images; ntops_conv2d_workspace returns the bytes
 * that cover the whole batch in one chunk (0 when the problem runs without a
 * workspace): a per-call part plus a part per image, so its value for N = 1
 * is what one chunk of one image needs, and for fp32 on the unfold path room
 * for the GEMM's partial products over K slices (used when what a chunk of
 * images leaves of the workspace covers them; optional).  With less than the
 * N = 1 value the direct kernel runs. */
NTOPS_API int64_t ntops_conv2d_workspace(int dtype, int64_t N, int64_t C, int64_t H, int64_t W,
               int64_t K, int64_t R, int64_t S, int64_t P, int64_t Q,
               int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
               int64_t dil_h, int64_t dil_w,
               const int64_t* w_strides, const int64_t* out_strides);
NTOPS_API int ntops_conv2d(int dtype, int64_t N, int64_t C, int64_t H, int64_t W,
               int64_t K, int64_t R, int64_t S, int64_t P, int64_t Q,
               int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
               int64_t dil_h, int64_t dil_w,
               const void* x, const int64_t* x_strides,
               const void* w, const int64_t* w_strides,
               const void* bias, int64_t bias_stride,
               void* out, const int64_t* out_strides,
               void* workspace, int64_t workspace_bytes, void* stream);

/* out (N, C * kernel_h * kernel_w, oh * ow) = the unfolded input x
 * (N, C, H, W): out[n, (c * kernel_h + r) * kernel_w + s, p * ow + q] =
 * x[n, c, p * stride_h - pad_h + r * dil_h, q * stride_w - pad_w + s * dil_w],
 * zero outside the image, with oh = (H + 2 pad_h - dil_h (kernel_h - 1) - 1)
 * / stride_h + 1 (ow alike).  x and out are described by their 4 and 3
 * element strides.  Any dtype (pure data movement, bit-exact).  kernel,
 * dilation and stride >= 1, padding >= 0, and an output size of at least
 * one, else NTOPS_ERR_INVALID. */
NTOPS_API int ntops_im2col(int dtype, int64_t N, int64_t C, int64_t H, int64_t W,
               int64_t kernel_h, int64_t kernel_w, int64_t dil_h, int64_t dil_w,
               int64_t pad_h, int64_t pad_w, int64_t stride_h, int64_t stride_w,
               const void* x, const int64_t* x_strides,
               void* out, const int64_t* out_strides, void* stream);

/* ---- measurement ---------------------------------------------------------- */
/* Matrix-core rate probe (no ntops counterpart; the ceiling bench.py reports
 * for the matrix-bound kernels): `workgroups` workgroups of 4 waves, each
 * wave running `iters` (even) rounds of 8 v_mfma_f32_32x32x16_bf16 on
 * register operands, i.e. workgroups * 4 * iters * 8 * 32768 flops, and
 * writing one checksum float per wave to out (workgroups * 4 floats). */
NTOPS_API int ntops_mfma_rate_probe(int64_t workgroups, int64_t iters, float* out, void* stream);

/* ntops_conv2d without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  No ntops counterpart.  The workspace is a
 * fixed scratch array inside the library, NTOPS_CONV2D_NOALLOC_MAX_SCRATCH
 * bytes on each GPU it runs on, held until the process ends; images run in
 * chunks that fit it, and a problem whose single image needs more is
 * rejected with NTOPS_ERR_UNSUPPORTED.  Nothing is allocated or freed by the
 * call.  Every call on one GPU shares that GPU's scratch: calls that overlap
 * on one GPU (concurrent streams or host threads) race.  Arguments and
 * results otherwise as ntops_conv2d. */
#define NTOPS_CONV2D_NOALLOC_MAX_SCRATCH ((int64_t)64 << 20)
NTOPS_API int ntops_conv2d_noalloc(int dtype, int64_t N, int64_t C, int64_t H, int64_t W,
               int64_t K, int64_t R, int64_t S, int64_t P, int64_t Q,
               int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
               int64_t dil_h, int64_t dil_w,
               const void* x, const int64_t* x_strides,
               const void* w, const int64_t* w_strides,
               const void* bias, int64_t bias_stride,
               void* out, const int64_t* out_strides, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NTOPS_AMD_H */
