// Internal (not exported) matrix-core GEMM entry points shared between
// translation units of the library.
#pragma once

#include "dispatch.h"

namespace ntops {

// out[b][m][n] = sum_k W[m][k] * B_b[k][n] (+ bias[m]) on the matrix cores
// (dtype BF16 or F16), where B_b is an implicit convolution operand: k-row
// kg = (c * R + r) * S + s of batch b starts at element
// b * b_batch + s * per_s + c * per_c + r * per_r of `b_base` and holds N
// contiguous elements.  W is row-major with row stride w_ld (16-byte
// aligned, w_ld % 8 == 0), shared by every batch; bias (may be NULL) has
// element stride bias_stride; out rows have unit column stride.  Requires
// N, per_s, per_c, per_r and b_batch to be multiples of 8 and a 16-byte
// aligned b_base.
int gemm_implicit_conv(int dtype, int batch, int M, int N, int K, const void* w, int64_t w_ld,
                       const void* b_base, int64_t b_batch, int R, int S, int64_t per_s, int64_t per_c,
                       int64_t per_r, const void* bias, int64_t bias_stride, void* out, int64_t out_batch,
                       int64_t out_ld, hipStream_t st);

// out[b][m][n] = sum_k W[m][k] * X_b[k][n] (+ bias[m]) on the matrix cores
// (BF16 or F16) for a convolution over a channels-last, zero-padded copy of
// the input: xt holds `batch` images of img_elems elements, each rows of wp
// pixels of C channels; output pixel n = p * Q + q, tap (r, s) and channel
// c = 32 cb + ci (k = ((cb * R + r) * S + s) * 32 + ci) read
// xt_b[((p * sh + r * dh) * wp + q * sw + s * dw) * C + c].  W is row-major (row stride K = R * S * C, 16-byte
// aligned), shared by every batch; bias (may be NULL) has element stride
// bias_stride; out rows have unit column stride.  Requires C % 32 == 0,
// N % 4 == 0, a 16-byte aligned xt and img_elems % 8 == 0.
int gemm_conv_channels_last(int dtype, int batch, int M, int N, int K, const void* w, const void* xt,
                            int64_t img_elems, int R, int S, int C, int Q, int sh, int sw, int wp, int dh,
                            int dw, const void* bias, int64_t bias_stride, void* out, int64_t out_batch,
                            int64_t out_ld, hipStream_t st);

}  // namespace ntops
