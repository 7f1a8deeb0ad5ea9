// softmax over one axis, viewed as (outer, dim_size, inner).
//
// Math follows kernels/softmax.py:9-29 (max, sum of exp(x - max), then
// exp(x - max) / sum) with torch's accumulation rule, which the build keeps:
// max and sum in fp32 (fp64 for fp64 output) and a single rounding of
// exp(x - max) * (1 / sum) to the output dtype.  The input is first rounded to
// the output dtype, as torch does for softmax(..., dtype=).  A row that is all
// -inf yields NaN (exp(-inf - -inf) = NaN), like torch.
//
// inner == 1 (softmax over a contiguous last axis):
//   vector path -- row held in VGPRs (rowcommon.h), one HBM read and one HBM
//   write per element;
//   looped path -- any stride or dtype pair, one 256-thread block per row.
// inner > 1: one thread per (outer, inner) column walking dim_size; adjacent
//   threads touch adjacent inner elements, so every pass is coalesced.
#include "dispatch.h"
#include "rowcommon.h"

namespace ntops {
namespace {

__device__ __forceinline__ float ex(float v) { return expf(v); }
__device__ __forceinline__ double ex(double v) { return exp(v); }

template <typename C>
__device__ __forceinline__ C cmax(C a, C b) {
  return (a > b || a != a) ? a : b;
}

template <typename T, typename C, int CHUNKS, int WPR>
__global__ __launch_bounds__(RowShape<WPR>::kThreads) void k_softmax_vec(
    const T* __restrict__ x, int64_t xs, T* __restrict__ y, int64_t ys, int64_t rows, int cols) {
  constexpr int V = Pack16<T>::N;
  constexpr int RPB = RowShape<WPR>::kRowsPerBlock;
  __shared__ C red0[RPB * WPR];
  __shared__ C red1[RPB * WPR];
  const RowPos p = row_pos<WPR>();
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + p.row_in_block;
  const bool row_ok = row < rows;
  const int npk = cols / V;
  const T* xr = x + row * xs;
  const C ninf = -__builtin_huge_val();

  C v[CHUNKS][V];
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int pk = pack_of<WPR>(p, c);
    if (row_ok && pk < npk) {
      const Pack16<T> r = load16_nt(xr + pk * V);
#pragma unroll
      for (int i = 0; i < V; ++i) v[c][i] = static_cast<C>(r.v[i]);
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i) v[c][i] = ninf;
    }
  }
  C m = ninf;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
    for (int i = 0; i < V; ++i) m = cmax(m, v[c][i]);
  m = row_max<WPR>(m, red0, p);
  C s = 0;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const bool ok = pack_of<WPR>(p, c) < npk;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      v[c][i] = ex(v[c][i] - m);
      if (ok) s += v[c][i];
    }
  }
  s = row_sum<WPR>(s, red1, p);
  const C inv = C(1) / s;
  if (!row_ok) return;
  T* yr = y + row * ys;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int pk = pack_of<WPR>(p, c);
    if (pk < npk) {
      Pack16<T> o;
#pragma unroll
      for (int i = 0; i < V; ++i) o.v[i] = static_cast<T>(v[c][i] * inv);
      store16_nt(yr + pk * V, o);
    }
  }
}

// One block per row, any element stride, input converted to the output dtype
// first.
template <typename Ti, typename To, typename C>
__global__ __launch_bounds__(256) void k_softmax_loop(const Ti* x, int64_t xs0, int64_t xs1,
                                                      To* y, int64_t ys0, int64_t ys1,
                                                      int64_t cols) {
  __shared__ C red[4];
  const int64_t row = blockIdx.x;
  const Ti* xr = x + row * xs0;
  To* yr = y + row * ys0;
  C m = -__builtin_huge_val();
  for (int64_t j = threadIdx.x; j < cols; j += 256)
    m = cmax(m, static_cast<C>(convert<To>(xr[j * xs1])));
  m = block_max256(m, red);
  C s = 0;
  for (int64_t j = threadIdx.x; j < cols; j += 256)
    s += ex(static_cast<C>(convert<To>(xr[j * xs1])) - m);
  s = block_sum256(s, red);
  const C inv = C(1) / s;
  for (int64_t j = threadIdx.x; j < cols; j += 256)
    yr[j * ys1] = convert<To>(ex(static_cast<C>(convert<To>(xr[j * xs1])) - m) * inv);
}

// One thread per (outer, inner) column.
template <typename Ti, typename To, typename C>
__global__ __launch_bounds__(256) void k_softmax_col(const Ti* x, int64_t xs0, int64_t xs1,
                                                     int64_t xs2, To* y, int64_t ys0,
                                                     int64_t ys1, int64_t ys2, int64_t outer,
                                                     int64_t dim, int64_t inner) {
  const int64_t cols_total = outer * inner;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; t < cols_total;
       t += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t o = t / inner;
    const int64_t in = t - o * inner;
    const Ti* xc = x + o * xs0 + in * xs2;
    To* yc = y + o * ys0 + in * ys2;
    C m = -__builtin_huge_val();
    for (int64_t j = 0; j < dim; ++j) m = cmax(m, static_cast<C>(convert<To>(xc[j * xs1])));
    C s = 0;
    for (int64_t j = 0; j < dim; ++j) s += ex(static_cast<C>(convert<To>(xc[j * xs1])) - m);
    const C inv = C(1) / s;
    for (int64_t j = 0; j < dim; ++j)
      yc[j * ys1] = convert<To>(ex(static_cast<C>(convert<To>(xc[j * xs1])) - m) * inv);
  }
}

template <typename Ti, typename To>
int run_softmax(int64_t outer, int64_t dim, int64_t inner, const void* xv, const int64_t* xs,
                void* yv, const int64_t* ys, hipStream_t st) {
  using C = typename std::conditional<std::is_same<To, double>::value, double, float>::type;
  const Ti* x = static_cast<const Ti*>(xv);
  To* y = static_cast<To*>(yv);
  if (inner == 1) {
    if constexpr (std::is_same<Ti, To>::value) {
      constexpr int V = Pack16<To>::N;
      VecCfg cfg;
      const bool vec = xs[1] == 1 && ys[1] == 1 && dim % V == 0 && xs[0] % V == 0 &&
                       ys[0] % V == 0 && aligned16(x) && aligned16(y) && pick_row_cfg(dim / V, &cfg) &&
                       outer <= 0x7fffffffLL * 4;
      if (vec) {
#define NTOPS_SM_CASE(CH, WP)                                                                  \
  if (cfg.chunks == CH && cfg.wpr == WP) {                                                     \
    constexpr int RPB = RowShape<WP>::kRowsPerBlock;                                           \
    hipLaunchKernelGGL((k_softmax_vec<To, C, CH, WP>), dim3(ceil_div(outer, RPB)),             \
                       dim3(RowShape<WP>::kThreads), 0, st, x, xs[0], y, ys[0], outer,         \
                       static_cast<int>(dim));                                                 \
    return check_launch("softmax");                                                            \
  }
        NTOPS_ROW_CASES(NTOPS_SM_CASE)
#undef NTOPS_SM_CASE
      }
    }
    if (outer > 0x7fffffffLL) return set_error(NTOPS_ERR_UNSUPPORTED, "softmax: too many rows");
    hipLaunchKernelGGL((k_softmax_loop<Ti, To, C>), dim3(outer), dim3(256), 0, st, x, xs[0], xs[1],
                       y, ys[0], ys[1], dim);
    return check_launch("softmax");
  }
  int64_t blocks = ceil_div(outer * inner, 256);
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL((k_softmax_col<Ti, To, C>), dim3(blocks), dim3(256), 0, st, x, xs[0], xs[1],
                     xs[2], y, ys[0], ys[1], ys[2], outer, dim, inner);
  return check_launch("softmax");
}

}  // namespace
}  // namespace ntops

using namespace ntops;

extern "C" int ntops_softmax(int in_dtype, int out_dtype, int64_t outer, int64_t dim_size,
                             int64_t inner, const void* x, const int64_t* x_strides, void* y,
                             const int64_t* y_strides, void* stream) {
  if (outer < 0 || dim_size < 0 || inner < 0)
    return set_error(NTOPS_ERR_INVALID, "softmax: negative size");
  if (outer == 0 || dim_size == 0 || inner == 0) return NTOPS_OK;
  if (x == nullptr || y == nullptr || x_strides == nullptr || y_strides == nullptr)
    return set_error(NTOPS_ERR_INVALID, "softmax: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  return dispatch_float(in_dtype, "softmax", [&](auto itag) {
    using Ti = decltype(itag);
    return dispatch_float(out_dtype, "softmax", [&](auto otag) {
      using To = decltype(otag);
      return run_softmax<Ti, To>(outer, dim_size, inner, x, x_strides, y, y_strides, st);
    });
  });
}
