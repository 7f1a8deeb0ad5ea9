// Dtype conversion / layout copy.  The wrappers use it for torch's type
// promotion (operands converted to the common dtype before an elementwise
// op) and to materialise contiguous copies of views the row kernels cannot
// address, so no data movement falls back to torch.
#include <algorithm>

#include "dispatch.h"

namespace ntops {
namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 8;

template <typename S, typename D>
__global__ __launch_bounds__(kThreads) void k_cast_dense(const S* x, D* y, int64_t n) {
  const int64_t base = block_id() * (kThreads * kPerThread) + threadIdx.x;  // blocks_2d grid
  S r[kPerThread];
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    const int64_t i = base + u * kThreads;
    if (i < n) r[u] = x[i];
  }
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    const int64_t i = base + u * kThreads;
    if (i < n) y[i] = convert<D>(r[u]);
  }
}

// Dense conversion between element types of one size (incl. the plain copy
// S == D): one 16-byte pack per thread, non-temporal loads and stores (the
// data streams through once), block 0 converts the tail.
template <typename S, typename D>
__global__ __launch_bounds__(kThreads) void k_cast_pack(const S* x, D* y, int64_t npack, int64_t n) {
  static_assert(sizeof(S) == sizeof(D), "same-size element types");
  constexpr int V = Pack16<S>::N;
  const int64_t p = block_id() * kThreads + threadIdx.x;  // blocks_2d grid
  if (p < npack) {
    const Pack16<S> r = load16_nt(x + p * V);
    Pack16<D> o;
#pragma unroll
    for (int i = 0; i < V; ++i) o.v[i] = convert<D>(r.v[i]);
    store16_nt(y + p * V, o);
  }
  if (block_id() == 0) {
    const int64_t i = npack * V + threadIdx.x;
    if (threadIdx.x < V && i < n) y[i] = convert<D>(x[i]);
  }
}

template <typename S, typename D, typename I>
__global__ __launch_bounds__(kThreads) void k_cast_strided(KSpace<2, I> sp, const S* x, D* y,
                                                           I n) {
  for (I i = static_cast<I>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<I>(gridDim.x) * kThreads) {
    I off[2];
    strided_offsets<2, I>(sp, i, off);
    y[off[1]] = convert<D>(x[off[0]]);
  }
}

template <typename S, typename D>
int launch_cast(int ndim, const int64_t* shape, const void* xv, const int64_t* xs, void* yv,
                const int64_t* ys, hipStream_t st) {
  const int64_t* strides[2] = {xs, ys};
  StridedSpace<2> sp;
  int64_t n = 0;
  if (!build_space<2>(ndim, shape, strides, &sp, &n))
    return set_error(NTOPS_ERR_INVALID, "ntops_cast: more than %d non-mergeable dims",
                     NTOPS_MAX_DIMS);
  if (n == 0) return NTOPS_OK;
  const S* x = static_cast<const S*>(xv);
  D* y = static_cast<D*>(yv);
  const bool dense = sp.ndim == 0 || (sp.ndim == 1 && sp.stride[0][0] == 1 && sp.stride[1][0] == 1);
  if constexpr (sizeof(S) == sizeof(D) && sizeof(S) <= 16) {
    if (dense && aligned16(x) && aligned16(y)) {
      constexpr int V = 16 / sizeof(S);
      const int64_t npack = n / V;
      const int64_t blocks = std::max<int64_t>(1, ceil_div(npack, static_cast<int64_t>(kThreads)));
      hipLaunchKernelGGL((k_cast_pack<S, D>), blocks_2d(blocks), dim3(kThreads), 0, st, x, y, npack, n);
      return check_launch("ntops_cast");
    }
  }
  if (dense) {
    const int64_t blocks = ceil_div(n, static_cast<int64_t>(kThreads) * kPerThread);
    hipLaunchKernelGGL((k_cast_dense<S, D>), blocks_2d(blocks), dim3(kThreads), 0, st, x, y, n);
  } else {
    int64_t blocks = ceil_div(n, kThreads);
    if (blocks > 65536) blocks = 65536;
    if (fits_int32(sp, n))
      hipLaunchKernelGGL((k_cast_strided<S, D, int32_t>), dim3(blocks), dim3(kThreads), 0, st,
                         to_kspace<2, int32_t>(sp), x, y, static_cast<int32_t>(n));
    else
      hipLaunchKernelGGL((k_cast_strided<S, D, int64_t>), dim3(blocks), dim3(kThreads), 0, st,
                         to_kspace<2, int64_t>(sp), x, y, n);
  }
  return check_launch("ntops_cast");
}

}  // namespace
}  // namespace ntops

using namespace ntops;

extern "C" int ntops_cast(int src_dtype, int dst_dtype, int ndim, const int64_t* shape,
                          const void* x, const int64_t* x_strides, void* y,
                          const int64_t* y_strides, void* stream) {
  if (ndim < 0 || ndim > 64) return set_error(NTOPS_ERR_INVALID, "ntops_cast: bad ndim %d", ndim);
  int64_t numel = 1;
  for (int d = 0; d < ndim; ++d) {
    if (shape[d] < 0) return set_error(NTOPS_ERR_INVALID, "ntops_cast: negative extent");
    numel *= shape[d];
  }
  if (numel > 0 && (x == nullptr || y == nullptr))
    return set_error(NTOPS_ERR_INVALID, "ntops_cast: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  return dispatch_all(src_dtype, "ntops_cast", [&](auto stag) {
    using S = decltype(stag);
    return dispatch_all(dst_dtype, "ntops_cast", [&](auto dtag) {
      using D = decltype(dtag);
      return launch_cast<S, D>(ndim, shape, x, x_strides, y, y_strides, st);
    });
  });
}
