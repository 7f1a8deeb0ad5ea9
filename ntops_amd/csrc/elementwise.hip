// Elementwise family for gfx950: silu, gelu (erf / tanh), exp, bitwise_not,
// add, mul, bitwise_and, bitwise_or.
//
// Per-element math follows the reference applications
//   kernels/silu.py:10, kernels/gelu.py:11,14-26, kernels/exp.py:10,
//   kernels/bitwise_not.py:9-14, kernels/add.py:10, kernels/mul.py:9,
//   kernels/bitwise_and.py:9, kernels/bitwise_or.py:9
// with torch's CPU conventions where ntops leaves them open (16-bit floats
// compute in fp32 and round once; add's alpha is rounded to the tensor dtype
// and applied with a fused multiply-add).
//
// Two launch shapes:
//  * dense: every operand is one contiguous, 16-byte aligned run.  Each
//    thread moves UNROLL 16-byte packs per operand, all loads issued before
//    the first use so that ~UNROLL*16 B per lane are in flight; packs of a
//    block are consecutive 4 KiB runs (fully coalesced).
//  * strided: any strides (0 = broadcast) over up to 8 merged dims, 32-bit
//    index math whenever every offset fits.
#include "dispatch.h"

namespace ntops {
namespace {

constexpr int kThreads = 256;
// One 16-byte pack per operand per thread and many workgroups: on MI355X this
// streams at ~6.3 TB/s on 128 MiB copies, ahead of deeper per-thread unrolls.
constexpr int kUnroll = 1;

__device__ __forceinline__ float ex(float v) { return expf(v); }
__device__ __forceinline__ double ex(double v) { return exp(v); }
__device__ __forceinline__ float er(float v) { return erff(v); }
__device__ __forceinline__ double er(double v) { return erf(v); }
__device__ __forceinline__ float th(float v) { return tanhf(v); }
__device__ __forceinline__ double th(double v) { return tanh(v); }
__device__ __forceinline__ float fm(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double fm(double a, double b, double c) { return __builtin_fma(a, b, c); }

// ------------------------------------------------------------ unary ops --
// silu.py:10   output = input / (1 + exp(-fp32(input)))
struct SiluF {
  template <typename T>
  __device__ __forceinline__ T operator()(T v) const {
    using C = opmath_t<T>;
    const C x = convert<C>(v);
    return convert<T>(x / (C(1) + ex(-x)));
  }
};
// gelu.py:11   input * 0.5 * (1 + erf(input / sqrt(2))); the 1/sqrt(2) factor
// is applied as a multiply by M_SQRT1_2, as torch's CPU kernel does.
struct GeluF {
  template <typename T>
  __device__ __forceinline__ T operator()(T v) const {
    using C = opmath_t<T>;
    const C x = convert<C>(v);
    return convert<T>(x * C(0.5) * (C(1) + er(x * C(M_SQRT1_2))));
  }
};
// gelu.py:14-26  0.5 * x * (1 + tanh(sqrt(2/pi) * (x + 0.044715 x^3)))
struct GeluTanhF {
  template <typename T>
  __device__ __forceinline__ T operator()(T v) const {
    using C = opmath_t<T>;
    const C x = convert<C>(v);
    const C beta = C(M_SQRT2 * M_2_SQRTPI * 0.5);
    const C kappa = C(0.044715);
    const C cube = x * x * x;
    const C inner = beta * (x + kappa * cube);
    return convert<T>(C(0.5) * x * (C(1) + th(inner)));
  }
};
// exp.py:10
struct ExpF {
  template <typename T>
  __device__ __forceinline__ T operator()(T v) const {
    using C = opmath_t<T>;
    return convert<T>(ex(convert<C>(v)));
  }
};
// bitwise_not.py:10 (~x) and :14 (logical not for bool)
struct NotF {
  template <typename T>
  __device__ __forceinline__ T operator()(T v) const {
    if constexpr (std::is_same<T, bool>::value)
      return !v;
    else
      return static_cast<T>(~v);
  }
};

// ----------------------------------------------------------- binary ops --
// add.py:10  input + alpha * other.  Floating: alpha rounded to T, then
// fma(other, alpha, input) in opmath.  Integral: modular arithmetic.
template <typename T, bool F = IsFloat<T>::v>
struct AddF;
template <typename T>
struct AddF<T, true> {
  double alpha;
  __device__ __forceinline__ T operator()(T a, T b) const {
    using C = opmath_t<T>;
    const C al = convert<C>(convert<T>(alpha));
    return convert<T>(fm(convert<C>(b), al, convert<C>(a)));
  }
  // Python-number `other`: torch's CPU add rounds it to T as well.
  __device__ __forceinline__ opmath_t<T> scalar_b(double b) const {
    return convert<opmath_t<T>>(convert<T>(b));
  }
  __device__ __forceinline__ T with_scalar(T a, opmath_t<T> b) const {
    using C = opmath_t<T>;
    const C al = convert<C>(convert<T>(alpha));
    return convert<T>(fm(b, al, convert<C>(a)));
  }
};
template <typename T>
struct AddF<T, false> {
  int64_t alpha;
  __device__ __forceinline__ T operator()(T a, T b) const {
    const uint64_t r = static_cast<uint64_t>(static_cast<int64_t>(a)) +
                       static_cast<uint64_t>(alpha) * static_cast<uint64_t>(static_cast<int64_t>(b));
    if constexpr (std::is_same<T, bool>::value)
      return r != 0;
    else
      return static_cast<T>(r);
  }
  __device__ __forceinline__ int64_t scalar_b(int64_t b) const { return b; }
  __device__ __forceinline__ T with_scalar(T a, int64_t b) const {
    const uint64_t r = static_cast<uint64_t>(static_cast<int64_t>(a)) +
                       static_cast<uint64_t>(alpha) * static_cast<uint64_t>(b);
    if constexpr (std::is_same<T, bool>::value)
      return r != 0;
    else
      return static_cast<T>(r);
  }
};

// mul.py:9  input * other.  A Python-number `other` stays in opmath (torch's
// CPU mul does not round it to T).
template <typename T, bool F = IsFloat<T>::v>
struct MulF;
template <typename T>
struct MulF<T, true> {
  __device__ __forceinline__ T operator()(T a, T b) const {
    using C = opmath_t<T>;
    return convert<T>(convert<C>(a) * convert<C>(b));
  }
  __device__ __forceinline__ opmath_t<T> scalar_b(double b) const {
    return static_cast<opmath_t<T>>(b);
  }
  __device__ __forceinline__ T with_scalar(T a, opmath_t<T> b) const {
    return convert<T>(convert<opmath_t<T>>(a) * b);
  }
};
template <typename T>
struct MulF<T, false> {
  __device__ __forceinline__ T operator()(T a, T b) const {
    if constexpr (std::is_same<T, bool>::value)
      return a && b;
    else
      return static_cast<T>(static_cast<uint64_t>(static_cast<int64_t>(a)) *
                            static_cast<uint64_t>(static_cast<int64_t>(b)));
  }
  __device__ __forceinline__ int64_t scalar_b(int64_t b) const { return b; }
  __device__ __forceinline__ T with_scalar(T a, int64_t b) const {
    if constexpr (std::is_same<T, bool>::value)
      return a && (b != 0);
    else
      return static_cast<T>(static_cast<uint64_t>(static_cast<int64_t>(a)) * static_cast<uint64_t>(b));
  }
};

// bitwise_and.py:9 / bitwise_or.py:9
template <bool OR>
struct BitF {
  template <typename T>
  __device__ __forceinline__ T operator()(T a, T b) const {
    if constexpr (std::is_same<T, bool>::value)
      return OR ? (a || b) : (a && b);
    else
      return OR ? static_cast<T>(a | b) : static_cast<T>(a & b);
  }
  __device__ __forceinline__ int64_t scalar_b(int64_t b) const { return b; }
  template <typename T>
  __device__ __forceinline__ T with_scalar(T a, int64_t b) const {
    if constexpr (std::is_same<T, bool>::value)
      return OR ? (a || b != 0) : (a && b != 0);
    else
      return OR ? static_cast<T>(a | static_cast<T>(b)) : static_cast<T>(a & static_cast<T>(b));
  }
};

// Scalar-operand type of a functor for element type T.
template <typename T>
using scalar_arg_t = typename std::conditional<IsFloat<T>::v, opmath_t<T>, int64_t>::type;

// ------------------------------------------------------------- kernels --
template <typename T, typename F>
__global__ __launch_bounds__(kThreads) void k_unary_dense(const T* x, T* y, int64_t npack,
                                                          int64_t n, F f) {
  constexpr int V = Pack16<T>::N;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kThreads * kUnroll) + threadIdx.x;
  Pack16<T> r[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t p = base + u * kThreads;
    if (p < npack) r[u] = load16_nt(x + p * V);
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t p = base + u * kThreads;
    if (p < npack) {
      Pack16<T> o;
#pragma unroll
      for (int i = 0; i < V; ++i) o.v[i] = f(r[u].v[i]);
      store16_nt(y + p * V, o);
    }
  }
  if (blockIdx.x == 0) {
    const int64_t i = npack * V + threadIdx.x;
    if (threadIdx.x < V && i < n) y[i] = f(x[i]);
  }
}

template <typename T, typename F, typename I>
__global__ __launch_bounds__(kThreads) void k_unary_strided(KSpace<2, I> sp, const T* x, T* y,
                                                            I n, F f) {
  for (I i = static_cast<I>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<I>(gridDim.x) * kThreads) {
    I off[2];
    strided_offsets<2, I>(sp, i, off);
    y[off[1]] = f(x[off[0]]);
  }
}

template <typename T, typename F>
__global__ __launch_bounds__(kThreads) void k_binary_dense(const T* a, const T* b, T* y,
                                                           int64_t npack, int64_t n, F f) {
  constexpr int V = Pack16<T>::N;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kThreads * kUnroll) + threadIdx.x;
  Pack16<T> ra[kUnroll], rb[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t p = base + u * kThreads;
    if (p < npack) {
      ra[u] = load16_nt(a + p * V);
      rb[u] = load16_nt(b + p * V);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t p = base + u * kThreads;
    if (p < npack) {
      Pack16<T> o;
#pragma unroll
      for (int i = 0; i < V; ++i) o.v[i] = f(ra[u].v[i], rb[u].v[i]);
      store16_nt(y + p * V, o);
    }
  }
  if (blockIdx.x == 0) {
    const int64_t i = npack * V + threadIdx.x;
    if (threadIdx.x < V && i < n) y[i] = f(a[i], b[i]);
  }
}

template <typename T, typename F, typename S>
__global__ __launch_bounds__(kThreads) void k_binary_scalar_dense(const T* a, S braw, T* y,
                                                                  int64_t npack, int64_t n, F f) {
  constexpr int V = Pack16<T>::N;
  const auto bs = f.scalar_b(braw);
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kThreads * kUnroll) + threadIdx.x;
  Pack16<T> ra[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t p = base + u * kThreads;
    if (p < npack) ra[u] = load16_nt(a + p * V);
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t p = base + u * kThreads;
    if (p < npack) {
      Pack16<T> o;
#pragma unroll
      for (int i = 0; i < V; ++i) o.v[i] = f.with_scalar(ra[u].v[i], bs);
      store16_nt(y + p * V, o);
    }
  }
  if (blockIdx.x == 0) {
    const int64_t i = npack * V + threadIdx.x;
    if (threadIdx.x < V && i < n) y[i] = f.with_scalar(a[i], bs);
  }
}

template <typename T, typename F, typename I>
__global__ __launch_bounds__(kThreads) void k_binary_strided(KSpace<3, I> sp, const T* a,
                                                             const T* b, T* y, I n, F f) {
  for (I i = static_cast<I>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<I>(gridDim.x) * kThreads) {
    I off[3];
    strided_offsets<3, I>(sp, i, off);
    y[off[2]] = f(a[off[0]], b[off[1]]);
  }
}

template <typename T, typename F, typename S, typename I>
__global__ __launch_bounds__(kThreads) void k_binary_scalar_strided(KSpace<2, I> sp, const T* a,
                                                                    S braw, T* y, I n, F f) {
  const auto bs = f.scalar_b(braw);
  for (I i = static_cast<I>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<I>(gridDim.x) * kThreads) {
    I off[2];
    strided_offsets<2, I>(sp, i, off);
    y[off[1]] = f.with_scalar(a[off[0]], bs);
  }
}

// ------------------------------------------------------------ launchers --
inline int64_t dense_blocks(int64_t npack) {
  return ceil_div(npack > 0 ? npack : 1, static_cast<int64_t>(kThreads) * kUnroll);
}
inline unsigned strided_blocks(int64_t n) {
  int64_t b = ceil_div(n, kThreads);
  if (b > 65536) b = 65536;
  return static_cast<unsigned>(b < 1 ? 1 : b);
}

template <int NOPS>
bool space_is_dense(const StridedSpace<NOPS>& sp) {
  if (sp.ndim == 0) return true;
  if (sp.ndim != 1) return false;
  for (int k = 0; k < NOPS; ++k)
    if (sp.stride[k][0] != 1) return false;
  return true;
}

template <typename T, typename F>
int launch_unary(const F& f, int ndim, const int64_t* shape, const void* xv, const int64_t* xs,
                 void* yv, const int64_t* ys, hipStream_t st, const char* what) {
  const int64_t* strides[2] = {xs, ys};
  StridedSpace<2> sp;
  int64_t n = 0;
  if (!build_space<2>(ndim, shape, strides, &sp, &n))
    return set_error(NTOPS_ERR_INVALID, "%s: more than %d non-mergeable dims", what, NTOPS_MAX_DIMS);
  if (n == 0) return NTOPS_OK;
  const T* x = static_cast<const T*>(xv);
  T* y = static_cast<T*>(yv);
  if (space_is_dense(sp) && aligned16(x) && aligned16(y)) {
    const int64_t npack = n / Pack16<T>::N;
    hipLaunchKernelGGL((k_unary_dense<T, F>), dim3(dense_blocks(npack)), dim3(kThreads), 0, st, x,
                       y, npack, n, f);
  } else if (fits_int32(sp, n)) {
    hipLaunchKernelGGL((k_unary_strided<T, F, int32_t>), dim3(strided_blocks(n)), dim3(kThreads),
                       0, st, to_kspace<2, int32_t>(sp), x, y, static_cast<int32_t>(n), f);
  } else {
    hipLaunchKernelGGL((k_unary_strided<T, F, int64_t>), dim3(strided_blocks(n)), dim3(kThreads),
                       0, st, to_kspace<2, int64_t>(sp), x, y, n, f);
  }
  return check_launch(what);
}

template <typename T, typename F>
int launch_binary(const F& f, int ndim, const int64_t* shape, const void* av, const int64_t* as,
                  const void* bv, const int64_t* bs, double b_f, int64_t b_i, void* yv,
                  const int64_t* ys, hipStream_t st, const char* what) {
  const T* a = static_cast<const T*>(av);
  const T* b = static_cast<const T*>(bv);
  T* y = static_cast<T*>(yv);
  using S = typename std::conditional<IsFloat<T>::v, double, int64_t>::type;
  S braw;
  if constexpr (IsFloat<T>::v) {
    braw = b_f;
    (void)b_i;
  } else {
    braw = b_i;
    (void)b_f;
  }
  if (b == nullptr) {
    const int64_t* strides[2] = {as, ys};
    StridedSpace<2> sp;
    int64_t n = 0;
    if (!build_space<2>(ndim, shape, strides, &sp, &n))
      return set_error(NTOPS_ERR_INVALID, "%s: more than %d non-mergeable dims", what, NTOPS_MAX_DIMS);
    if (n == 0) return NTOPS_OK;
    if (space_is_dense(sp) && aligned16(a) && aligned16(y)) {
      const int64_t npack = n / Pack16<T>::N;
      hipLaunchKernelGGL((k_binary_scalar_dense<T, F, S>), dim3(dense_blocks(npack)),
                         dim3(kThreads), 0, st, a, braw, y, npack, n, f);
    } else if (fits_int32(sp, n)) {
      hipLaunchKernelGGL((k_binary_scalar_strided<T, F, S, int32_t>), dim3(strided_blocks(n)),
                         dim3(kThreads), 0, st, to_kspace<2, int32_t>(sp), a, braw, y,
                         static_cast<int32_t>(n), f);
    } else {
      hipLaunchKernelGGL((k_binary_scalar_strided<T, F, S, int64_t>), dim3(strided_blocks(n)),
                         dim3(kThreads), 0, st, to_kspace<2, int64_t>(sp), a, braw, y, n, f);
    }
    return check_launch(what);
  }
  const int64_t* strides[3] = {as, bs, ys};
  StridedSpace<3> sp;
  int64_t n = 0;
  if (!build_space<3>(ndim, shape, strides, &sp, &n))
    return set_error(NTOPS_ERR_INVALID, "%s: more than %d non-mergeable dims", what, NTOPS_MAX_DIMS);
  if (n == 0) return NTOPS_OK;
  if (space_is_dense(sp) && aligned16(a) && aligned16(b) && aligned16(y)) {
    const int64_t npack = n / Pack16<T>::N;
    hipLaunchKernelGGL((k_binary_dense<T, F>), dim3(dense_blocks(npack)), dim3(kThreads), 0, st, a,
                       b, y, npack, n, f);
  } else if (fits_int32(sp, n)) {
    hipLaunchKernelGGL((k_binary_strided<T, F, int32_t>), dim3(strided_blocks(n)), dim3(kThreads),
                       0, st, to_kspace<3, int32_t>(sp), a, b, y, static_cast<int32_t>(n), f);
  } else {
    hipLaunchKernelGGL((k_binary_strided<T, F, int64_t>), dim3(strided_blocks(n)), dim3(kThreads),
                       0, st, to_kspace<3, int64_t>(sp), a, b, y, n, f);
  }
  return check_launch(what);
}

// Validates the index space; pointers are only required when it is not
// empty (an empty tensor may have a null data pointer).
int check_common(const char* what, int ndim, const int64_t* shape, const void* x, const void* y) {
  if (ndim < 0 || ndim > 64) return set_error(NTOPS_ERR_INVALID, "%s: bad ndim %d", what, ndim);
  if (ndim > 0 && shape == nullptr) return set_error(NTOPS_ERR_INVALID, "%s: null shape", what);
  int64_t numel = 1;
  for (int d = 0; d < ndim; ++d) {
    if (shape[d] < 0) return set_error(NTOPS_ERR_INVALID, "%s: negative extent", what);
    numel *= shape[d];
  }
  if (numel == 0) return NTOPS_OK;
  if (y == nullptr) return set_error(NTOPS_ERR_INVALID, "%s: null output pointer", what);
  if (x == nullptr) return set_error(NTOPS_ERR_INVALID, "%s: null input pointer", what);
  return NTOPS_OK;
}

}  // namespace
}  // namespace ntops

using namespace ntops;

extern "C" int ntops_unary(int op, int dtype, int ndim, const int64_t* shape, const void* x,
                           const int64_t* x_strides, void* y, const int64_t* y_strides,
                           void* stream) {
  const char* what = "ntops_unary";
  if (int e = check_common(what, ndim, shape, x, y)) return e;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (op) {
    case NTOPS_UNARY_SILU:
      return dispatch_float(dtype, "silu", [&](auto tag) {
        using T = decltype(tag);
        return launch_unary<T>(SiluF{}, ndim, shape, x, x_strides, y, y_strides, st, "silu");
      });
    case NTOPS_UNARY_GELU:
      return dispatch_float(dtype, "gelu", [&](auto tag) {
        using T = decltype(tag);
        return launch_unary<T>(GeluF{}, ndim, shape, x, x_strides, y, y_strides, st, "gelu");
      });
    case NTOPS_UNARY_GELU_TANH:
      return dispatch_float(dtype, "gelu(tanh)", [&](auto tag) {
        using T = decltype(tag);
        return launch_unary<T>(GeluTanhF{}, ndim, shape, x, x_strides, y, y_strides, st, "gelu");
      });
    case NTOPS_UNARY_EXP:
      return dispatch_float(dtype, "exp", [&](auto tag) {
        using T = decltype(tag);
        return launch_unary<T>(ExpF{}, ndim, shape, x, x_strides, y, y_strides, st, "exp");
      });
    case NTOPS_UNARY_BITWISE_NOT:
      return dispatch_integral(dtype, "bitwise_not", [&](auto tag) {
        using T = decltype(tag);
        return launch_unary<T>(NotF{}, ndim, shape, x, x_strides, y, y_strides, st, "bitwise_not");
      });
    default:
      return set_error(NTOPS_ERR_UNSUPPORTED, "%s: unknown op %d", what, op);
  }
}

extern "C" int ntops_binary(int op, int dtype, int ndim, const int64_t* shape, const void* a,
                            const int64_t* a_strides, const void* b, const int64_t* b_strides,
                            double b_f, int64_t b_i, double alpha_f, int64_t alpha_i, void* out,
                            const int64_t* out_strides, void* stream) {
  const char* what = "ntops_binary";
  if (int e = check_common(what, ndim, shape, a, out)) return e;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (op) {
    case NTOPS_BINARY_ADD:
      return dispatch_all(dtype, "add", [&](auto tag) {
        using T = decltype(tag);
        AddF<T> f;
        if constexpr (IsFloat<T>::v)
          f.alpha = alpha_f;
        else
          f.alpha = alpha_i;
        return launch_binary<T>(f, ndim, shape, a, a_strides, b, b_strides, b_f, b_i, out,
                                out_strides, st, "add");
      });
    case NTOPS_BINARY_MUL:
      return dispatch_all(dtype, "mul", [&](auto tag) {
        using T = decltype(tag);
        return launch_binary<T>(MulF<T>{}, ndim, shape, a, a_strides, b, b_strides, b_f, b_i, out,
                                out_strides, st, "mul");
      });
    case NTOPS_BINARY_BITWISE_AND:
      return dispatch_integral(dtype, "bitwise_and", [&](auto tag) {
        using T = decltype(tag);
        return launch_binary<T>(BitF<false>{}, ndim, shape, a, a_strides, b, b_strides, b_f, b_i,
                                out, out_strides, st, "bitwise_and");
      });
    case NTOPS_BINARY_BITWISE_OR:
      return dispatch_integral(dtype, "bitwise_or", [&](auto tag) {
        using T = decltype(tag);
        return launch_binary<T>(BitF<true>{}, ndim, shape, a, a_strides, b, b_strides, b_f, b_i,
                                out, out_strides, st, "bitwise_or");
      });
    default:
      return set_error(NTOPS_ERR_UNSUPPORTED, "%s: unknown op %d", what, op);
  }
}
