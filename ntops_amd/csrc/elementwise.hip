// Elementwise family for gfx950: silu, gelu (erf / tanh), exp, bitwise_not,
// relu, sigmoid, tanh, neg, abs, rsqrt, sin, cos; add, sub, mul, div (true /
// trunc / floor), pow, bitwise_and, bitwise_or; the comparisons eq ne gt ge
// lt le; isinf, isnan; clamp.
//
// Per-element math follows the reference applications
//   kernels/silu.py:10, kernels/gelu.py:11,14-26, kernels/exp.py:10,
//   kernels/bitwise_not.py:9-14, kernels/relu.py:9, kernels/sigmoid.py:10,
//   kernels/tanh.py:10-13, kernels/neg.py:9, kernels/abs.py:10,
//   kernels/rsqrt.py:10, kernels/sin.py:10, kernels/cos.py:10,
//   kernels/add.py:10, kernels/sub.py:10, kernels/mul.py:9,
//   kernels/div.py:9-18, kernels/pow.py:10, kernels/bitwise_and.py:9,
//   kernels/bitwise_or.py:9, kernels/{eq,ne,gt,ge,lt,le}.py:9,
//   kernels/isinf.py:9-11, kernels/isnan.py:9, kernels/clamp.py:9
// with torch's CPU conventions where ntops leaves them open (16-bit floats
// compute in fp32 and round once; add's alpha is rounded to the tensor dtype
// and applied with a fused multiply-add).
//
// Three launch shapes:
//  * dense: every operand is one contiguous, aligned run.  Each thread moves
//    one 16-byte pack of every input (V elements) and writes the V results
//    with one store (16 bytes, or V bytes for a bool result); packs of a
//    block are consecutive 4 KiB runs (fully coalesced).
//  * rows: two merged dims whose inner dim is unit-stride for every operand
//    and a whole number of packs, with any outer strides (0 included: a row
//    broadcast such as a bias, or row views of a wider tensor); one pack per
//    thread as in the dense shape, the row and pack from one division.
//  * strided: any strides (0 = broadcast) over up to 8 merged dims, 32-bit
//    index math whenever every offset fits.
// The output element type is the functor's result type (bool for the
// comparisons and isinf / isnan).
#include "dispatch.h"

namespace ntops {
namespace {

// One 16-byte pack per operand per thread and many 256-thread workgroups: on
// MI355X this streams at ~6.3 TB/s on 128 MiB copies, ahead of deeper
// per-thread unrolls.
constexpr int kThreads = 256;

__device__ __forceinline__ float ex(float v) { return expf(v); }
__device__ __forceinline__ double ex(double v) { return exp(v); }
__device__ __forceinline__ float er(float v) { return erff(v); }
__device__ __forceinline__ double er(double v) { return erf(v); }
__device__ __forceinline__ float th(float v) { return tanhf(v); }
__device__ __forceinline__ double th(double v) { return tanh(v); }
__device__ __forceinline__ float fm(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double fm(double a, double b, double c) { return __builtin_fma(a, b, c); }
__device__ __forceinline__ float sn(float v) { return sinf(v); }
__device__ __forceinline__ double sn(double v) { return sin(v); }
__device__ __forceinline__ float cs(float v) { return cosf(v); }
__device__ __forceinline__ double cs(double v) { return cos(v); }
__device__ __forceinline__ float sq(float v) { return __builtin_sqrtf(v); }  // IEEE (correctly rounded)
__device__ __forceinline__ double sq(double v) { return __builtin_sqrt(v); }
__device__ __forceinline__ float pw(float a, float b) { return powf(a, b); }
__device__ __forceinline__ double pw(double a, double b) { return pow(a, b); }
// Exact fmod.  When a and b are finite and the rounded quotient q = a / b
// has |trunc(q)| < 2^23, r = fma(-trunc(q), b, a) is exact: trunc(q) is the
// true truncated quotient n or, when a / b lies within half an ulp below an
// integer, n + 1 in magnitude; in the second case a - (n+1) b is a multiple
// of ulp(b) smaller than |b| (representable, so the fma is exact), has the
// opposite sign to a, and adding back |b| with a's sign is exact too.  A zero
// remainder takes a's sign, as fmod's does.  Everything else (huge
// quotients, infinities, NaN) goes to the library's bit-by-bit fmodf.
__device__ __forceinline__ float fmd(float a, float b) {
  const float n = __builtin_truncf(a / b);
  if (__builtin_fabsf(n) < 8388608.0f && __builtin_isfinite(b)) {
    float r = __builtin_fmaf(-n, b, a);
    if (r != 0.0f && __builtin_signbit(r) != __builtin_signbit(a)) r += __builtin_copysignf(__builtin_fabsf(b), a);
    return r == 0.0f ? __builtin_copysignf(0.0f, a) : r;
  }
  return fmodf(a, b);
}
__device__ __forceinline__ double fmd(double a, double b) { return fmod(a, b); }
__device__ __forceinline__ float flr(float v) { return floorf(v); }
__device__ __forceinline__ double flr(double v) { return floor(v); }
__device__ __forceinline__ float trc(float v) { return truncf(v); }
__device__ __forceinline__ double trc(double v) { return trunc(v); }
__device__ __forceinline__ float cpsgn(float a, float b) { return copysignf(a, b); }
__device__ __forceinline__ double cpsgn(double a, double b) { return copysign(a, b); }

// Two's complement negation without signed overflow.
template <typename T>
__device__ __forceinline__ T wrap_neg(T v) {
  return static_cast<T>(static_cast<uint64_t>(0) - static_cast<uint64_t>(static_cast<int64_t>(v)));
}

// clamp.py:9 with torch's rule: a NaN in x, then in lo, then in hi, is the
// result; otherwise min(max(x, lo), hi) (so lo > hi gives hi).  The result
// is always one of the three values, so no rounding happens.
template <typename T>
__device__ __forceinline__ T clamp_value(T x, T lo, T hi) {
  if constexpr (IsFloat<T>::v) {
    using C = opmath_t<T>;
    const C xv = convert<C>(x), l = convert<C>(lo), h = convert<C>(hi);
    if (xv != xv) return x;
    if (l != l) return lo;
    if (h != h) return hi;
    const T r = xv < l ? lo : x;
    return h < convert<C>(r) ? hi : r;
  } else {
    const T r = x < lo ? lo : x;
    return hi < r ? hi : r;
  }
}

// ------------------------------------------------- 16-bit fast routines --
// A 16-bit result keeps 8 (bf16) or 11 (fp16) significant bits, so for
// 16-bit T the transcendental ops below use the hardware exp2 / rcp / sin /
// cos (a few fp32 ulps) instead of the library's fp32-accurate routines,
// which made the bf16 forms VALU-bound (~58 % of HBM against ~77 % for
// fp32).  The error stays far below half a 16-bit ulp, so results differ
// from the fp32-accurate ones only where the fp32 value sits at a 16-bit
// rounding boundary (then by one ulp).
constexpr float kLog2eF = 1.44269504088896341f;
constexpr float kInv2PiF = 0.159154943091895336f;
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * kLog2eF); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
// 1 / (1 + exp(-x)): exp overflows to inf for x -> -inf, giving 0.
__device__ __forceinline__ float fast_sigmoid(float x) { return fast_rcp(1.0f + fast_exp(-x)); }
// tanh x = 1 - 2 / (exp(2x) + 1), odd-extended; below |x| = 2^-4 the odd
// Taylor polynomial x (1 - x^2/3 + 2x^4/15) (truncation < 2^-26 relative)
// avoids the cancellation.
__device__ __forceinline__ float fast_tanh(float x) {
  const float ax = __builtin_fabsf(x);
  const float big = 1.0f - 2.0f * fast_rcp(fast_exp(2.0f * ax) + 1.0f);
  const float x2 = x * x;
  const float small = ax * __builtin_fmaf(x2, __builtin_fmaf(x2, 0.133333333f, -0.333333333f), 1.0f);
  return __builtin_copysignf(ax < 0.0625f ? small : big, x);
}
// erf by Abramowitz & Stegun 7.1.26 (absolute error < 1.5e-7), odd-extended.
__device__ __forceinline__ float fast_erf(float x) {
  const float ax = __builtin_fabsf(x);
  const float t = fast_rcp(__builtin_fmaf(0.3275911f, ax, 1.0f));
  float p = __builtin_fmaf(1.061405429f, t, -1.453152027f);
  p = __builtin_fmaf(p, t, 1.421413741f);
  p = __builtin_fmaf(p, t, -0.284496736f);
  p = __builtin_fmaf(p, t, 0.254829592f);
  const float r = 1.0f - p * t * fast_exp(-ax * ax);
  return __builtin_copysignf(r, x);
}
// sin / cos from the hardware's v_sin / v_cos, which take the phase in
// revolutions (valid within +-256): x / (2 pi) carries an absolute error
// below |x| 2^-24 revolutions, so beyond |x| = 1024 (163 revolutions) the
// library routine (exact argument reduction) is used.
__device__ __forceinline__ float fast_sin(float x) {
  return __builtin_fabsf(x) < 1024.0f ? __builtin_amdgcn_sinf(x * kInv2PiF) : sinf(x);
}
__device__ __forceinline__ float fast_cos(float x) {
  return __builtin_fabsf(x) < 1024.0f ? __builtin_amdgcn_cosf(x * kInv2PiF) : cosf(x);
}
// a^b for a > 0, both finite: exp2(b log2 a) with the hardware log2 / exp2
// (relative error about |b log2 a| 2^-23 -- below 2^-12 while the result is
// within fp32 range of 2^+-126, far below a 16-bit ulp); every other case
// (negative or zero base, infinities, NaN, the integer-exponent rules) goes
// to the library pow.
__device__ __forceinline__ float fast_pow(float a, float b) {
  const bool plain = a > 0.0f && a < __builtin_huge_valf() && __builtin_fabsf(b) < __builtin_huge_valf();
  return plain ? __builtin_amdgcn_exp2f(b * __builtin_amdgcn_logf(a)) : powf(a, b);
}

// ------------------------------------------------------------ unary ops --
// silu.py:10   output = input / (1 + exp(-fp32(input)))
struct SiluF {
  template <typename T>
  __device__ __forceinline__ T operator()(T v) const {
    using C = opmath_t<T>;
    const C x = convert<C>(v);
    if constexpr (sizeof(T) == 2)
      return convert<T>(x * fast_sigmoid(x));
    else
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
    if constexpr (sizeof(T) == 2)
      return convert<T>(x * C(0.5) * (C(1) + fast_erf(x * C(M_SQRT1_2))));
    else
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
    if constexpr (sizeof(T) == 2)
      return convert<T>(C(0.5) * x * (C(1) + fast_tanh(inner)));
    else
      return convert<T>(C(0.5) * x * (C(1) + th(inner)));
  }
};
// exp.py:10
struct ExpF {
  template <typename T>
  __device__ __forceinline__ T operator()(T v) const {
    using C = opmath_t<T>;
    if constexpr (sizeof(T) == 2)
      return convert<T>(fast_exp(convert<C>(v)));
    else
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

// relu.py:9  max(0, x) as torch's clamp_min: NaN stays NaN, -0 stays -0.
struct ReluF {
  template <typename T>
  __device__ __forceinline__ T operator()(T v) const {
    if constexpr (IsFloat<T>::v) {
      using C = opmath_t<T>;
      return convert<C>(v) < C(0) ? T(0) : v;
    } else if constexpr (std::is_signed<T>::value) {
      return v < T(0) ? T(0) : v;
    } else {
      return v;
    }
  }
};
// sigmoid.py:10  1 / (1 + exp(-x)) in opmath, one rounding.
struct SigmoidF {
  template <typename T>
  __device__ __forceinline__ T operator()(T v) const {
    using C = opmath_t<T>;
    if constexpr (sizeof(T) == 2)
      return convert<T>(fast_sigmoid(convert<C>(v)));
    else
      return convert<T>(C(1) / (C(1) + ex(-convert<C>(v))));
  }
};
// tanh.py:10-13 (the reference spells tanh out through exp, which overflows
// to NaN for |x| > 88; the library tanh is used, as torch does).
struct TanhF {
  template <typename T>
  __device__ __forceinline__ T operator()(T v) const {
    using C = opmath_t<T>;
    if constexpr (sizeof(T) == 2)
      return convert<T>(fast_tanh(convert<C>(v)));
    else
      return convert<T>(th(convert<C>(v)));
  }
};
// neg.py:9
struct NegF {
  template <typename T>
  __device__ __forceinline__ T operator()(T v) const {
    if constexpr (IsFloat<T>::v)
      return -v;
    else
      return wrap_neg(v);
  }
};
// abs.py:10  (sign bit cleared for floats; integer minimum wraps)
struct AbsF {
  template <typename T>
  __device__ __forceinline__ T operator()(T v) const {
    if constexpr (std::is_same<T, double>::value) {
      return __builtin_fabs(v);
    } else if constexpr (IsFloat<T>::v) {
      return convert<T>(__builtin_fabsf(convert<float>(v)));
    } else if constexpr (std::is_signed<T>::value) {
      return v < T(0) ? wrap_neg(v) : v;
    } else {
      return v;
    }
  }
};
// rsqrt.py:10  1 / sqrt(x): IEEE square root, then IEEE division (bit-exact
// with torch's CPU kernel).
struct RsqrtF {
  template <typename T>
  __device__ __forceinline__ T operator()(T v) const {
    using C = opmath_t<T>;
    return convert<T>(C(1) / sq(convert<C>(v)));
  }
};
// sin.py:10 / cos.py:10
struct SinF {
  template <typename T>
  __device__ __forceinline__ T operator()(T v) const {
    using C = opmath_t<T>;
    if constexpr (sizeof(T) == 2)
      return convert<T>(fast_sin(convert<C>(v)));
    else
      return convert<T>(sn(convert<C>(v)));
  }
};
struct CosF {
  template <typename T>
  __device__ __forceinline__ T operator()(T v) const {
    using C = opmath_t<T>;
    if constexpr (sizeof(T) == 2)
      return convert<T>(fast_cos(convert<C>(v)));
    else
      return convert<T>(cs(convert<C>(v)));
  }
};
// clamp with scalar (or absent) bounds, already rounded to T.
template <typename T>
struct ClampSF {
  T lo, hi;
  __device__ __forceinline__ T operator()(T v) const { return clamp_value(v, lo, hi); }
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

// div.py:9-18.  Floating: in opmath, one rounding (trunc of two 16-bit
// tensors truncates the quotient after rounding it to T, as torch's CPU
// kernel does).  A Python-number divisor stays in opmath (not rounded to T).
// MODE 0 = true division, 1 = trunc,
// 2 = floor (Python's floor division: the quotient of (a - fmod(a, b)) / b,
// corrected by the sign of the remainder and rounded to the nearest integer,
// so that e.g. 7.5 // -inf = -1 and 0 // -3 = -0).
template <typename C>
__device__ __forceinline__ C floor_divide(C a, C b) {
  if (b == C(0)) return a / b;
  const C mod = fmd(a, b);
  C div = (a - mod) / b;
  if (mod != C(0) && ((b < C(0)) != (mod < C(0)))) div -= C(1);
  if (div == C(0)) return cpsgn(C(0), a / b);
  C fl = flr(div);
  if (div - fl > C(0.5)) fl += C(1);
  return fl;
}
// fp32: the same result without the second division.  When b is finite and
// the rounded quotient q = a / b has |trunc(q)| < 2^21, the exact remainder
// and truncated quotient n come from one fma (as in fmd), and the sequence
// above provably returns n - corr (corr = 1 when the remainder is nonzero
// with the opposite sign to b): its (a - mod) / b is n times two roundings
// of relative size 2^-24, i.e. within 2^21 * 2^-23 = 0.25 of n, the "- 1"
// adds at most 0.125 more, and floor plus round-half-down then lands on the
// integer.  A zero result takes the sign of a / b, as above.  Larger
// quotients and non-finite operands run the sequence above.
__device__ __forceinline__ float floor_divide(float a, float b) {
  if (b == 0.0f) return a / b;
  const float q = a / b;
  float n = __builtin_truncf(q);
  if (__builtin_fabsf(n) < 2097152.0f && __builtin_isfinite(b)) {
    float r = __builtin_fmaf(-n, b, a);
    if (r != 0.0f && __builtin_signbit(r) != __builtin_signbit(a)) {
      r += __builtin_copysignf(__builtin_fabsf(b), a);
      n -= __builtin_copysignf(1.0f, n);
    }
    const float res = n - ((r != 0.0f && ((b < 0.0f) != (r < 0.0f))) ? 1.0f : 0.0f);
    return res == 0.0f ? __builtin_copysignf(0.0f, q) : res;
  }
  return floor_divide<float>(a, b);
}

template <int MODE, typename T, bool F = IsFloat<T>::v>
struct DivF;
template <int MODE, typename T>
struct DivF<MODE, T, true> {
  using C = opmath_t<T>;
  // ROUNDQ: round a 16-bit trunc quotient to T before truncating (torch's
  // tensor / tensor path; its tensor / number path truncates in opmath).
  template <bool ROUNDQ>
  __device__ __forceinline__ static C apply(C a, C b) {
    if constexpr (MODE == 0)
      return a / b;
    else if constexpr (MODE == 1)
      return ROUNDQ ? trc(convert<C>(convert<T>(a / b))) : trc(a / b);
    else
      return floor_divide(a, b);
  }
  __device__ __forceinline__ T operator()(T a, T b) const {
    return convert<T>(apply<true>(convert<C>(a), convert<C>(b)));
  }
  __device__ __forceinline__ C scalar_b(double b) const { return static_cast<C>(b); }
  __device__ __forceinline__ T with_scalar(T a, C b) const {
    return convert<T>(apply<false>(convert<C>(a), b));
  }
};
// Integer trunc / floor division in int64; division by zero gives 0 (torch's
// CPU kernel raises), b = -1 negates with wraparound.
// Types of up to 32 bits divide in 32-bit arithmetic (exact for every
// value they hold once b = 0 and b = -1 are taken out; a 64-bit division is
// a long software sequence on the GPU), int64 and wider scalars in 64-bit.
template <int MODE, typename T>
struct DivF<MODE, T, false> {
  template <typename I>
  __device__ __forceinline__ static I apply(I a, I b) {
    using U = typename std::make_unsigned<I>::type;
    if (b == 0) return 0;
    if (b == -1) return static_cast<I>(static_cast<U>(0) - static_cast<U>(a));
    I q = a / b;
    if constexpr (MODE == 2)
      if ((a % b != 0) && ((a < 0) != (b < 0))) q -= 1;
    return q;
  }
  __device__ __forceinline__ T operator()(T a, T b) const {
    if constexpr (sizeof(T) <= 4)
      return static_cast<T>(apply<int32_t>(static_cast<int32_t>(a), static_cast<int32_t>(b)));
    else
      return static_cast<T>(apply<int64_t>(static_cast<int64_t>(a), static_cast<int64_t>(b)));
  }
  // A Python-number divisor is first converted to T with wraparound, as
  // torch does (uint8 by -7 divides by 249).
  __device__ __forceinline__ int64_t scalar_b(int64_t b) const { return static_cast<int64_t>(static_cast<T>(b)); }
  __device__ __forceinline__ T with_scalar(T a, int64_t b) const {
    if constexpr (sizeof(T) <= 4)
      return static_cast<T>(apply<int32_t>(static_cast<int32_t>(a), static_cast<int32_t>(b)));
    else
      return static_cast<T>(apply<int64_t>(static_cast<int64_t>(a), b));
  }
};

// pow.py:10.  Floating tensor ** tensor: the library pow in opmath, one
// rounding.  A Python-number exponent follows torch's CPU dispatch per dtype:
//  * f32 / f64: 0.5 -> sqrt, -0.5 -> 1/sqrt, -1 -> 1/x, 2 -> x*x,
//    3 -> x*x*x, -2 -> 1/(x*x); any other exponent (kept in double) -> pow
//    evaluated in double and rounded once;
//  * bf16: the exponent is rounded to bf16; the same special cases, the
//    products rounded to bf16 after every multiply (x^3 = (x*x)*x,
//    x^-2 = 1/(x*x)); other exponents -> powf, one rounding;
//  * f16: the exponent is rounded to f16, always powf (no special cases, so
//    e.g. (-inf)^0.5 = +inf).
template <typename T, bool F = IsFloat<T>::v>
struct PowF;
template <typename T>
struct PowF<T, true> {
  using C = opmath_t<T>;
  static constexpr bool kF16 = std::is_same<T, _Float16>::value;
  static constexpr bool kBF16 = std::is_same<T, __bf16>::value;
  __device__ __forceinline__ T operator()(T a, T b) const {
    if constexpr (kF16 || kBF16)
      return convert<T>(fast_pow(convert<C>(a), convert<C>(b)));
    else
      return convert<T>(pw(convert<C>(a), convert<C>(b)));
  }
  __device__ __forceinline__ double scalar_b(double b) const {
    if constexpr (kF16 || kBF16)
      return static_cast<double>(convert<float>(convert<T>(b)));
    else
      return b;
  }
  __device__ __forceinline__ T with_scalar(T a, double e) const {
    const C x = convert<C>(a);
    if constexpr (!kF16) {
      if (e == 0.5) return convert<T>(sq(x));
      if (e == -0.5) return convert<T>(C(1) / sq(x));
      if (e == -1.0) return convert<T>(C(1) / x);
      if (e == 2.0) return convert<T>(x * x);
      if (e == 3.0) {
        if constexpr (kBF16) return convert<T>(convert<C>(convert<T>(x * x)) * x);
        return convert<T>(x * x * x);
      }
      if (e == -2.0) {
        if constexpr (kBF16) return convert<T>(C(1) / convert<C>(convert<T>(x * x)));
        return convert<T>(C(1) / (x * x));
      }
    }
    if constexpr (std::is_same<T, float>::value)
      return static_cast<float>(pow(static_cast<double>(x), e));
    else if constexpr (std::is_same<T, double>::value)
      return pow(x, e);
    else
      return convert<T>(fast_pow(x, static_cast<float>(e)));
  }
};
// Integer powers by squaring with wraparound; negative exponents follow
// torch: base 1 -> 1, base -1 -> +-1 by parity, anything else -> 0.
template <typename T>
struct PowF<T, false> {
  __device__ __forceinline__ static T apply(int64_t a, int64_t e) {
    if (e < 0) {
      if (a == 1) return T(1);
      if (a == -1) return static_cast<T>((e & 1) ? -1 : 1);
      return T(0);
    }
    uint64_t base = static_cast<uint64_t>(a), r = 1;
    while (e) {
      if (e & 1) r *= base;
      base *= base;
      e >>= 1;
    }
    return static_cast<T>(r);
  }
  __device__ __forceinline__ T operator()(T a, T b) const {
    return apply(static_cast<int64_t>(a), static_cast<int64_t>(b));
  }
  __device__ __forceinline__ int64_t scalar_b(int64_t b) const { return b; }
  __device__ __forceinline__ T with_scalar(T a, int64_t b) const { return apply(static_cast<int64_t>(a), b); }
};

// {eq,ne,gt,ge,lt,le}.py:9 -> bool.  Floats compare in opmath (exact for the
// 16-bit types); a Python-number operand is first rounded to T (the common
// dtype), integers compare as int64.
template <int OP, typename T>
struct CmpF {
  static constexpr bool kBoolOut = true;
  using K = typename std::conditional<IsFloat<T>::v, opmath_t<T>, int64_t>::type;
  __device__ __forceinline__ static bool apply(K a, K b) {
    if constexpr (OP == NTOPS_CMP_EQ)
      return a == b;
    else if constexpr (OP == NTOPS_CMP_NE)
      return a != b;
    else if constexpr (OP == NTOPS_CMP_GT)
      return a > b;
    else if constexpr (OP == NTOPS_CMP_GE)
      return a >= b;
    else if constexpr (OP == NTOPS_CMP_LT)
      return a < b;
    else
      return a <= b;
  }
  __device__ __forceinline__ bool operator()(T a, T b) const {
    return apply(static_cast<K>(convert<K>(a)), static_cast<K>(convert<K>(b)));
  }
  template <typename S>
  __device__ __forceinline__ K scalar_b(S b) const {
    if constexpr (IsFloat<T>::v)
      return convert<K>(convert<T>(static_cast<double>(b)));
    else
      return static_cast<K>(b);
  }
  __device__ __forceinline__ bool with_scalar(T a, K b) const { return apply(convert<K>(a), b); }
};

// isinf.py:9-11 / isnan.py:9 -> bool (always false for integers)
template <bool NAN_TEST>
struct ClassifyF {
  static constexpr bool kBoolOut = true;
  template <typename T>
  __device__ __forceinline__ bool operator()(T v) const {
    if constexpr (IsFloat<T>::v) {
      using C = opmath_t<T>;
      const C x = convert<C>(v);
      if constexpr (NAN_TEST)
        return x != x;
      else
        return x == C(__builtin_huge_val()) || x == -C(__builtin_huge_val());
    } else {
      return false;
    }
  }
};

// Scalar-operand type of a functor for element type T.
template <typename T>
using scalar_arg_t = typename std::conditional<IsFloat<T>::v, opmath_t<T>, int64_t>::type;

// ------------------------------------------------------------- kernels --
// Result element type of functor F on element type T: bool for functors that
// declare `kBoolOut`, T otherwise.
template <typename F, typename = void>
struct BoolOut : std::false_type {};
template <typename F>
struct BoolOut<F, std::void_t<decltype(F::kBoolOut)>> : std::true_type {};
template <typename F, typename T>
using out1_t = typename std::conditional<BoolOut<F>::value, bool, T>::type;
template <typename F, typename T>
using out2_t = out1_t<F, T>;

// Stores V results of type O with one non-temporal store of V * sizeof(O)
// bytes (the caller guarantees that alignment).
template <typename O, int V>
__device__ __forceinline__ void store_out(O* p, const O (&v)[V]) {
  constexpr int B = V * static_cast<int>(sizeof(O));
  if constexpr (std::is_same<O, bool>::value || B != 16) {
    if constexpr (B == 16) {
      u32x4 w;
      __builtin_memcpy(&w, v, 16);
      __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
    } else if constexpr (B == 8) {
      uint64_t w;
      __builtin_memcpy(&w, v, 8);
      __builtin_nontemporal_store(w, reinterpret_cast<uint64_t*>(p));
    } else if constexpr (B == 4) {
      uint32_t w;
      __builtin_memcpy(&w, v, 4);
      __builtin_nontemporal_store(w, reinterpret_cast<uint32_t*>(p));
    } else if constexpr (B == 2) {
      uint16_t w;
      __builtin_memcpy(&w, v, 2);
      __builtin_nontemporal_store(w, reinterpret_cast<uint16_t*>(p));
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i) p[i] = v[i];
    }
  } else {
    Pack16<O> o;
#pragma unroll
    for (int i = 0; i < V; ++i) o.v[i] = v[i];
    store16_nt(p, o);
  }
}

template <typename T, typename O, typename F>
__global__ __launch_bounds__(kThreads) void k_unary_dense(const T* x, O* y, int64_t npack,
                                                          int64_t n, F f) {
  constexpr int V = Pack16<T>::N;
  const int64_t p = block_id() * kThreads + threadIdx.x;  // blocks_2d grid
  if (p < npack) {
    const Pack16<T> r = load16_nt(x + p * V);
    O o[V];
#pragma unroll
    for (int i = 0; i < V; ++i) o[i] = f(r.v[i]);
    store_out<O, V>(y + p * V, o);
  }
  if (block_id() == 0) {
    const int64_t i = npack * V + threadIdx.x;
    if (threadIdx.x < V && i < n) y[i] = f(x[i]);
  }
}

// One operand broadcast from a single element in memory (a 0-dim GPU
// tensor), the other and the output dense: the element is read once per
// thread, the dense operand in packs.  A_BCAST: the broadcast operand is a.
template <typename T, typename O, typename F, bool A_BCAST>
__global__ __launch_bounds__(kThreads) void k_binary_bcast_dense(const T* a, const T* b, O* y, int64_t npack,
                                                                 int64_t n, F f) {
  constexpr int V = Pack16<T>::N;
  const T* d = A_BCAST ? b : a;
  const T sv = A_BCAST ? a[0] : b[0];
  const int64_t p = block_id() * kThreads + threadIdx.x;  // blocks_2d grid
  if (p < npack) {
    const Pack16<T> r = load16_nt(d + p * V);
    O o[V];
#pragma unroll
    for (int i = 0; i < V; ++i) o[i] = A_BCAST ? f(sv, r.v[i]) : f(r.v[i], sv);
    store_out<O, V>(y + p * V, o);
  }
  if (block_id() == 0) {
    const int64_t i = npack * V + threadIdx.x;
    if (threadIdx.x < V && i < n) y[i] = A_BCAST ? f(sv, d[i]) : f(d[i], sv);
  }
}

// Rows shape: pack p is pack p % ppr of row p / ppr; operand k's row r
// starts at r * s0[k] (a multiple of the pack width).
template <typename T, typename O, typename F, typename I>
__global__ __launch_bounds__(kThreads) void k_unary_rows(const T* x, O* y, I xs0, I ys0, I ppr, I npack, F f) {
  constexpr int V = Pack16<T>::N;
  const I p = static_cast<I>(block_id()) * kThreads + threadIdx.x;  // blocks_2d grid
  if (p >= npack) return;
  const I r = p / ppr, c = (p - r * ppr) * V;
  const Pack16<T> v = load16_nt(x + r * xs0 + c);
  O o[V];
#pragma unroll
  for (int i = 0; i < V; ++i) o[i] = f(v.v[i]);
  store_out<O, V>(y + r * ys0 + c, o);
}

template <typename T, typename O, typename F, typename I>
__global__ __launch_bounds__(kThreads) void k_binary_rows(const T* a, const T* b, O* y, I as0, I bs0, I ys0, I ppr,
                                                          I npack, F f) {
  constexpr int V = Pack16<T>::N;
  const I p = static_cast<I>(block_id()) * kThreads + threadIdx.x;  // blocks_2d grid
  if (p >= npack) return;
  const I r = p / ppr, c = (p - r * ppr) * V;
  const Pack16<T> va = load16_nt(a + r * as0 + c);
  const Pack16<T> vb = load16_nt(b + r * bs0 + c);
  O o[V];
#pragma unroll
  for (int i = 0; i < V; ++i) o[i] = f(va.v[i], vb.v[i]);
  store_out<O, V>(y + r * ys0 + c, o);
}

template <typename T, typename O, typename F, typename S, typename I>
__global__ __launch_bounds__(kThreads) void k_binary_scalar_rows(const T* a, S braw, O* y, I as0, I ys0, I ppr,
                                                                 I npack, F f) {
  constexpr int V = Pack16<T>::N;
  const auto bs = f.scalar_b(braw);
  const I p = static_cast<I>(block_id()) * kThreads + threadIdx.x;  // blocks_2d grid
  if (p >= npack) return;
  const I r = p / ppr, c = (p - r * ppr) * V;
  const Pack16<T> va = load16_nt(a + r * as0 + c);
  O o[V];
#pragma unroll
  for (int i = 0; i < V; ++i) o[i] = f.with_scalar(va.v[i], bs);
  store_out<O, V>(y + r * ys0 + c, o);
}

template <typename T, typename O, typename F, typename I>
__global__ __launch_bounds__(kThreads) void k_unary_strided(KSpace<2, I> sp, const T* x, O* y,
                                                            I n, F f) {
  for (I i = static_cast<I>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<I>(gridDim.x) * kThreads) {
    I off[2];
    strided_offsets<2, I>(sp, i, off);
    y[off[1]] = f(x[off[0]]);
  }
}

template <typename T, typename O, typename F>
__global__ __launch_bounds__(kThreads) void k_binary_dense(const T* a, const T* b, O* y,
                                                           int64_t npack, int64_t n, F f) {
  constexpr int V = Pack16<T>::N;
  const int64_t p = block_id() * kThreads + threadIdx.x;  // blocks_2d grid
  if (p < npack) {
    const Pack16<T> ra = load16_nt(a + p * V);
    const Pack16<T> rb = load16_nt(b + p * V);
    O o[V];
#pragma unroll
    for (int i = 0; i < V; ++i) o[i] = f(ra.v[i], rb.v[i]);
    store_out<O, V>(y + p * V, o);
  }
  if (block_id() == 0) {
    const int64_t i = npack * V + threadIdx.x;
    if (threadIdx.x < V && i < n) y[i] = f(a[i], b[i]);
  }
}

template <typename T, typename O, typename F, typename S>
__global__ __launch_bounds__(kThreads) void k_binary_scalar_dense(const T* a, S braw, O* y,
                                                                  int64_t npack, int64_t n, F f) {
  constexpr int V = Pack16<T>::N;
  const auto bs = f.scalar_b(braw);
  const int64_t p = block_id() * kThreads + threadIdx.x;  // blocks_2d grid
  if (p < npack) {
    const Pack16<T> ra = load16_nt(a + p * V);
    O o[V];
#pragma unroll
    for (int i = 0; i < V; ++i) o[i] = f.with_scalar(ra.v[i], bs);
    store_out<O, V>(y + p * V, o);
  }
  if (block_id() == 0) {
    const int64_t i = npack * V + threadIdx.x;
    if (threadIdx.x < V && i < n) y[i] = f.with_scalar(a[i], bs);
  }
}

template <typename T, typename O, typename F, typename I>
__global__ __launch_bounds__(kThreads) void k_binary_strided(KSpace<3, I> sp, const T* a,
                                                             const T* b, O* y, I n, F f) {
  for (I i = static_cast<I>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<I>(gridDim.x) * kThreads) {
    I off[3];
    strided_offsets<3, I>(sp, i, off);
    y[off[2]] = f(a[off[0]], b[off[1]]);
  }
}

template <typename T, typename O, typename F, typename S, typename I>
__global__ __launch_bounds__(kThreads) void k_binary_scalar_strided(KSpace<2, I> sp, const T* a,
                                                                    S braw, O* y, I n, F f) {
  const auto bs = f.scalar_b(braw);
  for (I i = static_cast<I>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<I>(gridDim.x) * kThreads) {
    I off[2];
    strided_offsets<2, I>(sp, i, off);
    y[off[1]] = f.with_scalar(a[off[0]], bs);
  }
}

// clamp with at least one tensor bound: operands x, lo, hi, y.  A scalar
// bound is passed as a value (its pointer is unused and its strides are 0).
template <typename T, bool LO_T, bool HI_T>
__global__ __launch_bounds__(kThreads) void k_clamp_dense(const T* x, const T* lo, const T* hi,
                                                          T lo_s, T hi_s, T* y, int64_t npack,
                                                          int64_t n) {
  constexpr int V = Pack16<T>::N;
  const int64_t p = block_id() * kThreads + threadIdx.x;  // blocks_2d grid
  if (p < npack) {
    const Pack16<T> rx = load16_nt(x + p * V);
    Pack16<T> rl, rh;
    if constexpr (LO_T) rl = load16_nt(lo + p * V);
    if constexpr (HI_T) rh = load16_nt(hi + p * V);
    T o[V];
#pragma unroll
    for (int i = 0; i < V; ++i) o[i] = clamp_value(rx.v[i], LO_T ? rl.v[i] : lo_s, HI_T ? rh.v[i] : hi_s);
    store_out<T, V>(y + p * V, o);
  }
  if (block_id() == 0) {
    const int64_t i = npack * V + threadIdx.x;
    if (threadIdx.x < V && i < n) y[i] = clamp_value(x[i], LO_T ? lo[i] : lo_s, HI_T ? hi[i] : hi_s);
  }
}

template <typename T, bool LO_T, bool HI_T, typename I>
__global__ __launch_bounds__(kThreads) void k_clamp_strided(KSpace<4, I> sp, const T* x,
                                                            const T* lo, const T* hi, T lo_s,
                                                            T hi_s, T* y, I n) {
  for (I i = static_cast<I>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<I>(gridDim.x) * kThreads) {
    I off[4];
    strided_offsets<4, I>(sp, i, off);
    const T l = LO_T ? lo[off[1]] : lo_s;
    const T h = HI_T ? hi[off[2]] : hi_s;
    y[off[3]] = clamp_value(x[off[0]], l, h);
  }
}

// Mixed operand dtypes with an fp32 result (torch's promotion of, e.g., a
// bf16 tensor and an fp32 tensor, or int32 true division): both operands
// dense, converted to fp32 on load (exact for 16-bit floats; int32 rounds
// to nearest even, as torch's cast does) and combined by the fp32 functor,
// so the result equals casting first and then running the fp32 op.  Eight
// elements per thread: one or two 16-byte loads per operand, two 16-byte
// stores.
template <typename Ta, typename Tb, typename F>
__global__ __launch_bounds__(kThreads) void k_binary_cvt(const Ta* a, const Tb* b, float* y, int64_t n8, int64_t n,
                                                         F f) {
  const int64_t p = block_id() * kThreads + threadIdx.x;  // blocks_2d grid
  auto ld8 = [](auto* src, int64_t i, float (&v)[8]) {
    using S = typename std::remove_const<typename std::remove_pointer<decltype(src)>::type>::type;
    if constexpr (sizeof(S) == 2) {
      const Pack16<S> r = load16_nt(src + i);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = static_cast<float>(r.v[e]);
    } else {
      const Pack16<S> r0 = load16_nt(src + i), r1 = load16_nt(src + i + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = static_cast<float>(r0.v[e]);
        v[e + 4] = static_cast<float>(r1.v[e]);
      }
    }
  };
  if (p < n8) {
    float va[8], vb[8];
    ld8(a, p * 8, va);
    ld8(b, p * 8, vb);
    float o0[4], o1[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o0[e] = f(va[e], vb[e]);
      o1[e] = f(va[e + 4], vb[e + 4]);
    }
    store_out<float, 4>(y + p * 8, o0);
    store_out<float, 4>(y + p * 8 + 4, o1);
  }
  if (block_id() == 0) {
    const int64_t i = n8 * 8 + threadIdx.x;
    if (threadIdx.x < 8 && i < n) y[i] = f(static_cast<float>(a[i]), static_cast<float>(b[i]));
  }
}

template <typename F>
int launch_binary_cvt(const F& f, int a_dtype, int b_dtype, int64_t n, const void* a, const void* b, void* y,
                      hipStream_t st, const char* what) {
  auto cvt_type = [&](int dt, const char* w, auto&& fn) -> int {
    switch (dt) {
      case NTOPS_F32: return fn(float{});
      case NTOPS_F16: return fn(_Float16{});
      case NTOPS_BF16: return fn(__bf16{});
      case NTOPS_I32: return fn(int32_t{});
      default: return set_error(NTOPS_ERR_UNSUPPORTED, "%s: unsupported operand dtype %d", w, dt);
    }
  };
  return cvt_type(a_dtype, what, [&](auto ta) {
    using Ta = decltype(ta);
    return cvt_type(b_dtype, what, [&](auto tb) {
      using Tb = decltype(tb);
      const int64_t n8 = n / 8;
      hipLaunchKernelGGL((k_binary_cvt<Ta, Tb, F>), blocks_2d(ceil_div(n8 > 0 ? n8 : 1, int64_t{kThreads})), dim3(kThreads), 0, st,
                         static_cast<const Ta*>(a), static_cast<const Tb*>(b), static_cast<float*>(y), n8, n, f);
      return check_launch(what);
    });
  });
}

// ------------------------------------------------------------ launchers --
inline int64_t dense_blocks(int64_t npack) {
  return ceil_div(npack > 0 ? npack : 1, static_cast<int64_t>(kThreads));
}
inline unsigned strided_blocks(int64_t n) {
  int64_t b = ceil_div(n, kThreads);
  if (b > 65536) b = 65536;
  return static_cast<unsigned>(b < 1 ? 1 : b);
}

// Whether the rows shape applies: two dims, the inner one unit-stride for
// every operand and a whole number of V-element packs, outer strides
// multiples of V (every row starts on a pack boundary).
template <int NOPS>
bool space_is_rows(const StridedSpace<NOPS>& sp, int V) {
  if (sp.ndim != 2 || sp.shape[1] % V != 0) return false;
  for (int k = 0; k < NOPS; ++k)
    if (sp.stride[k][1] != 1 || sp.stride[k][0] % V != 0) return false;
  return true;
}

// Rows-shape operands: (npack, packs per row, outer strides) with the index
// type the launch uses (32-bit when every offset and pack index fits).
template <int NOPS>
bool rows_fit_int32(const StridedSpace<NOPS>& sp, int64_t n) {
  return fits_int32(sp, n) && n < (int64_t(1) << 31);
}

template <int NOPS>
bool space_is_dense(const StridedSpace<NOPS>& sp) {
  if (sp.ndim == 0) return true;
  if (sp.ndim != 1) return false;
  for (int k = 0; k < NOPS; ++k)
    if (sp.stride[k][0] != 1) return false;
  return true;
}

// Dense-path alignment of an output run of type O written V at a time.
template <typename O, int V>
bool out_aligned(const O* p) {
  constexpr int B = V * static_cast<int>(sizeof(O));
  const uintptr_t a = static_cast<uintptr_t>(B < 16 ? B : 16);
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

template <typename T, typename F>
int launch_unary(const F& f, int ndim, const int64_t* shape, const void* xv, const int64_t* xs,
                 void* yv, const int64_t* ys, hipStream_t st, const char* what) {
  using O = out1_t<F, T>;
  constexpr int V = Pack16<T>::N;
  const int64_t* strides[2] = {xs, ys};
  StridedSpace<2> sp;
  int64_t n = 0;
  if (!build_space<2>(ndim, shape, strides, &sp, &n))
    return set_error(NTOPS_ERR_INVALID, "%s: more than %d non-mergeable dims", what, NTOPS_MAX_DIMS);
  if (n == 0) return NTOPS_OK;
  const T* x = static_cast<const T*>(xv);
  O* y = static_cast<O*>(yv);
  if (space_is_dense(sp) && aligned16(x) && out_aligned<O, V>(y)) {
    const int64_t npack = n / V;
    hipLaunchKernelGGL((k_unary_dense<T, O, F>), blocks_2d(dense_blocks(npack)), dim3(kThreads), 0, st,
                       x, y, npack, n, f);
  } else if (space_is_rows(sp, V) && aligned16(x) && out_aligned<O, V>(y)) {
    const int64_t npack = n / V, ppr = sp.shape[1] / V;
    if (rows_fit_int32(sp, n))
      hipLaunchKernelGGL((k_unary_rows<T, O, F, int32_t>), blocks_2d(dense_blocks(npack)), dim3(kThreads), 0, st, x,
                         y, static_cast<int32_t>(sp.stride[0][0]), static_cast<int32_t>(sp.stride[1][0]),
                         static_cast<int32_t>(ppr), static_cast<int32_t>(npack), f);
    else
      hipLaunchKernelGGL((k_unary_rows<T, O, F, int64_t>), blocks_2d(dense_blocks(npack)), dim3(kThreads), 0, st, x,
                         y, sp.stride[0][0], sp.stride[1][0], ppr, npack, f);
  } else if (fits_int32(sp, n)) {
    hipLaunchKernelGGL((k_unary_strided<T, O, F, int32_t>), dim3(strided_blocks(n)),
                       dim3(kThreads), 0, st, to_kspace<2, int32_t>(sp), x, y,
                       static_cast<int32_t>(n), f);
  } else {
    hipLaunchKernelGGL((k_unary_strided<T, O, F, int64_t>), dim3(strided_blocks(n)),
                       dim3(kThreads), 0, st, to_kspace<2, int64_t>(sp), x, y, n, f);
  }
  return check_launch(what);
}

template <typename T, typename F>
int launch_binary(const F& f, int ndim, const int64_t* shape, const void* av, const int64_t* as,
                  const void* bv, const int64_t* bs, double b_f, int64_t b_i, void* yv,
                  const int64_t* ys, hipStream_t st, const char* what) {
  using O = out2_t<F, T>;
  constexpr int V = Pack16<T>::N;
  const T* a = static_cast<const T*>(av);
  const T* b = static_cast<const T*>(bv);
  O* y = static_cast<O*>(yv);
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
    if (space_is_dense(sp) && aligned16(a) && out_aligned<O, V>(y)) {
      const int64_t npack = n / V;
      hipLaunchKernelGGL((k_binary_scalar_dense<T, O, F, S>), blocks_2d(dense_blocks(npack)),
                         dim3(kThreads), 0, st, a, braw, y, npack, n, f);
    } else if (space_is_rows(sp, V) && aligned16(a) && out_aligned<O, V>(y)) {
      const int64_t npack = n / V, ppr = sp.shape[1] / V;
      if (rows_fit_int32(sp, n))
        hipLaunchKernelGGL((k_binary_scalar_rows<T, O, F, S, int32_t>), blocks_2d(dense_blocks(npack)), dim3(kThreads),
                           0, st, a, braw, y, static_cast<int32_t>(sp.stride[0][0]),
                           static_cast<int32_t>(sp.stride[1][0]), static_cast<int32_t>(ppr),
                           static_cast<int32_t>(npack), f);
      else
        hipLaunchKernelGGL((k_binary_scalar_rows<T, O, F, S, int64_t>), blocks_2d(dense_blocks(npack)), dim3(kThreads),
                           0, st, a, braw, y, sp.stride[0][0], sp.stride[1][0], ppr, npack, f);
    } else if (fits_int32(sp, n)) {
      hipLaunchKernelGGL((k_binary_scalar_strided<T, O, F, S, int32_t>), dim3(strided_blocks(n)),
                         dim3(kThreads), 0, st, to_kspace<2, int32_t>(sp), a, braw, y,
                         static_cast<int32_t>(n), f);
    } else {
      hipLaunchKernelGGL((k_binary_scalar_strided<T, O, F, S, int64_t>), dim3(strided_blocks(n)),
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
  if (space_is_dense(sp) && aligned16(a) && aligned16(b) && out_aligned<O, V>(y)) {
    const int64_t npack = n / V;
    hipLaunchKernelGGL((k_binary_dense<T, O, F>), blocks_2d(dense_blocks(npack)), dim3(kThreads), 0, st,
                       a, b, y, npack, n, f);
  } else if (sp.ndim == 1 && sp.stride[2][0] == 1 && (sp.stride[0][0] == 0) != (sp.stride[1][0] == 0) &&
             (sp.stride[0][0] == 1 || sp.stride[1][0] == 1) && out_aligned<O, V>(y) &&
             aligned16(sp.stride[0][0] == 0 ? b : a)) {
    // one operand a single element broadcast over a dense run
    const int64_t npack = n / V;
    if (sp.stride[0][0] == 0)
      hipLaunchKernelGGL((k_binary_bcast_dense<T, O, F, true>), blocks_2d(dense_blocks(npack)), dim3(kThreads), 0,
                         st, a, b, y, npack, n, f);
    else
      hipLaunchKernelGGL((k_binary_bcast_dense<T, O, F, false>), blocks_2d(dense_blocks(npack)), dim3(kThreads), 0,
                         st, a, b, y, npack, n, f);
  } else if (space_is_rows(sp, V) && aligned16(a) && aligned16(b) && out_aligned<O, V>(y)) {
    const int64_t npack = n / V, ppr = sp.shape[1] / V;
    if (rows_fit_int32(sp, n))
      hipLaunchKernelGGL((k_binary_rows<T, O, F, int32_t>), blocks_2d(dense_blocks(npack)), dim3(kThreads), 0, st, a,
                         b, y, static_cast<int32_t>(sp.stride[0][0]), static_cast<int32_t>(sp.stride[1][0]),
                         static_cast<int32_t>(sp.stride[2][0]), static_cast<int32_t>(ppr),
                         static_cast<int32_t>(npack), f);
    else
      hipLaunchKernelGGL((k_binary_rows<T, O, F, int64_t>), blocks_2d(dense_blocks(npack)), dim3(kThreads), 0, st, a,
                         b, y, sp.stride[0][0], sp.stride[1][0], sp.stride[2][0], ppr, npack, f);
  } else if (fits_int32(sp, n)) {
    hipLaunchKernelGGL((k_binary_strided<T, O, F, int32_t>), dim3(strided_blocks(n)),
                       dim3(kThreads), 0, st, to_kspace<3, int32_t>(sp), a, b, y,
                       static_cast<int32_t>(n), f);
  } else {
    hipLaunchKernelGGL((k_binary_strided<T, O, F, int64_t>), dim3(strided_blocks(n)),
                       dim3(kThreads), 0, st, to_kspace<3, int64_t>(sp), a, b, y, n, f);
  }
  return check_launch(what);
}

// clamp: scalar-only bounds take the unary path; a tensor bound takes the
// four-operand kernel (scalar bounds ride along as values).
template <typename T, bool LO_T, bool HI_T>
int launch_clamp_t(int ndim, const int64_t* shape, const T* x, const int64_t* xs, const T* lo,
                   const int64_t* los, const T* hi, const int64_t* his, T lo_s, T hi_s, T* y,
                   const int64_t* ys, hipStream_t st) {
  int64_t zeros[64] = {0};
  const int64_t* strides[4] = {xs, LO_T ? los : zeros, HI_T ? his : zeros, ys};
  StridedSpace<4> sp;
  int64_t n = 0;
  if (!build_space<4>(ndim, shape, strides, &sp, &n))
    return set_error(NTOPS_ERR_INVALID, "clamp: more than %d non-mergeable dims", NTOPS_MAX_DIMS);
  if (n == 0) return NTOPS_OK;
  bool dense = sp.ndim <= 1 && aligned16(x) && aligned16(y) && (!LO_T || aligned16(lo)) &&
               (!HI_T || aligned16(hi));
  if (sp.ndim == 1)
    dense = dense && sp.stride[0][0] == 1 && sp.stride[3][0] == 1 &&
            (!LO_T || sp.stride[1][0] == 1) && (!HI_T || sp.stride[2][0] == 1);
  if (dense) {
    const int64_t npack = n / Pack16<T>::N;
    hipLaunchKernelGGL((k_clamp_dense<T, LO_T, HI_T>), blocks_2d(dense_blocks(npack)), dim3(kThreads),
                       0, st, x, lo, hi, lo_s, hi_s, y, npack, n);
  } else if (fits_int32(sp, n)) {
    hipLaunchKernelGGL((k_clamp_strided<T, LO_T, HI_T, int32_t>), dim3(strided_blocks(n)),
                       dim3(kThreads), 0, st, to_kspace<4, int32_t>(sp), x, lo, hi, lo_s, hi_s, y,
                       static_cast<int32_t>(n));
  } else {
    hipLaunchKernelGGL((k_clamp_strided<T, LO_T, HI_T, int64_t>), dim3(strided_blocks(n)),
                       dim3(kThreads), 0, st, to_kspace<4, int64_t>(sp), x, lo, hi, lo_s, hi_s, y,
                       n);
  }
  return check_launch("clamp");
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
    case NTOPS_UNARY_SIGMOID:
      return dispatch_float(dtype, "sigmoid", [&](auto tag) {
        using T = decltype(tag);
        return launch_unary<T>(SigmoidF{}, ndim, shape, x, x_strides, y, y_strides, st, "sigmoid");
      });
    case NTOPS_UNARY_TANH:
      return dispatch_float(dtype, "tanh", [&](auto tag) {
        using T = decltype(tag);
        return launch_unary<T>(TanhF{}, ndim, shape, x, x_strides, y, y_strides, st, "tanh");
      });
    case NTOPS_UNARY_RSQRT:
      return dispatch_float(dtype, "rsqrt", [&](auto tag) {
        using T = decltype(tag);
        return launch_unary<T>(RsqrtF{}, ndim, shape, x, x_strides, y, y_strides, st, "rsqrt");
      });
    case NTOPS_UNARY_SIN:
      return dispatch_float(dtype, "sin", [&](auto tag) {
        using T = decltype(tag);
        return launch_unary<T>(SinF{}, ndim, shape, x, x_strides, y, y_strides, st, "sin");
      });
    case NTOPS_UNARY_COS:
      return dispatch_float(dtype, "cos", [&](auto tag) {
        using T = decltype(tag);
        return launch_unary<T>(CosF{}, ndim, shape, x, x_strides, y, y_strides, st, "cos");
      });
    case NTOPS_UNARY_RELU:
    case NTOPS_UNARY_NEG:
    case NTOPS_UNARY_ABS: {
      const char* name = op == NTOPS_UNARY_RELU ? "relu" : op == NTOPS_UNARY_NEG ? "neg" : "abs";
      if (dtype == NTOPS_BOOL) return set_error(NTOPS_ERR_UNSUPPORTED, "%s: bool input is not supported", name);
      return dispatch_all(dtype, name, [&](auto tag) {
        using T = decltype(tag);
        if (op == NTOPS_UNARY_RELU)
          return launch_unary<T>(ReluF{}, ndim, shape, x, x_strides, y, y_strides, st, name);
        if (op == NTOPS_UNARY_NEG)
          return launch_unary<T>(NegF{}, ndim, shape, x, x_strides, y, y_strides, st, name);
        return launch_unary<T>(AbsF{}, ndim, shape, x, x_strides, y, y_strides, st, name);
      });
    }
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
    case NTOPS_BINARY_SUB:
      // sub.py:10; torch evaluates a - alpha * b as add with -alpha.
      if (dtype == NTOPS_BOOL)
        return set_error(NTOPS_ERR_UNSUPPORTED, "sub: subtraction of bool tensors is not supported");
      return dispatch_all(dtype, "sub", [&](auto tag) {
        using T = decltype(tag);
        AddF<T> f;
        if constexpr (IsFloat<T>::v)
          f.alpha = -alpha_f;
        else
          f.alpha = static_cast<int64_t>(static_cast<uint64_t>(0) - static_cast<uint64_t>(alpha_i));
        return launch_binary<T>(f, ndim, shape, a, a_strides, b, b_strides, b_f, b_i, out,
                                out_strides, st, "sub");
      });
    case NTOPS_BINARY_DIV:
      return dispatch_float(dtype, "div", [&](auto tag) {
        using T = decltype(tag);
        return launch_binary<T>(DivF<0, T>{}, ndim, shape, a, a_strides, b, b_strides, b_f, b_i,
                                out, out_strides, st, "div");
      });
    case NTOPS_BINARY_DIV_TRUNC:
    case NTOPS_BINARY_DIV_FLOOR:
      if (dtype == NTOPS_BOOL)
        return set_error(NTOPS_ERR_UNSUPPORTED, "div: rounded division of bool tensors is not supported");
      return dispatch_all(dtype, "div", [&](auto tag) {
        using T = decltype(tag);
        if (op == NTOPS_BINARY_DIV_TRUNC)
          return launch_binary<T>(DivF<1, T>{}, ndim, shape, a, a_strides, b, b_strides, b_f, b_i,
                                  out, out_strides, st, "div(trunc)");
        return launch_binary<T>(DivF<2, T>{}, ndim, shape, a, a_strides, b, b_strides, b_f, b_i,
                                out, out_strides, st, "div(floor)");
      });
    case NTOPS_BINARY_POW:
      if (dtype == NTOPS_BOOL) return set_error(NTOPS_ERR_UNSUPPORTED, "pow: bool tensors are not supported");
      return dispatch_all(dtype, "pow", [&](auto tag) {
        using T = decltype(tag);
        return launch_binary<T>(PowF<T>{}, ndim, shape, a, a_strides, b, b_strides, b_f, b_i, out,
                                out_strides, st, "pow");
      });
    default:
      return set_error(NTOPS_ERR_UNSUPPORTED, "%s: unknown op %d", what, op);
  }
}

extern "C" int ntops_binary_cvt(int op, int a_dtype, int b_dtype, int dtype, int64_t n, const void* a,
                                const void* b, double alpha_f, void* out, void* stream) {
  const char* what = "ntops_binary_cvt";
  if (n < 0) return set_error(NTOPS_ERR_INVALID, "%s: negative size", what);
  if (n == 0) return NTOPS_OK;
  if (a == nullptr || b == nullptr || out == nullptr) return set_error(NTOPS_ERR_INVALID, "%s: null pointer", what);
  if (dtype != NTOPS_F32) return set_error(NTOPS_ERR_UNSUPPORTED, "%s: the result must be fp32", what);
  if (!aligned16(a) || !aligned16(b) || !aligned16(out))
    return set_error(NTOPS_ERR_INVALID, "%s: operands must be 16-byte aligned", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (op) {
    case NTOPS_BINARY_ADD:
    case NTOPS_BINARY_SUB: {
      AddF<float> f;
      f.alpha = op == NTOPS_BINARY_SUB ? -alpha_f : alpha_f;
      return launch_binary_cvt(f, a_dtype, b_dtype, n, a, b, out, st, what);
    }
    case NTOPS_BINARY_MUL:
      return launch_binary_cvt(MulF<float>{}, a_dtype, b_dtype, n, a, b, out, st, what);
    case NTOPS_BINARY_DIV:
      return launch_binary_cvt(DivF<0, float>{}, a_dtype, b_dtype, n, a, b, out, st, what);
    default:
      return set_error(NTOPS_ERR_UNSUPPORTED, "%s: unsupported op %d", what, op);
  }
}

extern "C" int ntops_compare(int op, int dtype, int ndim, const int64_t* shape, const void* a,
                             const int64_t* a_strides, const void* b, const int64_t* b_strides,
                             double b_f, int64_t b_i, void* out, const int64_t* out_strides,
                             void* stream) {
  const char* what = "ntops_compare";
  if (int e = check_common(what, ndim, shape, a, out)) return e;
  if (op < NTOPS_CMP_EQ || op > NTOPS_CMP_LE)
    return set_error(NTOPS_ERR_UNSUPPORTED, "%s: unknown op %d", what, op);
  hipStream_t st = static_cast<hipStream_t>(stream);
  return dispatch_all(dtype, what, [&](auto tag) {
    using T = decltype(tag);
    switch (op) {
      case NTOPS_CMP_EQ:
        return launch_binary<T>(CmpF<NTOPS_CMP_EQ, T>{}, ndim, shape, a, a_strides, b, b_strides, b_f,
                                b_i, out, out_strides, st, "eq");
      case NTOPS_CMP_NE:
        return launch_binary<T>(CmpF<NTOPS_CMP_NE, T>{}, ndim, shape, a, a_strides, b, b_strides, b_f,
                                b_i, out, out_strides, st, "ne");
      case NTOPS_CMP_GT:
        return launch_binary<T>(CmpF<NTOPS_CMP_GT, T>{}, ndim, shape, a, a_strides, b, b_strides, b_f,
                                b_i, out, out_strides, st, "gt");
      case NTOPS_CMP_GE:
        return launch_binary<T>(CmpF<NTOPS_CMP_GE, T>{}, ndim, shape, a, a_strides, b, b_strides, b_f,
                                b_i, out, out_strides, st, "ge");
      case NTOPS_CMP_LT:
        return launch_binary<T>(CmpF<NTOPS_CMP_LT, T>{}, ndim, shape, a, a_strides, b, b_strides, b_f,
                                b_i, out, out_strides, st, "lt");
      default:
        return launch_binary<T>(CmpF<NTOPS_CMP_LE, T>{}, ndim, shape, a, a_strides, b, b_strides, b_f,
                                b_i, out, out_strides, st, "le");
    }
  });
}

extern "C" int ntops_classify(int op, int dtype, int ndim, const int64_t* shape, const void* x,
                              const int64_t* x_strides, void* out, const int64_t* out_strides,
                              void* stream) {
  const char* what = "ntops_classify";
  if (int e = check_common(what, ndim, shape, x, out)) return e;
  if (op != NTOPS_CLASSIFY_ISINF && op != NTOPS_CLASSIFY_ISNAN)
    return set_error(NTOPS_ERR_UNSUPPORTED, "%s: unknown op %d", what, op);
  hipStream_t st = static_cast<hipStream_t>(stream);
  return dispatch_all(dtype, what, [&](auto tag) {
    using T = decltype(tag);
    if (op == NTOPS_CLASSIFY_ISNAN)
      return launch_unary<T>(ClassifyF<true>{}, ndim, shape, x, x_strides, out, out_strides, st, "isnan");
    return launch_unary<T>(ClassifyF<false>{}, ndim, shape, x, x_strides, out, out_strides, st, "isinf");
  });
}

extern "C" int ntops_clamp(int dtype, int ndim, const int64_t* shape, const void* x,
                           const int64_t* x_strides, const void* lo, const int64_t* lo_strides,
                           double lo_f, int64_t lo_i, int has_lo, const void* hi,
                           const int64_t* hi_strides, double hi_f, int64_t hi_i, int has_hi,
                           void* out, const int64_t* out_strides, void* stream) {
  const char* what = "ntops_clamp";
  if (int e = check_common(what, ndim, shape, x, out)) return e;
  if (dtype == NTOPS_BOOL) return set_error(NTOPS_ERR_UNSUPPORTED, "clamp: bool tensors are not supported");
  if (!has_lo && !has_hi) return set_error(NTOPS_ERR_INVALID, "clamp: at least one of min / max is required");
  const bool lo_t = has_lo && lo != nullptr, hi_t = has_hi && hi != nullptr;
  if ((lo_t && lo_strides == nullptr) || (hi_t && hi_strides == nullptr))
    return set_error(NTOPS_ERR_INVALID, "clamp: null bound strides");
  hipStream_t st = static_cast<hipStream_t>(stream);
  return dispatch_all(dtype, "clamp", [&](auto tag) {
    using T = decltype(tag);
    // Scalar bounds rounded to T; an absent bound is the extreme value.
    T lo_s, hi_s;
    if constexpr (IsFloat<T>::v) {
      lo_s = has_lo ? static_cast<T>(lo_f) : static_cast<T>(-__builtin_huge_val());
      hi_s = has_hi ? static_cast<T>(hi_f) : static_cast<T>(__builtin_huge_val());
    } else {
      lo_s = has_lo ? static_cast<T>(lo_i) : std::numeric_limits<T>::lowest();
      hi_s = has_hi ? static_cast<T>(hi_i) : std::numeric_limits<T>::max();
    }
    const T* xp = static_cast<const T*>(x);
    const T* lp = static_cast<const T*>(lo);
    const T* hp = static_cast<const T*>(hi);
    T* yp = static_cast<T*>(out);
    if (lo_t && hi_t)
      return launch_clamp_t<T, true, true>(ndim, shape, xp, x_strides, lp, lo_strides, hp, hi_strides,
                                           lo_s, hi_s, yp, out_strides, st);
    if (lo_t)
      return launch_clamp_t<T, true, false>(ndim, shape, xp, x_strides, lp, lo_strides, hp, hi_strides,
                                            lo_s, hi_s, yp, out_strides, st);
    if (hi_t)
      return launch_clamp_t<T, false, true>(ndim, shape, xp, x_strides, lp, lo_strides, hp, hi_strides,
                                            lo_s, hi_s, yp, out_strides, st);
    return launch_unary<T>(ClampSF<T>{lo_s, hi_s}, ndim, shape, x, x_strides, out, out_strides, st,
                           "clamp");
  });
}
