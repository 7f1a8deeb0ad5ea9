// Shared device and host helpers for the gfx950 kernels of ntops_amd.
//
// Element types are the compiler's native ones (__bf16, _Float16, ...) so
// that conversions lower to gfx950's hardware converts (v_cvt_pk_bf16_f32
// rounds to nearest even, like torch's c10::BFloat16).  All arithmetic on
// 16-bit floats is done in fp32 ("opmath"), fp64 stays fp64.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/ntops_amd.h"

namespace ntops {

// ---------------------------------------------------------------- errors --
// Records `msg` as this thread's last error and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Converts the HIP runtime's sticky launch error (if any) into a status.
int check_launch(const char* what);
// Records the name of the kernel this thread is about to launch (returned by
// ntops_last_kernel(), so tests can assert which path served a call).
void note_kernel(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
// Number of CUs of the current device (queried once per device; 256 if the
// query fails).
int cu_count_cached();

// ------------------------------------------------------------ wave size --
constexpr int kWave = 64;

// ------------------------------------------------------------ type maps --
template <int D> struct DTypeOf;
template <> struct DTypeOf<NTOPS_F32> { using T = float; };
template <> struct DTypeOf<NTOPS_F16> { using T = _Float16; };
template <> struct DTypeOf<NTOPS_BF16> { using T = __bf16; };
template <> struct DTypeOf<NTOPS_F64> { using T = double; };
template <> struct DTypeOf<NTOPS_BOOL> { using T = bool; };
template <> struct DTypeOf<NTOPS_U8> { using T = uint8_t; };
template <> struct DTypeOf<NTOPS_I8> { using T = int8_t; };
template <> struct DTypeOf<NTOPS_I16> { using T = int16_t; };
template <> struct DTypeOf<NTOPS_I32> { using T = int32_t; };
template <> struct DTypeOf<NTOPS_I64> { using T = int64_t; };

inline int dtype_size(int dt) {
  switch (dt) {
    case NTOPS_F32: return 4;
    case NTOPS_F16: return 2;
    case NTOPS_BF16: return 2;
    case NTOPS_F64: return 8;
    case NTOPS_BOOL: return 1;
    case NTOPS_U8: return 1;
    case NTOPS_I8: return 1;
    case NTOPS_I16: return 2;
    case NTOPS_I32: return 4;
    case NTOPS_I64: return 8;
    default: return 0;
  }
}
inline bool dtype_is_float(int dt) {
  return dt == NTOPS_F32 || dt == NTOPS_F16 || dt == NTOPS_BF16 || dt == NTOPS_F64;
}

// Compute ("opmath") type: fp32 for 16-bit floats, identity otherwise.
template <typename T> struct OpMath { using T_ = T; };
template <> struct OpMath<_Float16> { using T_ = float; };
template <> struct OpMath<__bf16> { using T_ = float; };
template <typename T> using opmath_t = typename OpMath<T>::T_;

template <typename T> struct IsFloat { static constexpr bool v = false; };
template <> struct IsFloat<float> { static constexpr bool v = true; };
template <> struct IsFloat<double> { static constexpr bool v = true; };
template <> struct IsFloat<_Float16> { static constexpr bool v = true; };
template <> struct IsFloat<__bf16> { static constexpr bool v = true; };

// Conversion between any two element types with torch's rules: float ->
// integer truncates toward zero, anything -> bool is (v != 0), 16-bit float
// targets round to nearest even.
template <typename D, typename S>
__device__ __forceinline__ D convert(S v) {
  if constexpr (std::is_same<D, S>::value) {
    return v;
  } else if constexpr (std::is_same<D, bool>::value) {
    if constexpr (std::is_same<S, __bf16>::value || std::is_same<S, _Float16>::value)
      return static_cast<float>(v) != 0.0f;
    else
      return v != S(0);
  } else if constexpr (std::is_same<S, __bf16>::value || std::is_same<S, _Float16>::value) {
    // via fp32 (exact) then to the destination
    return static_cast<D>(static_cast<float>(v));
  } else if constexpr (std::is_same<D, __bf16>::value || std::is_same<D, _Float16>::value) {
    if constexpr (std::is_same<S, double>::value) {
      // torch converts double -> bf16/half through float as well
      return static_cast<D>(static_cast<float>(v));
    } else if constexpr (IsFloat<S>::v) {
      return static_cast<D>(v);
    } else {
      return static_cast<D>(static_cast<float>(v));
    }
  } else {
    return static_cast<D>(v);
  }
}

// ------------------------------------------- uncontracted fp32 arithmetic --
// hipcc contracts a*b+c into an fma by default.  These keep each operation
// separately rounded (the contract flag is off on the emitted instruction),
// for the places that must reproduce torch's separately rounded CPU code.
__device__ __forceinline__ float mul_nc(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_nc(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ __forceinline__ float sub_nc(float a, float b) {
#pragma clang fp contract(off)
  return a - b;
}

// ------------------------------------------------------- 16-byte vectors --
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct alignas(16) Pack16 {
  static constexpr int N = 16 / sizeof(T);
  T v[N];
};

template <typename T>
__device__ __forceinline__ Pack16<T> load16(const T* p) {
  u32x4 r = *reinterpret_cast<const u32x4*>(p);
  return __builtin_bit_cast(Pack16<T>, r);
}
template <typename T>
__device__ __forceinline__ Pack16<T> load16_nt(const T* p) {
  u32x4 r = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return __builtin_bit_cast(Pack16<T>, r);
}
template <typename T>
__device__ __forceinline__ void store16(T* p, const Pack16<T>& v) {
  *reinterpret_cast<u32x4*>(p) = __builtin_bit_cast(u32x4, v);
}
template <typename T>
__device__ __forceinline__ void store16_nt(T* p, const Pack16<T>& v) {
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), reinterpret_cast<u32x4*>(p));
}

// Buffer resource (V#) over `bytes` bytes at the wave-uniform address
// `base` (raw, stride 0).  Buffer loads at byte offsets at or past `bytes`
// return zeros and buffer stores there are dropped, so a ragged tail or a
// row past the end needs no branch around its accesses -- and without such
// branches the compiler can count outstanding memory operations exactly
// (a load issued on a maybe-skipped path forces a full vmcnt(0) wait).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}
// The same resource with its address and size read from the first active
// lane.  Where the compiler cannot prove `base` / `bytes` uniform it keeps the
// resource in VGPRs and wraps every buffer access in a readfirstlane loop (a
// branch per load, which also splits the schedule around it); this form tells
// it they are uniform.  Only for values that really are wave-uniform.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc_uniform(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo), 0,
                                           static_cast<int>(__builtin_amdgcn_readfirstlane(bytes)), 0x00020000);
}
constexpr int kBufNT = 2;  // cache-policy bit: nontemporal (streamed once)
template <typename T>
__device__ __forceinline__ Pack16<T> buffer_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(Pack16<T>, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kBufNT));
}
template <typename T>
__device__ __forceinline__ void buffer_store16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off, const Pack16<T>& v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, kBufNT);
}

// ------------------------------------------------------- wave reductions --
// All-reduce over the 64 lanes of a wavefront; every lane gets the result.
// float: within each 16-lane row the partners arrive through DPP operand
// swizzles (quad_perm xor 1, quad_perm xor 2, half-row mirror, row mirror:
// no LDS round trip, a few cycles each); the four row results are then read
// with v_readlane and combined as op(op(r0, r16), op(r32, r48)).  After the
// two quad steps every lane of a quad holds the same value, so the mirrors
// pair exactly the lanes a xor-4 / xor-8 butterfly pairs: for a commutative
// op the result is bit-identical to the 64-lane xor butterfly.  All 64 lanes
// must be active (every caller reduces in wave-uniform control flow).
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <- lane 7-i within 8
constexpr int kDppMirror = 0x140;      // lane i <- lane 15-i within 16

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_read(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// op(a, b) -> combined value; commutative.
template <typename Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
  v = op(v, dpp_mov<kDppXor1>(v));
  v = op(v, dpp_mov<kDppXor2>(v));
  v = op(v, dpp_mov<kDppHalfMirror>(v));
  v = op(v, dpp_mov<kDppMirror>(v));
  return op(op(lane_read(v, 0), lane_read(v, 16)), op(lane_read(v, 32), lane_read(v, 48)));
}

// Two-value form: merge(a, b, a2, b2) folds (a2, b2) into (a, b); commutative.
template <typename Merge>
__device__ __forceinline__ void wave_reduce2(float& a, float& b, Merge merge) {
  merge(a, b, dpp_mov<kDppXor1>(a), dpp_mov<kDppXor1>(b));
  merge(a, b, dpp_mov<kDppXor2>(a), dpp_mov<kDppXor2>(b));
  merge(a, b, dpp_mov<kDppHalfMirror>(a), dpp_mov<kDppHalfMirror>(b));
  merge(a, b, dpp_mov<kDppMirror>(a), dpp_mov<kDppMirror>(b));
  float a0 = lane_read(a, 0), b0 = lane_read(b, 0);
  float a2 = lane_read(a, 32), b2 = lane_read(b, 32);
  merge(a0, b0, lane_read(a, 16), lane_read(b, 16));
  merge(a2, b2, lane_read(a, 48), lane_read(b, 48));
  merge(a0, b0, a2, b2);
  a = a0;
  b = b0;
}

__device__ __forceinline__ float wave_sum(float v) {
  return wave_reduce(v, [](float x, float y) { return x + y; });
}
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) v += __shfl_xor(v, m, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  return wave_reduce(v, [](float x, float y) { return fmaxf(x, y); });
}
__device__ __forceinline__ double wave_max(double v) {
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) v = fmax(v, __shfl_xor(v, m, kWave));
  return v;
}

// ------------------------------------------------------ strided indexing --
// Index space of up to NTOPS_MAX_DIMS dims with per-operand element strides.
// Operands are addressed by decomposing a linear index (row-major over
// `shape`) into coordinates.
template <int NOPS>
struct StridedSpace {
  int ndim;
  int64_t shape[NTOPS_MAX_DIMS];
  int64_t stride[NOPS][NTOPS_MAX_DIMS];
};

// Same space with index type I (int32_t when every offset fits), passed to
// kernels by value.
template <int NOPS, typename I>
struct KSpace {
  int ndim;
  I shape[NTOPS_MAX_DIMS];
  I stride[NOPS][NTOPS_MAX_DIMS];
};

template <int NOPS, typename I>
KSpace<NOPS, I> to_kspace(const StridedSpace<NOPS>& sp) {
  KSpace<NOPS, I> k{};
  k.ndim = sp.ndim;
  for (int d = 0; d < sp.ndim; ++d) {
    k.shape[d] = static_cast<I>(sp.shape[d]);
    for (int o = 0; o < NOPS; ++o) k.stride[o][d] = static_cast<I>(sp.stride[o][d]);
  }
  return k;
}

// True when numel and every reachable offset (positive or negative) of the
// space fit in int32.
template <int NOPS>
bool fits_int32(const StridedSpace<NOPS>& sp, int64_t numel) {
  if (numel >= (int64_t(1) << 31)) return false;
  for (int o = 0; o < NOPS; ++o) {
    int64_t span = 0;
    for (int d = 0; d < sp.ndim; ++d) {
      int64_t s = sp.stride[o][d];
      span += (s < 0 ? -s : s) * (sp.shape[d] - 1);
    }
    if (span >= (int64_t(1) << 31)) return false;
  }
  return true;
}

template <int NOPS, typename I>
__device__ __forceinline__ void strided_offsets(const KSpace<NOPS, I>& sp, I linear,
                                                I (&off)[NOPS]) {
#pragma unroll
  for (int k = 0; k < NOPS; ++k) off[k] = 0;
  for (int d = sp.ndim - 1; d >= 0; --d) {
    const I n = sp.shape[d];
    const I q = linear / n;
    const I c = linear - q * n;
    linear = q;
#pragma unroll
    for (int k = 0; k < NOPS; ++k) off[k] += c * sp.stride[k][d];
  }
}

// Host: drops size-1 dims, orders the rest by the last operand's (the
// output's) strides, largest outermost -- an elementwise result does not
// depend on the order in which elements are visited, and this order makes a
// permuted dense layout (a transposed view and the empty_like output that
// follows it) one dense run -- then merges adjacent dims that are
// contiguous with respect to every operand.  Returns false if ndim exceeds
// the limit after merging.  numel is written to *numel.
template <int NOPS>
bool build_space(int ndim, const int64_t* shape, const int64_t* const strides[NOPS],
                 StridedSpace<NOPS>* sp, int64_t* numel) {
  int64_t shp[64];
  int64_t st[NOPS][64];
  int n = 0;
  int64_t total = 1;
  for (int d = 0; d < ndim; ++d) {
    total *= shape[d];
    if (shape[d] == 1) continue;
    shp[n] = shape[d];
    for (int k = 0; k < NOPS; ++k) st[k][n] = strides[k][d];
    ++n;
  }
  *numel = total;
  // stable insertion sort by |output stride|, descending
  auto key = [](int64_t v) { return v < 0 ? -v : v; };
  for (int i = 1; i < n; ++i) {
    for (int j = i; j > 0 && key(st[NOPS - 1][j - 1]) < key(st[NOPS - 1][j]); --j) {
      const int64_t t = shp[j];
      shp[j] = shp[j - 1];
      shp[j - 1] = t;
      for (int k = 0; k < NOPS; ++k) {
        const int64_t u = st[k][j];
        st[k][j] = st[k][j - 1];
        st[k][j - 1] = u;
      }
    }
  }
  // merge from the innermost side
  int m = 0;
  int64_t oshp[64];
  int64_t ost[NOPS][64];
  for (int d = 0; d < n; ++d) {
    if (m > 0) {
      bool ok = true;
      for (int k = 0; k < NOPS; ++k)
        if (ost[k][m - 1] != st[k][d] * shp[d]) ok = false;
      if (ok) {
        oshp[m - 1] *= shp[d];
        for (int k = 0; k < NOPS; ++k) ost[k][m - 1] = st[k][d];
        continue;
      }
    }
    oshp[m] = shp[d];
    for (int k = 0; k < NOPS; ++k) ost[k][m] = st[k][d];
    ++m;
  }
  if (m > NTOPS_MAX_DIMS) return false;
  sp->ndim = m;
  for (int d = 0; d < m; ++d) {
    sp->shape[d] = oshp[d];
    for (int k = 0; k < NOPS; ++k) sp->stride[k][d] = ost[k][d];
  }
  return true;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
// n > 0 blocks as an x * y grid (x <= 65536): a dispatch counts each
// dimension's work-items in 32 bits, so a one-dimensional grid of 256-thread
// blocks would end at 2^24 blocks.  Kernels index blocks with block_id() and
// ignore ids >= n (the tail of the last grid row).
inline dim3 blocks_2d(int64_t n) {
  const int64_t x = n < 65536 ? n : 65536;
  return dim3(static_cast<unsigned>(x), static_cast<unsigned>((n + x - 1) / x));
}
__device__ __forceinline__ int64_t block_id() { return blockIdx.x + static_cast<int64_t>(blockIdx.y) * gridDim.x; }

}  // namespace ntops
