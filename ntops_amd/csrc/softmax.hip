// softmax over one axis, viewed as (outer, dim_size, inner).
//
// Math follows kernels/softmax.py:9-29 (an online max / sum of
// exp(x - max), then exp(x - max) / sum) with torch's accumulation rule,
// which the build keeps: max and sum in fp32 (fp64 for fp64 output) and a
// single rounding of each output to the output dtype.  The input is first rounded to
// the output dtype, as torch does for softmax(..., dtype=).  A row that is all
// -inf yields NaN (exp(-inf - -inf) = NaN), like torch.
//
// inner == 1 (softmax over a contiguous last axis):
//   vector path -- row held in VGPRs (rowcommon.h), one HBM read and one HBM
//   write per element;
//   looped path -- any stride or dtype pair, one 256-thread block per row.
// inner > 1: a 256-thread block takes CW adjacent (outer, inner) columns
//   and splits dim_size over 256 / CW row slices (adjacent threads touch
//   adjacent inner elements, so every pass is coalesced); the slices' maxima
//   and sums combine through LDS in a fixed order, CW chosen so that the
//   grid has at least two blocks per CU where it can.
#include "dispatch.h"
#include "rowcommon.h"
#include "rowwide.h"

namespace ntops {
namespace {

__device__ __forceinline__ float ex(float v) { return expf(v); }
__device__ __forceinline__ double ex(double v) { return exp(v); }

template <typename C>
__device__ __forceinline__ C cmax(C a, C b) {
  return (a > b || a != a) ? a : b;
}

// exp(d) for the register-resident path: fp32 uses the hardware base-2
// exponential, exp(d) = 2^(d * log2 e) (v_exp_f32), keeping the kernel under
// the HBM bound (an accurate expf costs ~3x the VALU work per element, which
// at 4 bytes per bf16 element is the same order as the memory time).  The
// argument is <= 0 here, so the product's rounding changes the result by
// less than |d| * 2^-24 relative.  fp64 keeps the accurate exp.
__device__ __forceinline__ float row_exp(float d) {
  return __builtin_amdgcn_exp2f(d * 1.44269504088896340736f);
}
__device__ __forceinline__ double row_exp(double d) { return exp(d); }

// Merges the (max, sum of exp(x - max)) summary of another part of the row
// into (m, s).  Parts whose max is -inf (no finite element) contribute 0; a
// NaN max propagates.
template <typename C>
__device__ __forceinline__ void merge_max_sum(C& m, C& s, C m2, C s2) {
  const C ninf = -__builtin_huge_val();
  const C mn = cmax(m, m2);
  const C ta = m == ninf ? C(0) : s * row_exp(m - mn);
  const C tb = m2 == ninf ? C(0) : s2 * row_exp(m2 - mn);
  m = mn;
  s = ta + tb;
}

// One pass over the register-resident row: each lane reduces its own
// elements to (max, sum of exp(x - max)), the lanes' summaries are merged
// (64-lane butterfly, then one LDS exchange across the row's waves), and
// every output is exp(x - lane max) * (exp(lane max - row max) / row sum).
template <typename T, typename C, int CHUNKS, int WPR>
__global__ __launch_bounds__(RowShape<WPR>::kThreads) void k_softmax_vec(
    const T* __restrict__ x, int64_t xs, T* __restrict__ y, int64_t ys, int64_t rows, int cols) {
  constexpr int V = Pack16<T>::N;
  constexpr int RPB = RowShape<WPR>::kRowsPerBlock;
  __shared__ C red_m[RPB * WPR];
  __shared__ C red_s[RPB * WPR];
  // Vector-register row position and per-lane branches around the loads:
  // on MI355X this measured ~3% faster for bf16 rows of 2048 than the
  // scalar position with branch-free buffer loads used by the norms.
  const RowPos p = row_pos<WPR, false>();
  const int64_t row = block_id() * RPB + p.row_in_block;
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
  // lane summary
  C ml = ninf;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
    for (int i = 0; i < V; ++i) ml = cmax(ml, v[c][i]);
  C sl = 0;
  const bool lane_empty = ml == ninf;  // every element -inf (or padding)
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
    for (int i = 0; i < V; ++i) {
      v[c][i] = lane_empty ? C(0) : row_exp(v[c][i] - ml);
      sl += v[c][i];  // padding is -inf, so it adds exp(-inf) = 0
    }
  // row summary
  C m = ml, s = sl;
  if constexpr (sizeof(C) == 4) {
    wave_reduce2(m, s, [](C& a, C& b, C a2, C b2) { merge_max_sum(a, b, a2, b2); });
  } else {
#pragma unroll
    for (int k = 1; k < 64; k <<= 1) merge_max_sum(m, s, __shfl_xor(m, k, 64), __shfl_xor(s, k, 64));
  }
  if constexpr (WPR > 1) {
    if (p.lane == 0) {
      red_m[p.row_in_block * WPR + p.wave_in_row] = m;
      red_s[p.row_in_block * WPR + p.wave_in_row] = s;
    }
    __syncthreads();
    m = red_m[p.row_in_block * WPR];
    s = red_s[p.row_in_block * WPR];
#pragma unroll
    for (int w = 1; w < WPR; ++w)
      merge_max_sum(m, s, red_m[p.row_in_block * WPR + w], red_s[p.row_in_block * WPR + w]);
  }
  if (!row_ok) return;
  const C f = (lane_empty ? C(0) : row_exp(ml - m)) / s;
  T* yr = y + row * ys;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int pk = pack_of<WPR>(p, c);
    if (pk < npk) {
      Pack16<T> o;
#pragma unroll
      for (int i = 0; i < V; ++i) o.v[i] = static_cast<T>(v[c][i] * f);
      store16_nt(yr + pk * V, o);
    }
  }
}

// Rows of more than 8192 packs (rowwide.h): one block per CU walking rows,
// each read once into VGPRs and LDS (the next one loading during the output
// pass of the current one); two passes over it there -- (max, sum of
// exp(x - max)) merged pack by pack as the packs land, then the outputs
// exp(x - max) / sum (the exponential evaluated again rather than kept: the
// registers hold the row itself).
template <typename T>
__global__ __launch_bounds__(kWideThreads) void k_softmax_wide(const T* __restrict__ x, int64_t xs,
                                                               T* __restrict__ y, int64_t ys, int64_t rows,
                                                               int cols) {
  constexpr int V = Pack16<T>::N;
  __shared__ float red_m[kWideWaves], red_s[kWideWaves];
  extern __shared__ __attribute__((aligned(16))) char wsm[];
  int64_t row = blockIdx.x;
  if (row >= rows) return;
  const int npk = cols / V;
  const float ninf = -__builtin_huge_valf();
  // this thread's (max, sum of exp(x - max)) of a row, merged pack by pack
  // as the packs land (every register pack of a wide row lies inside it)
  float mx = ninf, sx = 0.f;
  auto visit = [&](const Pack16<T>& v) {
    float f[V];
    float pm = ninf;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      f[i] = static_cast<float>(v.v[i]);
      pm = cmax(pm, f[i]);
    }
    float ps = 0.f;
#pragma unroll
    for (int i = 0; i < V; ++i) ps += row_exp(f[i] - pm);
    merge_max_sum(mx, sx, pm, ps);
  };
  WideRow<T> d;
  wide_load(d, x + row * xs, npk, wsm, visit);
  for (; row < rows; row += gridDim.x) {
    // row summary: the wave's lanes, then the block's waves
    float m = mx, s = sx;
    wave_reduce2(m, s, [](float& a, float& b, float a2, float b2) { merge_max_sum(a, b, a2, b2); });
    __syncthreads();  // the previous row's summaries have been read
    if ((threadIdx.x & 63) == 0) {
      red_m[threadIdx.x >> 6] = m;
      red_s[threadIdx.x >> 6] = s;
    }
    __syncthreads();
    m = red_m[0];
    s = red_s[0];
#pragma unroll
    for (int w = 1; w < kWideWaves; ++w) merge_max_sum(m, s, red_m[w], red_s[w]);
    mx = ninf;
    sx = 0.f;
    wide_launder(d);
    const float inv = 1.0f / s;
    // 16-bit outputs: exp(x - m) / s = 2^(x log2 e - (m log2 e + log2 s)), one
    // fma and one exponential per element (the fp32 result's relative error,
    // ~|x - m| * 2^-23, is far below the output's rounding)
    constexpr float kLog2e = 1.44269504088896340736f;
    const float c = fmaf(m, kLog2e, __builtin_amdgcn_logf(s));
    const __amdgpu_buffer_rsrc_t out = buffer_rsrc(y + row * ys, npk * 16u);
    struct None {};
    auto fetch = [](int) { return None{}; };
    auto emit = [&](const Pack16<T>& v, int pk, None) {
      Pack16<T> o;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float xv = static_cast<float>(v.v[i]);
        if constexpr (sizeof(T) == 2)
          o.v[i] = static_cast<T>(__builtin_amdgcn_exp2f(fmaf(xv, kLog2e, -c)));
        else
          o.v[i] = static_cast<T>(row_exp(xv - m) * inv);
      }
      buffer_store16_nt(out, pk * 16u, o);
    };
    const bool more = row + gridDim.x < rows;
    wide_emit_and_load<0>(d, more, x + (more ? row + gridDim.x : row) * xs, npk, fetch, emit, visit);
  }
}

// One block per row, any element stride, input converted to the output dtype
// first.
template <typename Ti, typename To, typename C>
__global__ __launch_bounds__(256) void k_softmax_loop(const Ti* x, int64_t xs0, int64_t xs1,
                                                      To* y, int64_t ys0, int64_t ys1,
                                                      int64_t rows, int64_t cols) {
  __shared__ C red[4];
  const int64_t row = block_id();
  if (row >= rows) return;  // the tail of a 2-D grid (the whole block)
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

// The same over unit-stride rows of any width and alignment when input and
// output share a dtype: each row as a scalar head up to its first 16-byte
// boundary, 16-byte packs, a scalar tail (a vocabulary-wide row of 50257
// bf16 elements is 16-byte aligned on at most one row in eight); the output
// in packs too when its row has the input row's alignment (contiguous
// tensors), else element by element.
template <typename T, typename C>
__global__ __launch_bounds__(256) void k_softmax_loop_v(const T* x, int64_t xs0, T* y, int64_t ys0,
                                                        int64_t rows, int64_t cols) {
  constexpr int V = Pack16<T>::N;
  __shared__ C red[4];
  const int64_t row = block_id();
  if (row >= rows) return;  // the tail of a 2-D grid (the whole block)
  const T* xr = x + row * xs0;
  T* yr = y + row * ys0;
  const int mis = static_cast<int>((reinterpret_cast<uintptr_t>(xr) & 15u) / sizeof(T));
  const int64_t head = mis ? (V - mis < cols ? V - mis : cols) : 0;
  const int64_t packs = (cols - head) / V;
  const int64_t tail = head + packs * V;
  const T* xb = xr + head;  // 16-byte aligned
  const int t = threadIdx.x;
  C m = -__builtin_huge_val();
  if (t < head) m = static_cast<C>(xr[t]);
  for (int64_t p = t; p < packs; p += 256) {
    const Pack16<T> v = load16(xb + p * V);
#pragma unroll
    for (int e = 0; e < V; ++e) m = cmax(m, static_cast<C>(v.v[e]));
  }
  for (int64_t j = tail + t; j < cols; j += 256) m = cmax(m, static_cast<C>(xr[j]));
  m = block_max256(m, red);
  C s = 0;
  if (t < head) s = ex(static_cast<C>(xr[t]) - m);
  for (int64_t p = t; p < packs; p += 256) {
    const Pack16<T> v = load16(xb + p * V);
#pragma unroll
    for (int e = 0; e < V; ++e) s += ex(static_cast<C>(v.v[e]) - m);
  }
  for (int64_t j = tail + t; j < cols; j += 256) s += ex(static_cast<C>(xr[j]) - m);
  s = block_sum256(s, red);
  const C inv = C(1) / s;
  if (t < head) yr[t] = convert<T>(ex(static_cast<C>(xr[t]) - m) * inv);
  const bool packed_out = ((reinterpret_cast<uintptr_t>(yr) ^ reinterpret_cast<uintptr_t>(xr)) & 15u) == 0;
  for (int64_t p = t; p < packs; p += 256) {
    const Pack16<T> v = load16(xb + p * V);
    Pack16<T> o;
#pragma unroll
    for (int e = 0; e < V; ++e) o.v[e] = convert<T>(ex(static_cast<C>(v.v[e]) - m) * inv);
    if (packed_out) {
      store16(yr + head + p * V, o);
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e) yr[head + p * V + e] = o.v[e];
    }
  }
  for (int64_t j = tail + t; j < cols; j += 256) yr[j] = convert<T>(ex(static_cast<C>(xr[j]) - m) * inv);
}

// Block = CW columns x (256 / CW) row slices; block b takes columns
// [b % tiles_per_outer * CW, + CW) of outer index b / tiles_per_outer.  Each
// pass (max, sum of exp(x - max), outputs) walks the slice's rows; the
// per-slice maxima and sums are combined in slice order through LDS.
template <typename Ti, typename To, typename C, int CW>
__global__ __launch_bounds__(256) void k_softmax_col(const Ti* x, int64_t xs0, int64_t xs1,
                                                     int64_t xs2, To* y, int64_t ys0,
                                                     int64_t ys1, int64_t ys2, int64_t outer,
                                                     int64_t dim, int64_t inner) {
  constexpr int RS = 256 / CW;
  __shared__ C red[RS][CW];
  const int64_t tiles = (inner + CW - 1) / CW;
  const int64_t b = block_id();  // blocks_2d grid
  if (b >= outer * tiles) return;  // the tail of the grid (the whole block)
  const int64_t o = b / tiles;
  const int tx = threadIdx.x % CW, ty = threadIdx.x / CW;
  const int64_t in = (b - o * tiles) * CW + tx;
  const bool ok = in < inner;
  const Ti* xc = x + o * xs0 + (ok ? in : 0) * xs2;
  To* yc = y + o * ys0 + (ok ? in : 0) * ys2;
  auto val = [&](int64_t j) { return static_cast<C>(convert<To>(xc[j * xs1])); };
  C m = -__builtin_huge_val();
  if (ok)
    for (int64_t j = ty; j < dim; j += RS) m = cmax(m, val(j));
  red[ty][tx] = m;
  __syncthreads();
  m = red[0][tx];
#pragma unroll
  for (int k = 1; k < RS; ++k) m = cmax(m, red[k][tx]);
  __syncthreads();
  C s = 0;
  if (ok)
    for (int64_t j = ty; j < dim; j += RS) s += ex(val(j) - m);
  red[ty][tx] = s;
  __syncthreads();
  s = red[0][tx];
#pragma unroll
  for (int k = 1; k < RS; ++k) s += red[k][tx];
  if (!ok) return;
  const C inv = C(1) / s;
  for (int64_t j = ty; j < dim; j += RS) yc[j * ys1] = convert<To>(ex(val(j) - m) * inv);
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
    hipLaunchKernelGGL((k_softmax_vec<To, C, CH, WP>), blocks_2d(ceil_div(outer, RPB)),        \
                       dim3(RowShape<WP>::kThreads), 0, st, x, xs[0], y, ys[0], outer,         \
                       static_cast<int>(dim));                                                 \
    return check_launch("softmax");                                                            \
  }
        NTOPS_ROW_CASES(NTOPS_SM_CASE)
#undef NTOPS_SM_CASE
      }
      if constexpr (sizeof(C) == 4) {
        if (xs[1] == 1 && ys[1] == 1 && dim % V == 0 && xs[0] % V == 0 && ys[0] % V == 0 && aligned16(x) &&
            aligned16(y) && wide_row_fits(dim / V) && outer <= 0x7fffffffLL) {
          static bool lds_set = false;
          if (int e = wide_lds_attr(k_softmax_wide<To>, lds_set)) return e;
          hipLaunchKernelGGL((k_softmax_wide<To>), dim3(wide_grid(outer)), dim3(kWideThreads), wide_lds_bytes(dim / V), st,
                             x, xs[0], y, ys[0], outer, static_cast<int>(dim));
          return check_launch("softmax");
        }
      }
      if (xs[1] == 1 && ys[1] == 1 && outer <= 0x7fffffffLL) {
        hipLaunchKernelGGL((k_softmax_loop_v<To, C>), blocks_2d(outer), dim3(256), 0, st, x, xs[0], y, ys[0],
                           outer, dim);
        return check_launch("softmax");
      }
    }
    if (outer > 0x7fffffffLL) return set_error(NTOPS_ERR_UNSUPPORTED, "softmax: too many rows");
    hipLaunchKernelGGL((k_softmax_loop<Ti, To, C>), blocks_2d(outer), dim3(256), 0, st, x, xs[0], xs[1],
                       y, ys[0], ys[1], outer, dim);
    return check_launch("softmax");
  }
  // the widest column tile (coalescing) that still gives two blocks per CU
  const int64_t want = 2 * static_cast<int64_t>(cu_count_cached());
  auto blocks_for = [&](int cw) { return outer * ((inner + cw - 1) / cw); };
  const int cw = blocks_for(64) >= want ? 64 : blocks_for(32) >= want ? 32 : blocks_for(16) >= want ? 16 : 8;
#define NTOPS_SM_COL(CW)                                                                              \
  hipLaunchKernelGGL((k_softmax_col<Ti, To, C, CW>), blocks_2d(blocks_for(CW)), dim3(256), 0, st, x, xs[0], \
                     xs[1], xs[2], y, ys[0], ys[1], ys[2], outer, dim, inner)
  if (cw == 64)
    NTOPS_SM_COL(64);
  else if (cw == 32)
    NTOPS_SM_COL(32);
  else if (cw == 16)
    NTOPS_SM_COL(16);
  else
    NTOPS_SM_COL(8);
#undef NTOPS_SM_COL
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
