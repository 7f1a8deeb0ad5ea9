// rms_norm and layer_norm over the trailing `cols` elements of each row.
//
// Math (fp32 accumulate, one rounding per output element):
//   rms_norm   kernels/rms_norm.py:10-20 -- y = x * rsqrt(mean(x^2) + eps) * w
//              (torch's fused CPU kernel applies the weight in fp32 before
//              the single rounding; eps defaults are resolved by the caller)
//   layer_norm kernels/layer_norm.py:11-31 -- mean, biased variance of
//              (x - mean) (two passes over the register-resident row),
//              rstd = 1 / sqrt(var + eps); written as torch's CPU kernel
//              evaluates it: y = (x * rstd + (-mean * rstd)) * w + b.
//
//   add_rms_norm  (no ntops counterpart; the residual step of an LLM block)
//              h = x + residual rounded to the element type (what torch's
//              `x + residual` produces), written out as the new residual,
//              then y = rms_norm(h) as above -- identical, element for
//              element, to the two separate kernels, in one pass.
//
// Vector path: one HBM read + one HBM write per element, row held in VGPRs
// (see rowcommon.h), one row group per block.  Looped path (unaligned rows, or rows wider than 64K
// 16-bit elements): one 256-thread block per row, scalar strided accesses,
// re-reading the row from L2 for the second / third pass.
//
// Weight and bias reads are cache traffic of their own: every row re-reads
// the whole parameter row from L1 / L2.  The kernels share one parameter
// load between the rows of a wave slot where the registers allow it.
#include "dispatch.h"
#include "rowcommon.h"
#include "rowwide.h"

namespace ntops {
namespace {

template <typename T>
__device__ __forceinline__ float to_f(T v) {
  return static_cast<float>(v);
}

// -------------------------------------------------------------- rms_norm --
// A wave slot owns R consecutive rows (R = 2 for rows of up to 2 packs per
// lane): the weight packs, loaded once next to the row loads, serve all R
// (wider shapes keep R = 1 and load the weight at its use, for registers).
// On MI355X the weight's cache traffic, not its instruction count, is what
// costs: rms_norm bf16 (16384, 4096) runs 42.2 us with the weight loads
// issued but returning zeros (extent 0), 44.1 us reading it once per row,
// 43.6 us once per two rows (same box, eager launches).
template <typename T, typename W, int CHUNKS, int WPR, int R>
__global__ __launch_bounds__(RowShape<WPR>::kThreads) void k_rms_vec(
    const T* __restrict__ x, int64_t xs, const W* __restrict__ w, T* __restrict__ y, int64_t ys,
    int64_t rows, int cols, float eps) {
  constexpr int V = Pack16<T>::N;
  constexpr int RPB = RowShape<WPR>::kRowsPerBlock;
  constexpr bool kEarly = R > 1;  // one row per slot: weight loaded at its use (fewer VGPRs)
  __shared__ float red[R * RPB * WPR];
  const RowPos p = row_pos<WPR>();
  const int npk = cols / V;
  // past the last row: loads read 0, stores are dropped
  const int64_t row0 = (block_id() * RPB + p.row_in_block) * R;
  Pack16<T> r[R][CHUNKS];
#pragma unroll
  for (int k = 0; k < R; ++k) load_row<WPR>(r[k], x, xs, rows, p, npk, row0 + k);
  const __amdgpu_buffer_rsrc_t wr = param_rsrc<V>(w, npk);
  ParamPack<W, V> wq[CHUNKS];
  if constexpr (kEarly)
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) wq[c].load(wr, pack_of<WPR>(p, c));
  float ss[R];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    ss[k] = 0.f;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float f = to_f(r[k][c].v[i]);
        ss[k] = fmaf(f, f, ss[k]);  // as k_add_rms_vec: one fma per element
      }
  }
  rows_sum<WPR>(ss, red, p);
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const float rstd = 1.0f / __fsqrt_rn(ss[k] / static_cast<float>(cols) + eps);
    const int64_t row = row0 + k;
    const bool row_ok = row < rows;
    const __amdgpu_buffer_rsrc_t out = buffer_rsrc(y + (row_ok ? row : 0) * ys, row_ok ? npk * 16u : 0u);
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      if constexpr (!kEarly) wq[c].load(wr, pack_of<WPR>(p, c));
      Pack16<T> o;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float wv = w != nullptr ? wq[c].get(i) : 1.0f;
        o.v[i] = static_cast<T>(mul_nc(mul_nc(to_f(r[k][c].v[i]), rstd), wv));
      }
      buffer_store16_nt(out, pack_of<WPR>(p, c) * 16u, o);
    }
  }
}

template <typename T, typename W>
__global__ __launch_bounds__(256) void k_rms_loop(const T* x, int64_t xs, const W* w, int64_t wrs, T* y,
                                                   int64_t ys, int64_t rows, int64_t cols, float eps) {
  __shared__ float red[4];
  const int64_t row = block_id();
  if (row >= rows) return;  // the tail of a 2-D grid (the whole block)
  const T* xr = x + row * xs;
  float ss = 0.f;
  for (int64_t j = threadIdx.x; j < cols; j += 256) {
    const float f = to_f(xr[j]);
    ss += f * f;
  }
  ss = block_sum256(ss, red);
  const float rstd = 1.0f / __fsqrt_rn(ss / static_cast<float>(cols) + eps);
  T* yr = y + row * ys;
  const W* wr = w != nullptr ? w + row * wrs : nullptr;
  for (int64_t j = threadIdx.x; j < cols; j += 256) {
    const float wv = wr != nullptr ? static_cast<float>(wr[j]) : 1.0f;
    yr[j] = static_cast<T>(mul_nc(mul_nc(to_f(xr[j]), rstd), wv));
  }
}

// ---------------------------------------------------- residual + rms_norm --
// Reads x and residual once, writes the rounded sum h (the new residual) and
// y = rms_norm(h); h stays in VGPRs between the two.  out / res_out may
// alias x / residual (each element is read and written by one thread).
// Up to 4 packs per lane, the weight is loaded with the rows and h is
// stored before the reduction (bf16 (16384, 4096): 88.7 -> 85.7 us, same
// box), spreading the writes over the kernel; wider shapes keep h packed
// across the reduction and load the weight after it, to fit the 128 VGPRs
// of a 1024-thread block.
template <typename T, typename W, int CHUNKS, int WPR>
__global__ __launch_bounds__(RowShape<WPR>::kThreads) void k_add_rms_vec(
    const T* x, int64_t xs, const T* res, int64_t rs, const W* __restrict__ w, T* y, int64_t ys, T* ro,
    int64_t ros, int64_t rows, int cols, float eps) {
  constexpr int V = Pack16<T>::N;
  constexpr int RPB = RowShape<WPR>::kRowsPerBlock;
  constexpr bool kEarly = CHUNKS <= 4;
  __shared__ float red[RPB * WPR];
  const RowPos p = row_pos<WPR>();
  const int64_t row = block_id() * RPB + p.row_in_block;
  const bool row_ok = row < rows;
  const int npk = cols / V;
  const uint32_t extent = row_ok ? npk * 16u : 0u;  // past the row end: loads give 0, stores dropped
  const int64_t row_c = row_ok ? row : 0;

  const __amdgpu_buffer_rsrc_t in_x = buffer_rsrc(x + row_c * xs, extent);
  const __amdgpu_buffer_rsrc_t in_r = buffer_rsrc(res + row_c * rs, extent);
  const __amdgpu_buffer_rsrc_t wr = param_rsrc<V>(w, npk);
  const __amdgpu_buffer_rsrc_t out_r = buffer_rsrc(ro + row_c * ros, extent);
  Pack16<T> h[CHUNKS];
  ParamPack<W, V> wq[CHUNKS];
  if constexpr (kEarly) {
    Pack16<T> a[CHUNKS], b[CHUNKS];
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      a[c] = buffer_load16_nt<T>(in_x, pack_of<WPR>(p, c) * 16u);
      b[c] = buffer_load16_nt<T>(in_r, pack_of<WPR>(p, c) * 16u);
    }
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) wq[c].load(wr, pack_of<WPR>(p, c));
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
      for (int i = 0; i < V; ++i) h[c].v[i] = static_cast<T>(add_nc(to_f(a[c].v[i]), to_f(b[c].v[i])));
  } else {
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const Pack16<T> a = buffer_load16_nt<T>(in_x, pack_of<WPR>(p, c) * 16u);
      const Pack16<T> b = buffer_load16_nt<T>(in_r, pack_of<WPR>(p, c) * 16u);
#pragma unroll
      for (int i = 0; i < V; ++i) h[c].v[i] = static_cast<T>(add_nc(to_f(a.v[i]), to_f(b.v[i])));
      // at most four chunks of both inputs in flight, or the two inputs plus
      // the sums overflow the 128 VGPRs of a 1024-thread block
      if ((c & 3) == 3) __builtin_amdgcn_sched_barrier(0);
    }
  }
  float ss[1] = {0.f};
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float f = to_f(h[c].v[i]);
      ss[0] = fmaf(f, f, ss[0]);  // as k_rms_vec: one fma per element
    }
  if constexpr (kEarly) {
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) buffer_store16_nt(out_r, pack_of<WPR>(p, c) * 16u, h[c]);
  } else {
    // keep h packed across the reduction (the fp32 copies the compiler would
    // otherwise carry do not fit beside it)
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      u32x4 bits = __builtin_bit_cast(u32x4, h[c]);
      asm volatile("" : "+v"(bits));
      h[c] = __builtin_bit_cast(Pack16<T>, bits);
    }
  }
  rows_sum<WPR>(ss, red, p);
  const float rstd = 1.0f / __fsqrt_rn(ss[0] / static_cast<float>(cols) + eps);

  const __amdgpu_buffer_rsrc_t out_y = buffer_rsrc(y + row_c * ys, extent);
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int pk = pack_of<WPR>(p, c);
    if constexpr (!kEarly) {
      buffer_store16_nt(out_r, pk * 16u, h[c]);
      wq[c].load(wr, pk);
    }
    Pack16<T> o;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float wv = w != nullptr ? wq[c].get(i) : 1.0f;
      o.v[i] = static_cast<T>(mul_nc(mul_nc(to_f(h[c].v[i]), rstd), wv));
    }
    buffer_store16_nt(out_y, pk * 16u, o);
  }
}

// ------------------------------------------------------------ layer_norm --
// Each element is converted to fp32 once and the row stays in fp32 VGPRs
// through both reductions and the write.  Packs past the row end load as
// zeros; the variance pass sums each pack's squares apart and adds the sum
// only for packs inside the row (one select per pack, not per element;
// subtracting the pads' known share n_pad * mean^2 instead loses the
// variance to cancellation when |mean| >> std).  The output is
// fma(fma(x, rstd, -mean * rstd), w, b): torch's CPU expression with the two
// products contracted (a different bf16 rounding only within ~2 fp32 ulps
// of a rounding boundary).
// R rows per wave slot share the weight and bias packs, which are then
// loaded with the rows (R = 2 up to 2 packs per lane: bf16 (16384, 4096) on
// 2 packs x 4 waves 45.3 us, against 46.1 us for one row per slot on 4 x 2
// with the parameters loaded at their use; loaded early for one row per
// slot they cost occupancy and measured 48.2 us).
template <typename T, typename W, int CHUNKS, int WPR, int R>
__global__ __launch_bounds__(RowShape<WPR>::kThreads) void k_ln_vec(
    const T* __restrict__ x, int64_t xs, const W* __restrict__ w, const W* __restrict__ b,
    T* __restrict__ y, int64_t ys, int64_t rows, int cols, float eps) {
  constexpr int V = Pack16<T>::N;
  constexpr int RPB = RowShape<WPR>::kRowsPerBlock;
  constexpr bool kEarly = R > 1;
  __shared__ float red0[R * RPB * WPR];
  __shared__ float red1[R * RPB * WPR];
  const RowPos p = row_pos<WPR>();
  const int npk = cols / V;
  // past the last row: loads read 0, stores are dropped
  const int64_t row0 = (block_id() * RPB + p.row_in_block) * R;
  const __amdgpu_buffer_rsrc_t wr = param_rsrc<V>(w, npk);
  const __amdgpu_buffer_rsrc_t br = param_rsrc<V>(b, npk);
  float f[R][CHUNKS][V];
  ParamPack<W, V> wq[CHUNKS], bq[CHUNKS];
  {
    Pack16<T> r[R][CHUNKS];
#pragma unroll
    for (int k = 0; k < R; ++k) load_row<WPR>(r[k], x, xs, rows, p, npk, row0 + k);
    if constexpr (kEarly) {
#pragma unroll
      for (int c = 0; c < CHUNKS; ++c) {
        wq[c].load(wr, pack_of<WPR>(p, c));
        bq[c].load(br, pack_of<WPR>(p, c));
      }
    }
#pragma unroll
    for (int k = 0; k < R; ++k)
#pragma unroll
      for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
        for (int i = 0; i < V; ++i) f[k][c][i] = to_f(r[k][c].v[i]);
  }
  float mean[R], acc[R];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
      for (int i = 0; i < V; i += 2) {
        s0 += f[k][c][i];
        s1 += f[k][c][i + 1];
      }
    acc[k] = s0 + s1;
  }
  rows_sum<WPR>(acc, red0, p);
#pragma unroll
  for (int k = 0; k < R; ++k) {
    // divided, not scaled by 1 / cols: a constant row's mean must come out exact
    mean[k] = acc[k] / static_cast<float>(cols);
    float q = 0.f;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      float q0 = 0.f, q1 = 0.f;
#pragma unroll
      for (int i = 0; i < V; i += 2) {
        const float d0 = f[k][c][i] - mean[k], d1 = f[k][c][i + 1] - mean[k];
        q0 = fmaf(d0, d0, q0);
        q1 = fmaf(d1, d1, q1);
      }
      q += pack_of<WPR>(p, c) < npk ? q0 + q1 : 0.f;
    }
    acc[k] = q;
  }
  rows_sum<WPR>(acc, red1, p);
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const float var = acc[k] * (1.0f / static_cast<float>(cols));
    const float rstd = 1.0f / __fsqrt_rn(fmaxf(var, 0.f) + eps);
    const float shift = -rstd * mean[k];
    const int64_t row = row0 + k;
    const bool row_ok = row < rows;
    const __amdgpu_buffer_rsrc_t out = buffer_rsrc(y + (row_ok ? row : 0) * ys, row_ok ? npk * 16u : 0u);
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int pk = pack_of<WPR>(p, c);
      if constexpr (!kEarly) {
        wq[c].load(wr, pk);
        bq[c].load(br, pk);
      }
      Pack16<T> o;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float wv = w != nullptr ? wq[c].get(i) : 1.0f;
        const float bv = b != nullptr ? bq[c].get(i) : 0.0f;
        o.v[i] = static_cast<T>(fmaf(fmaf(f[k][c][i], rstd, shift), wv, bv));
      }
      buffer_store16_nt(out, pk * 16u, o);
    }
  }
}

template <typename T, typename W>
__global__ __launch_bounds__(256) void k_ln_loop(const T* x, int64_t xs, const W* w, const W* b, int64_t wrs,
                                                  T* y, int64_t ys, int64_t rows, int64_t cols, float eps) {
  __shared__ float red[4];
  const int64_t row = block_id();
  if (row >= rows) return;  // the tail of a 2-D grid (the whole block)
  const T* xr = x + row * xs;
  float s = 0.f;
  for (int64_t j = threadIdx.x; j < cols; j += 256) s += to_f(xr[j]);
  const float mean = block_sum256(s, red) / static_cast<float>(cols);
  float q = 0.f;
  for (int64_t j = threadIdx.x; j < cols; j += 256) {
    const float d = to_f(xr[j]) - mean;
    q += d * d;
  }
  const float var = block_sum256(q, red) / static_cast<float>(cols);
  const float rstd = 1.0f / __fsqrt_rn(fmaxf(var, 0.f) + eps);
  const float shift = -rstd * mean;
  T* yr = y + row * ys;
  const W* wr = w != nullptr ? w + row * wrs : nullptr;
  const W* br = b != nullptr ? b + row * wrs : nullptr;
  for (int64_t j = threadIdx.x; j < cols; j += 256) {
    const float wv = wr != nullptr ? static_cast<float>(wr[j]) : 1.0f;
    const float bv = br != nullptr ? static_cast<float>(br[j]) : 0.0f;
    const float n = add_nc(mul_nc(to_f(xr[j]), rstd), shift);
    yr[j] = static_cast<T>(add_nc(mul_nc(n, wv), bv));
  }
}

// ------------------------------------------------------------ wide rows --
// Parameter packs fetched ahead of their use in the wide kernels' output
// pass (rms_norm: the weight; layer_norm: weight and bias, twice the VGPRs).
constexpr int kWideRmsPrefetch = 2, kWideLnPrefetch = 1;

// Rows of more than 8192 packs (rowwide.h): one block per CU walking rows;
// a row is read once into VGPRs and LDS (the next one loading during the
// output pass of the current one), each pass reads it there; the weight and
// bias are read at their use.
template <typename T, typename W>
__global__ __launch_bounds__(kWideThreads) void k_rms_wide(const T* __restrict__ x, int64_t xs,
                                                           const W* __restrict__ w, T* __restrict__ y,
                                                           int64_t ys, int64_t rows, int cols, float eps) {
  constexpr int V = Pack16<T>::N;
  __shared__ float red[kWideWaves];
  extern __shared__ __attribute__((aligned(16))) char wsm[];
  int64_t row = blockIdx.x;
  if (row >= rows) return;
  const int npk = cols / V, t = threadIdx.x;
  const __amdgpu_buffer_rsrc_t wr = param_rsrc<V>(w, npk);
  // the sum of squares of a row, accumulated as its packs land
  float ss = 0.f;
  auto visit = [&](const Pack16<T>& v) {
#pragma unroll
    for (int i = 0; i < V; ++i) ss = fmaf(to_f(v.v[i]), to_f(v.v[i]), ss);
  };
  WideRow<T> d;
  wide_load(d, x + row * xs, npk, wsm, visit);
  for (; row < rows; row += gridDim.x) {
    const float tot = wide_reduce(ss, red, [](float a, float b) { return a + b; });
    ss = 0.f;
    const float rstd = 1.0f / __fsqrt_rn(tot / static_cast<float>(cols) + eps);
    const __amdgpu_buffer_rsrc_t out = buffer_rsrc(y + row * ys, npk * 16u);
    auto fetch = [&](int pk) {
      ParamPack<W, V> wq;
      wq.load(wr, pk);
      return wq;
    };
    auto emit = [&](const Pack16<T>& v, int pk, const ParamPack<W, V>& wq) {
      Pack16<T> o;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float wv = w != nullptr ? wq.get(i) : 1.0f;
        o.v[i] = static_cast<T>(mul_nc(mul_nc(to_f(v.v[i]), rstd), wv));
      }
      buffer_store16_nt(out, pk * 16u, o);
    };
    const bool more = row + gridDim.x < rows;
    wide_emit_and_load<kWideRmsPrefetch>(d, more, x + (more ? row + gridDim.x : row) * xs, npk, fetch, emit,
                                         visit);
  }
}

template <typename T, typename W>
__global__ __launch_bounds__(kWideThreads) void k_ln_wide(const T* __restrict__ x, int64_t xs,
                                                          const W* __restrict__ w, const W* __restrict__ b,
                                                          T* __restrict__ y, int64_t ys, int64_t rows, int cols,
                                                          float eps) {
  constexpr int V = Pack16<T>::N;
  __shared__ float red[kWideWaves];
  extern __shared__ __attribute__((aligned(16))) char wsm[];
  int64_t row = blockIdx.x;
  if (row >= rows) return;
  const int npk = cols / V, t = threadIdx.x;
  const __amdgpu_buffer_rsrc_t wr = param_rsrc<V>(w, npk);
  const __amdgpu_buffer_rsrc_t br = param_rsrc<V>(b, npk);
  // the sum of a row, accumulated as its packs land
  float s = 0.f;
  auto visit = [&](const Pack16<T>& v) {
#pragma unroll
    for (int i = 0; i < V; ++i) s += to_f(v.v[i]);
  };
  WideRow<T> d;
  wide_load(d, x + row * xs, npk, wsm, visit);
  for (; row < rows; row += gridDim.x) {
    const auto sum = [](float a, float b) { return a + b; };
    const float mean = wide_reduce(s, red, sum) / static_cast<float>(cols);
    s = 0.f;
    wide_launder(d);
    float q2 = 0.f;
#pragma unroll
    for (int c = 0; c < kWideRegChunks; ++c) {
      float qc = 0.f;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float dv = to_f(d.r[c].v[i]) - mean;
        qc = fmaf(dv, dv, qc);
      }
      q2 += c * kWideThreads + t < npk ? qc : 0.f;
    }
    for (int q = t; q < d.nl; q += kWideThreads) {
      const Pack16<T> v = wide_lds_pack(d, q);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float dv = to_f(v.v[i]) - mean;
        q2 = fmaf(dv, dv, q2);
      }
    }
    const float var = wide_reduce(q2, red, sum) * (1.0f / static_cast<float>(cols));
    wide_launder(d);
    const float rstd = 1.0f / __fsqrt_rn(fmaxf(var, 0.f) + eps);
    const float shift = -rstd * mean;
    const __amdgpu_buffer_rsrc_t out = buffer_rsrc(y + row * ys, npk * 16u);
    struct WB {
      ParamPack<W, V> w, b;
    };
    auto fetch = [&](int pk) {
      WB p;
      p.w.load(wr, pk);
      p.b.load(br, pk);
      return p;
    };
    auto emit = [&](const Pack16<T>& v, int pk, const WB& p) {
      const ParamPack<W, V>& wq = p.w;
      const ParamPack<W, V>& bq = p.b;
      Pack16<T> o;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float wv = w != nullptr ? wq.get(i) : 1.0f;
        const float bv = b != nullptr ? bq.get(i) : 0.0f;
        o.v[i] = static_cast<T>(fmaf(fmaf(to_f(v.v[i]), rstd, shift), wv, bv));
      }
      buffer_store16_nt(out, pk * 16u, o);
    };
    const bool more = row + gridDim.x < rows;
    wide_emit_and_load<kWideLnPrefetch>(d, more, x + (more ? row + gridDim.x : row) * xs, npk, fetch, emit,
                                        visit);
  }
}

// ------------------------------------------- rows that are not 16-byte runs --
// Rows whose width or start is not a multiple of 16 bytes (an odd width such
// as 4100, or a view into wider rows), with the output rows laid out at the
// same offset within 16 bytes as the input rows: each row splits into a
// head of `head` elements up to the first 16-byte boundary, `npk` whole
// packs and a tail (head, tail < V).  The packs travel as in the aligned
// kernels (register-resident, one HBM read and one write); lanes 0..head-1
// of the row's first wave hold the head elements and lanes 0..tail-1 of its
// last wave the tail (element loads and stores through buffer resources
// whose extent is the head / tail: branch-free, zeros elsewhere).  The
// weight and bias rows are staged once per block in LDS, where element j is
// read at any offset: a pack of the row starts `head` elements past a
// parameter pack boundary.
struct OddRow {
  int head, npk, tail;
};
template <typename T>
__device__ __forceinline__ OddRow odd_row(const T* row, int cols) {
  constexpr int V = Pack16<T>::N;
  const int off = static_cast<int>((reinterpret_cast<uintptr_t>(row) & 15u) / sizeof(T));
  const int head = min((V - off) & (V - 1), cols);
  const int npk = (cols - head) / V;
  return {head, npk, cols - head - npk * V};
}

template <typename T>
__device__ __forceinline__ T buffer_load_elem(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  if constexpr (sizeof(T) == 2)
    return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, kBufNT));
  else
    return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kBufNT));
}
template <typename T>
__device__ __forceinline__ void buffer_store_elem(__amdgpu_buffer_rsrc_t r, uint32_t off, T v) {
  if constexpr (sizeof(T) == 2)
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, v), r, off, 0, kBufNT);
  else
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, v), r, off, 0, kBufNT);
}

// One row of an odd-layout slot as this lane holds it: the packs, and the
// head / tail element this lane owns (zero where it owns none).
template <typename T, int CHUNKS>
struct OddSlot {
  Pack16<T> pk[CHUNKS];
  T hd, tl;
  bool own_hd, own_tl;
};

template <int WPR, typename T, int CHUNKS>
__device__ __forceinline__ void odd_load(OddSlot<T, CHUNKS>& d, const T* row, const OddRow& g, bool row_ok,
                                         const RowPos& p) {
  const bool first = p.wave_in_row == 0, last = p.wave_in_row == WPR - 1;
  const __amdgpu_buffer_rsrc_t rp = buffer_rsrc(row + g.head, row_ok ? g.npk * 16u : 0u);
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) d.pk[c] = buffer_load16_nt<T>(rp, pack_of<WPR>(p, c) * 16u);
  const __amdgpu_buffer_rsrc_t rh = buffer_rsrc(row, row_ok && first ? g.head * sizeof(T) : 0u);
  const __amdgpu_buffer_rsrc_t rt =
      buffer_rsrc(row + g.head + g.npk * Pack16<T>::N, row_ok && last ? g.tail * sizeof(T) : 0u);
  d.hd = buffer_load_elem<T>(rh, p.lane * sizeof(T));
  d.tl = buffer_load_elem<T>(rt, p.lane * sizeof(T));
  d.own_hd = row_ok && first && p.lane < g.head;
  d.own_tl = row_ok && last && p.lane < g.tail;
}

// This lane's sum of squares over its elements of the row: head, packs,
// tail.  rms_norm and add_rms_norm share it, so their outputs agree bit for
// bit on the same row layout.  The products and sums are spelled as explicit
// fmas: left to contraction, `hd * hd + p * p` may become fma(p, p, hd * hd)
// in one kernel and fma(hd, hd, p * p) in the other.
template <typename T, int CHUNKS>
__device__ __forceinline__ float odd_sumsq(const OddSlot<T, CHUNKS>& d) {
  constexpr int V = Pack16<T>::N;
  float ss = mul_nc(to_f(d.hd), to_f(d.hd));
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float f = to_f(d.pk[c].v[i]);
      ss = fmaf(f, f, ss);
    }
  return fmaf(to_f(d.tl), to_f(d.tl), ss);
}

// Stages `cols` parameters of type W at `src` into LDS at `dst` (16-byte
// packs, then the last cols % per-pack elements one by one).
template <typename W>
__device__ __forceinline__ void stage_param(W* dst, const W* src, int cols) {
  constexpr int kPer = Pack16<W>::N;
  const int full = cols / kPer;
  for (int q = threadIdx.x; q < full; q += blockDim.x)
    *reinterpret_cast<u32x4*>(dst + q * kPer) = *reinterpret_cast<const u32x4*>(src + q * kPer);
  for (int e = full * kPer + threadIdx.x; e < cols; e += blockDim.x) dst[e] = src[e];
}

// Writes one row's normalised values: packs, head and tail; f(v, j) gives
// the output for element value v at column j.
template <int WPR, typename T, int CHUNKS, typename F>
__device__ __forceinline__ void odd_store(T* row, const OddRow& g, bool row_ok, const RowPos& p,
                                          const OddSlot<T, CHUNKS>& d, F f) {
  constexpr int V = Pack16<T>::N;
  const bool first = p.wave_in_row == 0, last = p.wave_in_row == WPR - 1;
  const __amdgpu_buffer_rsrc_t rp = buffer_rsrc(row + g.head, row_ok ? g.npk * 16u : 0u);
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int pk = pack_of<WPR>(p, c);
    const int j0 = g.head + pk * V;
    Pack16<T> o;
#pragma unroll
    for (int i = 0; i < V; ++i) o.v[i] = f(d.pk[c].v[i], pk < g.npk ? j0 + i : 0);
    buffer_store16_nt(rp, pk * 16u, o);
  }
  const __amdgpu_buffer_rsrc_t rh = buffer_rsrc(row, row_ok && first ? g.head * sizeof(T) : 0u);
  const __amdgpu_buffer_rsrc_t rt =
      buffer_rsrc(row + g.head + g.npk * V, row_ok && last ? g.tail * sizeof(T) : 0u);
  buffer_store_elem<T>(rh, p.lane * sizeof(T), f(d.hd, d.own_hd ? p.lane : 0));
  buffer_store_elem<T>(rt, p.lane * sizeof(T), f(d.tl, d.own_tl ? g.head + g.npk * V + p.lane : 0));
}

// Bytes of LDS the odd-layout kernels stage per parameter row.
template <typename W>
__host__ __device__ inline int64_t odd_param_bytes(int64_t cols) {
  return (cols * static_cast<int64_t>(sizeof(W)) + 15) / 16 * 16;
}
// Their most staged-parameter LDS: under the 64 KiB a launch may take without
// raising its limit, with room for the kernels' static reduction scratch.
constexpr int64_t kOddLdsMax = 60 * 1024;

template <typename T, typename W, int CHUNKS, int WPR>
__global__ __launch_bounds__(RowShape<WPR>::kThreads) void k_rms_odd(
    const T* __restrict__ x, int64_t xs, const W* __restrict__ w, T* __restrict__ y, int64_t ys,
    int64_t rows, int cols, float eps) {
  constexpr int RPB = RowShape<WPR>::kRowsPerBlock;
  __shared__ float red[RPB * WPR];
  extern __shared__ __attribute__((aligned(16))) char psm[];
  W* wl = reinterpret_cast<W*>(psm);
  const RowPos p = row_pos<WPR>();
  const int64_t row = block_id() * RPB + p.row_in_block;
  const bool row_ok = row < rows;
  const T* xr = x + (row_ok ? row : 0) * xs;
  const OddRow g = odd_row(xr, cols);
  OddSlot<T, CHUNKS> d;
  odd_load<WPR>(d, xr, g, row_ok, p);
  if (w != nullptr) stage_param(wl, w, cols);
  float ss[1] = {odd_sumsq(d)};
  __syncthreads();  // the staged weight (and, for one wave per row, nothing else)
  rows_sum<WPR>(ss, red, p);
  const float rstd = 1.0f / __fsqrt_rn(ss[0] / static_cast<float>(cols) + eps);
  odd_store<WPR>(y + (row_ok ? row : 0) * ys, g, row_ok, p, d, [&](T v, int j) {
    const float wv = w != nullptr ? static_cast<float>(wl[j]) : 1.0f;
    return static_cast<T>(mul_nc(mul_nc(to_f(v), rstd), wv));
  });
}

// x, residual, new residual and output share one layout; h = x + residual
// is rounded, stored, and normalised exactly as k_rms_odd normalises a row
// of that layout.
template <typename T, typename W, int CHUNKS, int WPR>
__global__ __launch_bounds__(RowShape<WPR>::kThreads) void k_add_rms_odd(
    const T* x, int64_t xs, const T* res, int64_t rs, const W* __restrict__ w, T* y, int64_t ys, T* ro,
    int64_t ros, int64_t rows, int cols, float eps) {
  constexpr int V = Pack16<T>::N;
  constexpr int RPB = RowShape<WPR>::kRowsPerBlock;
  __shared__ float red[RPB * WPR];
  extern __shared__ __attribute__((aligned(16))) char psm[];
  W* wl = reinterpret_cast<W*>(psm);
  const RowPos p = row_pos<WPR>();
  const int64_t row = block_id() * RPB + p.row_in_block;
  const bool row_ok = row < rows;
  const int64_t rc = row_ok ? row : 0;
  const OddRow g = odd_row(x + rc * xs, cols);
  OddSlot<T, CHUNKS> d, e;
  odd_load<WPR>(d, x + rc * xs, g, row_ok, p);
  odd_load<WPR>(e, res + rc * rs, g, row_ok, p);
  if (w != nullptr) stage_param(wl, w, cols);
  auto add = [](T a, T b) { return static_cast<T>(add_nc(to_f(a), to_f(b))); };
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
    for (int i = 0; i < V; ++i) d.pk[c].v[i] = add(d.pk[c].v[i], e.pk[c].v[i]);
  d.hd = add(d.hd, e.hd);
  d.tl = add(d.tl, e.tl);
  odd_store<WPR>(ro + rc * ros, g, row_ok, p, d, [](T v, int) { return v; });
  float ss[1] = {odd_sumsq(d)};
  __syncthreads();
  rows_sum<WPR>(ss, red, p);
  const float rstd = 1.0f / __fsqrt_rn(ss[0] / static_cast<float>(cols) + eps);
  odd_store<WPR>(y + rc * ys, g, row_ok, p, d, [&](T v, int j) {
    const float wv = w != nullptr ? static_cast<float>(wl[j]) : 1.0f;
    return static_cast<T>(mul_nc(mul_nc(to_f(v), rstd), wv));
  });
}

template <typename T, typename W, int CHUNKS, int WPR>
__global__ __launch_bounds__(RowShape<WPR>::kThreads) void k_ln_odd(
    const T* __restrict__ x, int64_t xs, const W* __restrict__ w, const W* __restrict__ b,
    T* __restrict__ y, int64_t ys, int64_t rows, int cols, float eps) {
  constexpr int V = Pack16<T>::N;
  constexpr int RPB = RowShape<WPR>::kRowsPerBlock;
  __shared__ float red0[RPB * WPR];
  __shared__ float red1[RPB * WPR];
  extern __shared__ __attribute__((aligned(16))) char psm[];
  W* wl = reinterpret_cast<W*>(psm);
  W* bl = reinterpret_cast<W*>(psm + odd_param_bytes<W>(cols));
  const RowPos p = row_pos<WPR>();
  const int64_t row = block_id() * RPB + p.row_in_block;
  const bool row_ok = row < rows;
  const T* xr = x + (row_ok ? row : 0) * xs;
  const OddRow g = odd_row(xr, cols);
  OddSlot<T, CHUNKS> d;
  odd_load<WPR>(d, xr, g, row_ok, p);
  if (w != nullptr) stage_param(wl, w, cols);
  if (b != nullptr) stage_param(bl, b, cols);
  float acc[1];
  {
    float s0 = to_f(d.hd), s1 = 0.f;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
      for (int i = 0; i < V; i += 2) {
        s0 += to_f(d.pk[c].v[i]);
        s1 += to_f(d.pk[c].v[i + 1]);
      }
    acc[0] = s0 + s1 + to_f(d.tl);
  }
  __syncthreads();
  rows_sum<WPR>(acc, red0, p);
  const float mean = acc[0] / static_cast<float>(cols);
  {
    const float dh = to_f(d.hd) - mean, dt = to_f(d.tl) - mean;
    float q = (d.own_hd ? dh * dh : 0.f) + (d.own_tl ? dt * dt : 0.f);
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      float q0 = 0.f, q1 = 0.f;
#pragma unroll
      for (int i = 0; i < V; i += 2) {
        const float d0 = to_f(d.pk[c].v[i]) - mean, d1 = to_f(d.pk[c].v[i + 1]) - mean;
        q0 = fmaf(d0, d0, q0);
        q1 = fmaf(d1, d1, q1);
      }
      q += pack_of<WPR>(p, c) < g.npk ? q0 + q1 : 0.f;
    }
    acc[0] = q;
  }
  rows_sum<WPR>(acc, red1, p);
  const float var = acc[0] * (1.0f / static_cast<float>(cols));
  const float rstd = 1.0f / __fsqrt_rn(fmaxf(var, 0.f) + eps);
  const float shift = -rstd * mean;
  odd_store<WPR>(y + (row_ok ? row : 0) * ys, g, row_ok, p, d, [&](T v, int j) {
    const float wv = w != nullptr ? static_cast<float>(wl[j]) : 1.0f;
    const float bv = b != nullptr ? static_cast<float>(bl[j]) : 0.0f;
    return static_cast<T>(fmaf(fmaf(to_f(v), rstd, shift), wv, bv));
  });
}

// -------------------------------------------------------------- dispatch --
// Rows of a and b start at the same offset within 16 bytes, row for row.
template <typename T>
bool same_layout(const void* a, int64_t as, const void* b, int64_t bs) {
  return ((reinterpret_cast<uintptr_t>(a) - reinterpret_cast<uintptr_t>(b)) & 15u) == 0 &&
         (((as - bs) * static_cast<int64_t>(sizeof(T))) & 15) == 0;
}

// Rows of whole 16-byte packs, every row 16-byte aligned, in x and y.
template <typename T>
bool aligned16_rows(const void* x, int64_t xs, const void* y, int64_t ys, int64_t cols) {
  constexpr int V = Pack16<T>::N;
  return cols % V == 0 && xs % V == 0 && ys % V == 0 && aligned16(x) && aligned16(y);
}

// Launch shape of the odd-layout kernels: from the most whole packs a row
// can hold (at least one pack, for rows shorter than a pack).
inline bool pick_odd_cfg(int64_t cols, int v, VecCfg* cfg) { return pick_row_cfg(cols / v > 0 ? cols / v : 1, cfg); }

template <typename T, typename W>
int run_rms(int64_t rows, int64_t cols, const void* xv, int64_t xs, const void* wv, int64_t wrs, double eps,
            void* yv, int64_t ys, hipStream_t st) {
  const T* x = static_cast<const T*>(xv);
  const W* w = static_cast<const W*>(wv);
  T* y = static_cast<T*>(yv);
  constexpr int V = Pack16<T>::N;
  VecCfg cfg;
  // a weight that differs per row (wrs != 0) takes the looped kernel
  const bool vec = (cols % V == 0) && (xs % V == 0) && (ys % V == 0) && aligned16(x) &&
                   aligned16(y) && (w == nullptr || (aligned16(w) && wrs == 0)) && pick_row_cfg(cols / V, &cfg);
  const float feps = static_cast<float>(eps);
  if (vec) {
#define NTOPS_RMS_CASE(CH, WP)                                                                    \
  if (cfg.chunks == CH && cfg.wpr == WP) {                                                        \
    constexpr int R = CH <= 2 ? 2 : 1;                                                            \
    hipLaunchKernelGGL((k_rms_vec<T, W, CH, WP, R>),                                              \
                       blocks_2d(ceil_div(rows, RowShape<WP>::kRowsPerBlock * R)),                \
                       dim3(RowShape<WP>::kThreads), 0, st, x, xs, w, y, ys, rows,                \
                       static_cast<int>(cols), feps);                                             \
    return check_launch("rms_norm");                                                              \
  }
    NTOPS_ROW_CASES(NTOPS_RMS_CASE)
#undef NTOPS_RMS_CASE
  }
  if (aligned16_rows<T>(x, xs, y, ys, cols) && (w == nullptr || (aligned16(w) && wrs == 0)) &&
      wide_row_fits(cols / V)) {
    static bool lds_set = false;
    if (int e = wide_lds_attr(k_rms_wide<T, W>, lds_set)) return e;
    hipLaunchKernelGGL((k_rms_wide<T, W>), dim3(wide_grid(rows)), dim3(kWideThreads), wide_lds_bytes(cols / V), st, x, xs,
                       w, y, ys, rows, static_cast<int>(cols), feps);
    return check_launch("rms_norm");
  }
  const int64_t lds = w != nullptr ? odd_param_bytes<W>(cols) : 0;
  if (same_layout<T>(x, xs, y, ys) && (w == nullptr || (aligned16(w) && wrs == 0)) && lds <= kOddLdsMax &&
      pick_odd_cfg(cols, V, &cfg)) {
#define NTOPS_RMS_ODD_CASE(CH, WP)                                                                \
  if (cfg.chunks == CH && cfg.wpr == WP) {                                                        \
    hipLaunchKernelGGL((k_rms_odd<T, W, CH, WP>), blocks_2d(ceil_div(rows, RowShape<WP>::kRowsPerBlock)), \
                       dim3(RowShape<WP>::kThreads), static_cast<unsigned>(lds), st, x, xs, w, y, ys,    \
                       rows, static_cast<int>(cols), feps);                                       \
    return check_launch("rms_norm");                                                              \
  }
    NTOPS_ROW_CASES(NTOPS_RMS_ODD_CASE)
#undef NTOPS_RMS_ODD_CASE
  }
  hipLaunchKernelGGL((k_rms_loop<T, W>), blocks_2d(rows), dim3(256), 0, st, x, xs, w, wrs, y, ys, rows, cols, feps);
  return check_launch("rms_norm");
}

template <typename T, typename W>
int run_ln(int64_t rows, int64_t cols, const void* xv, int64_t xs, const void* wv,
           const void* bv, int64_t wrs, double eps, void* yv, int64_t ys, hipStream_t st) {
  const T* x = static_cast<const T*>(xv);
  const W* w = static_cast<const W*>(wv);
  const W* b = static_cast<const W*>(bv);
  T* y = static_cast<T*>(yv);
  constexpr int V = Pack16<T>::N;
  VecCfg cfg;
  const bool vec = (cols % V == 0) && (xs % V == 0) && (ys % V == 0) && aligned16(x) &&
                   aligned16(y) && (w == nullptr || aligned16(w)) &&
                   (b == nullptr || aligned16(b)) && (wrs == 0 || (w == nullptr && b == nullptr)) &&
                   pick_row_cfg(cols / V, &cfg);
  const float feps = static_cast<float>(eps);
  if (vec) {
#define NTOPS_LN_CASE(CH, WP)                                                                     \
  if (cfg.chunks == CH && cfg.wpr == WP) {                                                        \
    constexpr int R = CH <= 2 ? 2 : 1;                                                            \
    hipLaunchKernelGGL((k_ln_vec<T, W, CH, WP, R>),                                               \
                       blocks_2d(ceil_div(rows, RowShape<WP>::kRowsPerBlock * R)),                \
                       dim3(RowShape<WP>::kThreads), 0, st, x, xs, w, b, y, ys, rows,             \
                       static_cast<int>(cols), feps);                                             \
    return check_launch("layer_norm");                                                            \
  }
    NTOPS_ROW_CASES(NTOPS_LN_CASE)
#undef NTOPS_LN_CASE
  }
  if (aligned16_rows<T>(x, xs, y, ys, cols) && (w == nullptr || aligned16(w)) && (b == nullptr || aligned16(b)) &&
      wrs == 0 && wide_row_fits(cols / V)) {
    static bool lds_set = false;
    if (int e = wide_lds_attr(k_ln_wide<T, W>, lds_set)) return e;
    hipLaunchKernelGGL((k_ln_wide<T, W>), dim3(wide_grid(rows)), dim3(kWideThreads), wide_lds_bytes(cols / V), st, x, xs, w,
                       b, y, ys, rows, static_cast<int>(cols), feps);
    return check_launch("layer_norm");
  }
  const int64_t lds = (w != nullptr || b != nullptr) ? 2 * odd_param_bytes<W>(cols) : 0;
  if (same_layout<T>(x, xs, y, ys) && (w == nullptr || aligned16(w)) && (b == nullptr || aligned16(b)) &&
      wrs == 0 && lds <= kOddLdsMax && pick_odd_cfg(cols, V, &cfg)) {
#define NTOPS_LN_ODD_CASE(CH, WP)                                                                 \
  if (cfg.chunks == CH && cfg.wpr == WP) {                                                        \
    hipLaunchKernelGGL((k_ln_odd<T, W, CH, WP>), blocks_2d(ceil_div(rows, RowShape<WP>::kRowsPerBlock)), \
                       dim3(RowShape<WP>::kThreads), static_cast<unsigned>(lds), st, x, xs, w, b, y, ys, \
                       rows, static_cast<int>(cols), feps);                                       \
    return check_launch("layer_norm");                                                            \
  }
    NTOPS_ROW_CASES(NTOPS_LN_ODD_CASE)
#undef NTOPS_LN_ODD_CASE
  }
  hipLaunchKernelGGL((k_ln_loop<T, W>), blocks_2d(rows), dim3(256), 0, st, x, xs, w, b, wrs, y, ys, rows, cols,
                     feps);
  return check_launch("layer_norm");
}

// run_add_rms's answer for layouts it leaves to add followed by rms_norm
// (not a status code).
constexpr int kComposeAddRms = -1;

template <typename T, typename W>
int run_add_rms(int64_t rows, int64_t cols, const void* xv, int64_t xs, const void* rv, int64_t rs,
                const void* wv, int64_t wrs, double eps, void* yv, int64_t ys, void* rov, int64_t ros,
                hipStream_t st) {
  const T* x = static_cast<const T*>(xv);
  const T* r = static_cast<const T*>(rv);
  const W* w = static_cast<const W*>(wv);
  T* y = static_cast<T*>(yv);
  T* ro = static_cast<T*>(rov);
  constexpr int V = Pack16<T>::N;
  VecCfg cfg;
  const bool vec = (cols % V == 0) && (xs % V == 0) && (rs % V == 0) && (ys % V == 0) && (ros % V == 0) &&
                   aligned16(x) && aligned16(r) && aligned16(y) && aligned16(ro) &&
                   (w == nullptr || (aligned16(w) && wrs == 0)) && pick_row_cfg(cols / V, &cfg);
  const float feps = static_cast<float>(eps);
  if (vec) {
#define NTOPS_ADD_RMS_CASE(CH, WP)                                                                \
  if (cfg.chunks == CH && cfg.wpr == WP) {                                                        \
    hipLaunchKernelGGL((k_add_rms_vec<T, W, CH, WP>), blocks_2d(ceil_div(rows, RowShape<WP>::kRowsPerBlock)), \
                       dim3(RowShape<WP>::kThreads), 0, st, x, xs, r, rs, w, y, ys, ro, ros,      \
                       rows, static_cast<int>(cols), feps);                                       \
    return check_launch("add_rms_norm");                                                          \
  }
    NTOPS_ROW_CASES(NTOPS_ADD_RMS_CASE)
#undef NTOPS_ADD_RMS_CASE
  }
  const int64_t lds = w != nullptr ? odd_param_bytes<W>(cols) : 0;
  if (same_layout<T>(x, xs, y, ys) && same_layout<T>(r, rs, y, ys) && same_layout<T>(ro, ros, y, ys) &&
      (w == nullptr || (aligned16(w) && wrs == 0)) && lds <= kOddLdsMax && pick_odd_cfg(cols, V, &cfg)) {
#define NTOPS_ADD_RMS_ODD_CASE(CH, WP)                                                            \
  if (cfg.chunks == CH && cfg.wpr == WP) {                                                        \
    hipLaunchKernelGGL((k_add_rms_odd<T, W, CH, WP>), blocks_2d(ceil_div(rows, RowShape<WP>::kRowsPerBlock)), \
                       dim3(RowShape<WP>::kThreads), static_cast<unsigned>(lds), st, x, xs, r, rs, w, y, ys,   \
                       ro, ros, rows, static_cast<int>(cols), feps);                              \
    return check_launch("add_rms_norm");                                                          \
  }
    NTOPS_ROW_CASES(NTOPS_ADD_RMS_ODD_CASE)
#undef NTOPS_ADD_RMS_ODD_CASE
  }
  return kComposeAddRms;
}

int check_rows(const char* what, int64_t rows, int64_t cols, const void* x, const void* y) {
  if (rows < 0 || cols < 0) return set_error(NTOPS_ERR_INVALID, "%s: negative size", what);
  if (rows > 0 && cols > 0 && (x == nullptr || y == nullptr))
    return set_error(NTOPS_ERR_INVALID, "%s: null pointer", what);
  if (rows > 0x7fffffffLL) return set_error(NTOPS_ERR_INVALID, "%s: too many rows", what);
  return NTOPS_OK;
}

}  // namespace
}  // namespace ntops

using namespace ntops;

extern "C" int ntops_rms_norm(int dtype, int64_t rows, int64_t cols, const void* x,
                              int64_t x_row_stride, const void* w, int64_t w_row_stride, int w_dtype,
                              double eps, void* y, int64_t y_row_stride, void* stream) {
  if (int e = check_rows("rms_norm", rows, cols, x, y)) return e;
  if (rows == 0 || cols == 0) return NTOPS_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (w != nullptr && w_dtype != dtype && w_dtype != NTOPS_F32)
    return set_error(NTOPS_ERR_UNSUPPORTED, "rms_norm: weight dtype must equal input dtype or be F32");
  return dispatch_float16_32(dtype, "rms_norm", [&](auto tag) {
    using T = decltype(tag);
    if (w != nullptr && w_dtype == NTOPS_F32 && dtype != NTOPS_F32)
      return run_rms<T, float>(rows, cols, x, x_row_stride, w, w_row_stride, eps, y, y_row_stride, st);
    return run_rms<T, T>(rows, cols, x, x_row_stride, w, w_row_stride, eps, y, y_row_stride, st);
  });
}

extern "C" int ntops_layer_norm(int dtype, int64_t rows, int64_t cols, const void* x,
                                int64_t x_row_stride, const void* w, const void* b, int64_t wb_row_stride,
                                int wb_dtype, double eps, void* y, int64_t y_row_stride, void* stream) {
  if (int e = check_rows("layer_norm", rows, cols, x, y)) return e;
  if (rows == 0 || cols == 0) return NTOPS_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if ((w != nullptr || b != nullptr) && wb_dtype != dtype && wb_dtype != NTOPS_F32)
    return set_error(NTOPS_ERR_UNSUPPORTED,
                     "layer_norm: weight/bias dtype must equal input dtype or be F32");
  return dispatch_float16_32(dtype, "layer_norm", [&](auto tag) {
    using T = decltype(tag);
    if ((w != nullptr || b != nullptr) && wb_dtype == NTOPS_F32 && dtype != NTOPS_F32)
      return run_ln<T, float>(rows, cols, x, x_row_stride, w, b, wb_row_stride, eps, y, y_row_stride, st);
    return run_ln<T, T>(rows, cols, x, x_row_stride, w, b, wb_row_stride, eps, y, y_row_stride, st);
  });
}

extern "C" int ntops_add_rms_norm(int dtype, int64_t rows, int64_t cols, const void* x, int64_t x_row_stride,
                                  const void* residual, int64_t residual_row_stride, const void* w,
                                  int64_t w_row_stride, int w_dtype, double eps, void* y, int64_t y_row_stride,
                                  void* residual_out,
                                  int64_t residual_out_row_stride, void* stream) {
  if (int e = check_rows("add_rms_norm", rows, cols, x, y)) return e;
  if (rows == 0 || cols == 0) return NTOPS_OK;
  if (residual == nullptr || residual_out == nullptr) return set_error(NTOPS_ERR_INVALID, "add_rms_norm: null pointer");
  if (y == residual_out) return set_error(NTOPS_ERR_INVALID, "add_rms_norm: out and residual_out must differ");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (w != nullptr && w_dtype != dtype && w_dtype != NTOPS_F32)
    return set_error(NTOPS_ERR_UNSUPPORTED, "add_rms_norm: weight dtype must equal input dtype or be F32");
  const int rc = dispatch_float16_32(dtype, "add_rms_norm", [&](auto tag) {
    using T = decltype(tag);
    if (w != nullptr && w_dtype == NTOPS_F32 && dtype != NTOPS_F32)
      return run_add_rms<T, float>(rows, cols, x, x_row_stride, residual, residual_row_stride, w, w_row_stride,
                                   eps, y, y_row_stride, residual_out, residual_out_row_stride, st);
    return run_add_rms<T, T>(rows, cols, x, x_row_stride, residual, residual_row_stride, w, w_row_stride, eps, y,
                             y_row_stride, residual_out, residual_out_row_stride, st);
  });
  if (rc != kComposeAddRms) return rc;
  // Layouts the one-pass kernels do not take (operands at different offsets
  // within 16 bytes, rows wider than the register budget, a weight that
  // differs per row): the sum through ntops_binary, then ntops_rms_norm over
  // the new residual -- the very kernels `add` and `rms_norm` run, so the
  // result is theirs element for element.
  const int64_t shape[2] = {rows, cols};
  const int64_t xst[2] = {x_row_stride, 1}, rst[2] = {residual_row_stride, 1}, ost[2] = {residual_out_row_stride, 1};
  if (int e = ntops_binary(NTOPS_BINARY_ADD, dtype, 2, shape, x, xst, residual, rst, 0.0, 0, 1.0, 1, residual_out,
                           ost, stream))
    return e;
  return ntops_rms_norm(dtype, rows, cols, residual_out, residual_out_row_stride, w, w_row_stride, w_dtype, eps, y,
                        y_row_stride, stream);
}
