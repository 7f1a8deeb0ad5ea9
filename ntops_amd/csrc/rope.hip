// rotary_position_embedding on (B, S, H, D) tensors.
//
// Rotation of each pair (kernels/rotary_position_embedding.py:39-47):
//   out0 = x0 * cos0 - x1 * sin0
//   out1 = x1 * cos1 + x0 * sin1
// where the pair is (i, i + D/2) for the half-rotation layout and (2i, 2i+1)
// for the interleaved layout (rotary_position_embedding.py:10-15).  With
// (S, D/2) tables (ntops' form) cos0 = cos1 = cos[s, i]; with (S, D) tables
// (the rotate_half form x*cos + rotate_half(x)*sin) each element uses its own
// table column.  Every product and every sum is rounded to the element type,
// which is exactly how torch evaluates that expression eagerly on bf16/fp16
// tensors (and how Triton evaluates ntops' application on them).
//
// Vector path: a thread owns one 16-byte pack of x0 values and the matching
// pack of x1 values (half layout) or one pack of interleaved pairs; a
// 256-thread block covers consecutive (b, s, h) rows, so the table row of a
// position is read by every head from L2.  Generic path: one thread per pair,
// any strides.
#include "dispatch.h"

namespace ntops {
namespace {

template <typename T>
__device__ __forceinline__ float rnd(float v) {
  if constexpr (std::is_same<T, float>::value)
    return v;
  else
    return static_cast<float>(static_cast<T>(v));
}

// One rotated pair with per-operation rounding to T.
template <typename T>
__device__ __forceinline__ void rotate(float x0, float x1, float c0, float s0, float c1, float s1,
                                       float& o0, float& o1) {
  o0 = rnd<T>(sub_nc(rnd<T>(mul_nc(x0, c0)), rnd<T>(mul_nc(x1, s0))));
  o1 = rnd<T>(add_nc(rnd<T>(mul_nc(x1, c1)), rnd<T>(mul_nc(x0, s1))));
}

struct RopeArgs {
  int64_t B, S, H, D;
  int64_t xs[4], ys[4];
  int64_t trs;    // table row stride
  int64_t tcols;  // D / 2 or D
};

// Half-rotation, vector path.  Work item = (row, pack j of the first half).
template <typename T>
__global__ __launch_bounds__(256) void k_rope_half_vec(const T* x, const T* sn, const T* cs, T* y,
                                                       RopeArgs a, int64_t items) {
  constexpr int V = Pack16<T>::N;
  const int64_t half = a.D / 2;
  const int64_t ppr = half / V;  // packs per half row
  const int64_t it = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (it >= items) return;
  const int64_t j = it % ppr;
  int64_t r = it / ppr;
  const int64_t h = r % a.H;
  r /= a.H;
  const int64_t s = r % a.S;
  const int64_t b = r / a.S;
  const int64_t xo = b * a.xs[0] + s * a.xs[1] + h * a.xs[2] + j * V;
  const int64_t yo = b * a.ys[0] + s * a.ys[1] + h * a.ys[2] + j * V;
  // x and y stream through once (non-temporal); the tables stay cacheable
  // because every head of a position re-reads them.
  const Pack16<T> x0 = load16_nt(x + xo);
  const Pack16<T> x1 = load16_nt(x + xo + half);
  const T* ct = cs + s * a.trs + j * V;
  const T* st = sn + s * a.trs + j * V;
  const Pack16<T> c0 = load16(ct);
  const Pack16<T> s0 = load16(st);
  Pack16<T> c1 = c0, s1 = s0;
  if (a.tcols != half) {
    c1 = load16(ct + half);
    s1 = load16(st + half);
  }
  Pack16<T> o0, o1;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    float r0, r1;
    rotate<T>(static_cast<float>(x0.v[i]), static_cast<float>(x1.v[i]),
              static_cast<float>(c0.v[i]), static_cast<float>(s0.v[i]),
              static_cast<float>(c1.v[i]), static_cast<float>(s1.v[i]), r0, r1);
    o0.v[i] = static_cast<T>(r0);
    o1.v[i] = static_cast<T>(r1);
  }
  store16_nt(y + yo, o0);
  store16_nt(y + yo + half, o1);
}

// Interleaved, vector path.  Work item = (row, pack j over the whole row);
// a pack holds V/2 pairs.
template <typename T>
__global__ __launch_bounds__(256) void k_rope_inter_vec(const T* x, const T* sn, const T* cs, T* y,
                                                        RopeArgs a, int64_t items) {
  constexpr int V = Pack16<T>::N;
  const int64_t ppr = a.D / V;
  const int64_t it = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (it >= items) return;
  const int64_t j = it % ppr;
  int64_t r = it / ppr;
  const int64_t h = r % a.H;
  r /= a.H;
  const int64_t s = r % a.S;
  const int64_t b = r / a.S;
  const int64_t xo = b * a.xs[0] + s * a.xs[1] + h * a.xs[2] + j * V;
  const int64_t yo = b * a.ys[0] + s * a.ys[1] + h * a.ys[2] + j * V;
  const Pack16<T> xv = load16_nt(x + xo);
  float c[V], sv[V];
  if (a.tcols == a.D) {
    const Pack16<T> cp = load16(cs + s * a.trs + j * V);
    const Pack16<T> sp = load16(sn + s * a.trs + j * V);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      c[i] = static_cast<float>(cp.v[i]);
      sv[i] = static_cast<float>(sp.v[i]);
    }
  } else {
    const T* ct = cs + s * a.trs + j * (V / 2);
    const T* st = sn + s * a.trs + j * (V / 2);
#pragma unroll
    for (int i = 0; i < V / 2; ++i) {
      c[2 * i] = c[2 * i + 1] = static_cast<float>(ct[i]);
      sv[2 * i] = sv[2 * i + 1] = static_cast<float>(st[i]);
    }
  }
  Pack16<T> o;
#pragma unroll
  for (int i = 0; i < V / 2; ++i) {
    float r0, r1;
    rotate<T>(static_cast<float>(xv.v[2 * i]), static_cast<float>(xv.v[2 * i + 1]), c[2 * i],
              sv[2 * i], c[2 * i + 1], sv[2 * i + 1], r0, r1);
    o.v[2 * i] = static_cast<T>(r0);
    o.v[2 * i + 1] = static_cast<T>(r1);
  }
  store16_nt(y + yo, o);
}

// Generic path: one thread per pair, any strides.
template <typename T>
__global__ __launch_bounds__(256) void k_rope_generic(const T* x, const T* sn, const T* cs, T* y,
                                                      RopeArgs a, int interleaved, int64_t pairs) {
  const int64_t half = a.D / 2;
  for (int64_t it = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; it < pairs;
       it += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t i = it % half;
    int64_t r = it / half;
    const int64_t h = r % a.H;
    r /= a.H;
    const int64_t s = r % a.S;
    const int64_t b = r / a.S;
    const int64_t d0 = interleaved ? 2 * i : i;
    const int64_t d1 = interleaved ? 2 * i + 1 : i + half;
    const int64_t xb = b * a.xs[0] + s * a.xs[1] + h * a.xs[2];
    const int64_t yb = b * a.ys[0] + s * a.ys[1] + h * a.ys[2];
    const float x0 = static_cast<float>(x[xb + d0 * a.xs[3]]);
    const float x1 = static_cast<float>(x[xb + d1 * a.xs[3]]);
    const T* ct = cs + s * a.trs;
    const T* st = sn + s * a.trs;
    float c0, s0, c1, s1;
    if (a.tcols == a.D) {
      c0 = static_cast<float>(ct[d0]);
      s0 = static_cast<float>(st[d0]);
      c1 = static_cast<float>(ct[d1]);
      s1 = static_cast<float>(st[d1]);
    } else {
      c0 = c1 = static_cast<float>(ct[i]);
      s0 = s1 = static_cast<float>(st[i]);
    }
    float r0, r1;
    rotate<T>(x0, x1, c0, s0, c1, s1, r0, r1);
    y[yb + d0 * a.ys[3]] = static_cast<T>(r0);
    y[yb + d1 * a.ys[3]] = static_cast<T>(r1);
  }
}

template <typename T>
int run_rope(const RopeArgs& a, const void* xv, const void* sv, const void* cv, int interleaved,
             void* yv, hipStream_t st) {
  const T* x = static_cast<const T*>(xv);
  const T* sn = static_cast<const T*>(sv);
  const T* cs = static_cast<const T*>(cv);
  T* y = static_cast<T*>(yv);
  constexpr int V = Pack16<T>::N;
  const int64_t rows = a.B * a.S * a.H;
  bool vec = a.xs[3] == 1 && a.ys[3] == 1 && aligned16(x) && aligned16(y) && aligned16(sn) &&
             aligned16(cs) && a.trs % V == 0;
  for (int d = 0; d < 3; ++d) vec = vec && a.xs[d] % V == 0 && a.ys[d] % V == 0;
  // An in-place call with different x / y strides would race between pairs.
  if (xv == yv)
    for (int d = 0; d < 4; ++d) vec = vec && a.xs[d] == a.ys[d];
  if (vec && !interleaved && (a.D / 2) % V == 0) {
    const int64_t items = rows * (a.D / 2 / V);
    hipLaunchKernelGGL((k_rope_half_vec<T>), dim3(ceil_div(items, 256)), dim3(256), 0, st, x, sn,
                       cs, y, a, items);
    return check_launch("rope");
  }
  if (vec && interleaved && a.D % V == 0 && (a.tcols == a.D || (a.D / 2) % (V / 2) == 0)) {
    const int64_t items = rows * (a.D / V);
    hipLaunchKernelGGL((k_rope_inter_vec<T>), dim3(ceil_div(items, 256)), dim3(256), 0, st, x, sn,
                       cs, y, a, items);
    return check_launch("rope");
  }
  const int64_t pairs = rows * (a.D / 2);
  int64_t blocks = ceil_div(pairs, 256);
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL((k_rope_generic<T>), dim3(blocks), dim3(256), 0, st, x, sn, cs, y, a,
                     interleaved, pairs);
  return check_launch("rope");
}

}  // namespace
}  // namespace ntops

using namespace ntops;

extern "C" int ntops_rope(int dtype, int64_t B, int64_t S, int64_t H, int64_t D, const void* x,
                          const int64_t* x_strides, const void* sin_table, const void* cos_table,
                          int64_t table_row_stride, int64_t table_cols, int interleaved, void* y,
                          const int64_t* y_strides, void* stream) {
  if (B < 0 || S < 0 || H < 0 || D < 0) return set_error(NTOPS_ERR_INVALID, "rope: negative size");
  if (D % 2 != 0) return set_error(NTOPS_ERR_INVALID, "rope: the embedding dim must be even");
  if (D > 1024) return set_error(NTOPS_ERR_UNSUPPORTED, "rope: embedding dim %lld > 1024", (long long)D);
  if (table_cols != D && table_cols != D / 2)
    return set_error(NTOPS_ERR_INVALID, "rope: tables must have D or D/2 columns");
  if (B == 0 || S == 0 || H == 0 || D == 0) return NTOPS_OK;
  if (!x || !y || !sin_table || !cos_table || !x_strides || !y_strides)
    return set_error(NTOPS_ERR_INVALID, "rope: null pointer");
  RopeArgs a;
  a.B = B;
  a.S = S;
  a.H = H;
  a.D = D;
  for (int d = 0; d < 4; ++d) {
    a.xs[d] = x_strides[d];
    a.ys[d] = y_strides[d];
  }
  a.trs = table_row_stride;
  a.tcols = table_cols;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return dispatch_float16_32(dtype, "rope", [&](auto tag) {
    using T = decltype(tag);
    return run_rope<T>(a, x, sin_table, cos_table, interleaved, y, st);
  });
}
