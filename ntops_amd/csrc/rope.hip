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
//
// Two tensors in one launch (q and k of an attention layer, which share the
// position tables): the grid walks every row of tensor 0 and then every row
// of tensor 1, each with its own pointers and strides (a wave-uniform
// branch picks the tensor); the 2 * S * D table bytes stay L2-resident for
// both.  A single tensor is the case of an empty tensor 1.
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

// One tensor's description: (B, S, H, D) with element strides.
struct RopeTensor {
  const void* x;
  void* y;
  int64_t H;
  int64_t xs[4], ys[4];
};

struct RopeArgs {
  int64_t B, S, D;
  RopeTensor t[2];  // t[1].H == 0: a single tensor
  int64_t trs;      // table row stride
  int64_t tcols;    // D / 2 or D
};

// Element offsets of row r = (b, s, h) of tensor d (I: index type, 32-bit
// whenever the item count allows, so the divisions are cheap).
template <typename I>
__device__ __forceinline__ void rope_row(const RopeArgs& a, const RopeTensor& d, I r, I& s, int64_t& xo,
                                         int64_t& yo) {
  const I h = r % static_cast<I>(d.H);
  r /= static_cast<I>(d.H);
  s = r % static_cast<I>(a.S);
  const I b = r / static_cast<I>(a.S);
  xo = b * d.xs[0] + s * d.xs[1] + h * d.xs[2];
  yo = b * d.ys[0] + s * d.ys[1] + h * d.ys[2];
}

// Every kernel below walks tensor 0's items and then tensor 1's: its body
// (a lambda taking the tensor and the item index within it) is called from
// two branches, uniform except in the one wave that straddles the boundary,
// so each inlined copy sees that tensor's strides as scalars.

// Half-rotation, vector path.  Work item = (row, pack j of the first half).
template <typename T, typename I>
__global__ __launch_bounds__(256) void k_rope_half_vec(const T* sn, const T* cs, RopeArgs a, I items0, I items) {
  constexpr int V = Pack16<T>::N;
  const I half = static_cast<I>(a.D / 2);
  const I ppr = half / V;  // packs per half row
  const I it = static_cast<I>(block_id()) * 256 + threadIdx.x;  // blocks_2d grid
  if (it >= items) return;
  auto body = [&](const RopeTensor& d, I li) {
    const I j = li % ppr;
    I s;
    int64_t xo, yo;
    rope_row<I>(a, d, li / ppr, s, xo, yo);
    const T* x = static_cast<const T*>(d.x);
    T* y = static_cast<T*>(d.y);
    xo += j * V;
    yo += j * V;
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
      rotate<T>(static_cast<float>(x0.v[i]), static_cast<float>(x1.v[i]), static_cast<float>(c0.v[i]),
                static_cast<float>(s0.v[i]), static_cast<float>(c1.v[i]), static_cast<float>(s1.v[i]), r0, r1);
      o0.v[i] = static_cast<T>(r0);
      o1.v[i] = static_cast<T>(r1);
    }
    store16_nt(y + yo, o0);
    store16_nt(y + yo + half, o1);
  };
  if (it < items0)
    body(a.t[0], it);
  else
    body(a.t[1], it - items0);
}

// Interleaved, vector path.  Work item = (row, pack j over the whole row);
// a pack holds V/2 pairs.
template <typename T, typename I>
__global__ __launch_bounds__(256) void k_rope_inter_vec(const T* sn, const T* cs, RopeArgs a, I items0, I items) {
  constexpr int V = Pack16<T>::N;
  const I ppr = static_cast<I>(a.D / V);
  const I it = static_cast<I>(block_id()) * 256 + threadIdx.x;  // blocks_2d grid
  if (it >= items) return;
  auto body = [&](const RopeTensor& d, I li) {
    const I j = li % ppr;
    I s;
    int64_t xo, yo;
    rope_row<I>(a, d, li / ppr, s, xo, yo);
    const T* x = static_cast<const T*>(d.x);
    T* y = static_cast<T*>(d.y);
    xo += j * V;
    yo += j * V;
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
      rotate<T>(static_cast<float>(xv.v[2 * i]), static_cast<float>(xv.v[2 * i + 1]), c[2 * i], sv[2 * i],
                c[2 * i + 1], sv[2 * i + 1], r0, r1);
      o.v[2 * i] = static_cast<T>(r0);
      o.v[2 * i + 1] = static_cast<T>(r1);
    }
    store16_nt(y + yo, o);
  };
  if (it < items0)
    body(a.t[0], it);
  else
    body(a.t[1], it - items0);
}

// Generic path: one thread per pair, any strides (64-bit indices).
template <typename T>
__global__ __launch_bounds__(256) void k_rope_generic(const T* sn, const T* cs, RopeArgs a, int interleaved,
                                                      int64_t pairs0, int64_t pairs) {
  using I = int64_t;
  const int64_t half = a.D / 2;
  for (int64_t it = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; it < pairs;
       it += static_cast<int64_t>(gridDim.x) * 256) {
    auto body = [&](const RopeTensor& d, I li) {
      const int64_t i = li % half;
      int64_t s, xb, yb;
      rope_row<I>(a, d, li / half, s, xb, yb);
      const T* x = static_cast<const T*>(d.x);
      T* y = static_cast<T*>(d.y);
      const int64_t d0 = interleaved ? 2 * i : i;
      const int64_t d1 = interleaved ? 2 * i + 1 : i + half;
      const float x0 = static_cast<float>(x[xb + d0 * d.xs[3]]);
      const float x1 = static_cast<float>(x[xb + d1 * d.xs[3]]);
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
      y[yb + d0 * d.ys[3]] = static_cast<T>(r0);
      y[yb + d1 * d.ys[3]] = static_cast<T>(r1);
    };
    if (it < pairs0)
      body(a.t[0], it);
    else
      body(a.t[1], it - pairs0);
  }
}

template <typename T>
int run_rope(const RopeArgs& a, const void* sv, const void* cv, int interleaved, hipStream_t st) {
  const T* sn = static_cast<const T*>(sv);
  const T* cs = static_cast<const T*>(cv);
  constexpr int V = Pack16<T>::N;
  const int64_t rows0 = a.B * a.S * a.t[0].H;
  const int64_t rows = rows0 + a.B * a.S * a.t[1].H;
  bool vec = aligned16(sn) && aligned16(cs) && a.trs % V == 0;
  for (int t = 0; t < 2; ++t) {
    const RopeTensor& d = a.t[t];
    if (d.H == 0) continue;
    vec = vec && d.xs[3] == 1 && d.ys[3] == 1 && aligned16(d.x) && aligned16(d.y);
    for (int k = 0; k < 3; ++k) vec = vec && d.xs[k] % V == 0 && d.ys[k] % V == 0;
    // An in-place call with different x / y strides would race between pairs.
    if (d.x == d.y)
      for (int k = 0; k < 4; ++k) vec = vec && d.xs[k] == d.ys[k];
  }
  const bool half_vec = vec && !interleaved && (a.D / 2) % V == 0;
  const bool inter_vec = vec && interleaved && a.D % V == 0 && (a.tcols == a.D || (a.D / 2) % (V / 2) == 0);
  if (half_vec || inter_vec) {
    const int64_t per_row = half_vec ? a.D / 2 / V : a.D / V;
    const int64_t items0 = rows0 * per_row, items = rows * per_row;
    const dim3 grid = blocks_2d(ceil_div(items, 256));
    if (items < 0x7fffffffLL) {
      using I = uint32_t;
      if (half_vec)
        hipLaunchKernelGGL((k_rope_half_vec<T, I>), grid, dim3(256), 0, st, sn, cs, a, static_cast<I>(items0),
                           static_cast<I>(items));
      else
        hipLaunchKernelGGL((k_rope_inter_vec<T, I>), grid, dim3(256), 0, st, sn, cs, a, static_cast<I>(items0),
                           static_cast<I>(items));
    } else {
      using I = int64_t;
      if (half_vec)
        hipLaunchKernelGGL((k_rope_half_vec<T, I>), grid, dim3(256), 0, st, sn, cs, a, items0, items);
      else
        hipLaunchKernelGGL((k_rope_inter_vec<T, I>), grid, dim3(256), 0, st, sn, cs, a, items0, items);
    }
    return check_launch("rope");
  }
  const int64_t pairs0 = rows0 * (a.D / 2), pairs = rows * (a.D / 2);
  int64_t blocks = ceil_div(pairs, 256);
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL((k_rope_generic<T>), dim3(blocks), dim3(256), 0, st, sn, cs, a, interleaved, pairs0, pairs);
  return check_launch("rope");
}

int check_rope(int64_t B, int64_t S, int64_t H, int64_t D, int64_t table_cols) {
  if (B < 0 || S < 0 || H < 0 || D < 0) return set_error(NTOPS_ERR_INVALID, "rope: negative size");
  if (D % 2 != 0) return set_error(NTOPS_ERR_INVALID, "rope: the embedding dim must be even");
  if (D > 1024) return set_error(NTOPS_ERR_UNSUPPORTED, "rope: embedding dim %lld > 1024", (long long)D);
  if (table_cols != D && table_cols != D / 2)
    return set_error(NTOPS_ERR_INVALID, "rope: tables must have D or D/2 columns");
  return NTOPS_OK;
}

}  // namespace
}  // namespace ntops

using namespace ntops;

extern "C" int ntops_rope(int dtype, int64_t B, int64_t S, int64_t H, int64_t D, const void* x,
                          const int64_t* x_strides, const void* sin_table, const void* cos_table,
                          int64_t table_row_stride, int64_t table_cols, int interleaved, void* y,
                          const int64_t* y_strides, void* stream) {
  if (int e = check_rope(B, S, H, D, table_cols)) return e;
  if (B == 0 || S == 0 || H == 0 || D == 0) return NTOPS_OK;
  if (!x || !y || !sin_table || !cos_table || !x_strides || !y_strides)
    return set_error(NTOPS_ERR_INVALID, "rope: null pointer");
  RopeArgs a{};
  a.B = B;
  a.S = S;
  a.D = D;
  a.t[0].x = x;
  a.t[0].y = y;
  a.t[0].H = H;
  for (int d = 0; d < 4; ++d) {
    a.t[0].xs[d] = x_strides[d];
    a.t[0].ys[d] = y_strides[d];
  }
  a.t[1] = a.t[0];
  a.t[1].H = 0;
  a.trs = table_row_stride;
  a.tcols = table_cols;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return dispatch_float16_32(dtype, "rope", [&](auto tag) {
    using T = decltype(tag);
    return run_rope<T>(a, sin_table, cos_table, interleaved, st);
  });
}

extern "C" int ntops_rope_qk(int dtype, int64_t B, int64_t S, int64_t Hq, int64_t Hk, int64_t D, const void* q,
                             const int64_t* q_strides, const void* k, const int64_t* k_strides,
                             const void* sin_table, const void* cos_table, int64_t table_row_stride,
                             int64_t table_cols, int interleaved, void* q_out, const int64_t* q_out_strides,
                             void* k_out, const int64_t* k_out_strides, void* stream) {
  if (Hk < 0) return set_error(NTOPS_ERR_INVALID, "rope_qk: negative size");
  if (int e = check_rope(B, S, Hq, D, table_cols)) return e;
  if (B == 0 || S == 0 || Hq + Hk == 0 || D == 0) return NTOPS_OK;
  if (!sin_table || !cos_table || (Hq > 0 && (!q || !q_out || !q_strides || !q_out_strides)) ||
      (Hk > 0 && (!k || !k_out || !k_strides || !k_out_strides)))
    return set_error(NTOPS_ERR_INVALID, "rope_qk: null pointer");
  RopeArgs a{};
  a.B = B;
  a.S = S;
  a.D = D;
  const void* xs[2] = {q, k};
  void* ys[2] = {q_out, k_out};
  const int64_t* xst[2] = {q_strides, k_strides};
  const int64_t* yst[2] = {q_out_strides, k_out_strides};
  const int64_t hs[2] = {Hq, Hk};
  for (int t = 0; t < 2; ++t) {
    a.t[t].H = hs[t];
    if (hs[t] == 0) continue;
    a.t[t].x = xs[t];
    a.t[t].y = ys[t];
    for (int d = 0; d < 4; ++d) {
      a.t[t].xs[d] = xst[t][d];
      a.t[t].ys[d] = yst[t][d];
    }
  }
  a.trs = table_row_stride;
  a.tcols = table_cols;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return dispatch_float16_32(dtype, "rope_qk", [&](auto tag) {
    using T = decltype(tag);
    return run_rope<T>(a, sin_table, cos_table, interleaved, st);
  });
}
