// Row-group machinery shared by the register-resident row kernels
// (rms_norm, layer_norm, softmax).
//
// A row of `cols` elements is owned by WPR wavefronts (WPR in 1..16).  Lane
// `l` of wave `w` (w < WPR within the row) holds the 16-byte packs
//     pack(c) = (c * WPR + w) * 64 + l,   c = 0 .. CHUNKS-1
// so each chunk step of a row reads one contiguous WPR KiB run: fully
// coalesced, 16 B per lane, all CHUNKS loads in flight before first use.
// The row lives in VGPRs between the reduction and the write, so HBM is read
// once and written once.  A block holds RPB rows (blocks have at least 256
// threads); reductions are 64-lane butterflies plus, for WPR > 1, one LDS
// exchange.
#pragma once

#include "common.h"

namespace ntops {

template <int WPR>
struct RowShape {
  static constexpr int kThreads = (64 * WPR < 256) ? 256 : 64 * WPR;
  static constexpr int kRowsPerBlock = kThreads / (64 * WPR);
};

struct RowPos {
  int lane, wave_in_row, row_in_block;
};

// SCALAR: read the wave index through lane 0 so that row indices and row
// base addresses live in SGPRs (scalar address math; required by the buffer
// resources of RowLoader and the branch-free stores).
template <int WPR, bool SCALAR = true>
__device__ __forceinline__ RowPos row_pos() {
  RowPos p;
  p.lane = threadIdx.x & 63;
  const int wave = SCALAR ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : (threadIdx.x >> 6);
  p.wave_in_row = wave % WPR;
  p.row_in_block = wave / WPR;
  return p;
}

template <int WPR>
__device__ __forceinline__ int pack_of(const RowPos& p, int c) {
  return (c * WPR + p.wave_in_row) * 64 + p.lane;
}

// Sum across the WPR waves of a row; `red` is an LDS buffer of
// kRowsPerBlock * WPR floats private to this reduction.
template <int WPR, typename C>
__device__ __forceinline__ C row_sum(C v, C* red, const RowPos& p) {
  v = wave_sum(v);
  if constexpr (WPR == 1) {
    return v;
  } else {
    if (p.lane == 0) red[p.row_in_block * WPR + p.wave_in_row] = v;
    __syncthreads();
    C s = 0;
#pragma unroll
    for (int i = 0; i < WPR; ++i) s += red[p.row_in_block * WPR + i];
    return s;
  }
}

template <int WPR, typename C>
__device__ __forceinline__ C row_max(C v, C* red, const RowPos& p) {
  v = wave_max(v);
  if constexpr (WPR == 1) {
    return v;
  } else {
    if (p.lane == 0) red[p.row_in_block * WPR + p.wave_in_row] = v;
    __syncthreads();
    C s = red[p.row_in_block * WPR];
#pragma unroll
    for (int i = 1; i < WPR; ++i) s = (s > red[p.row_in_block * WPR + i] || s != s) ? s : red[p.row_in_block * WPR + i];
    return s;
  }
}

// Launch shape for a row of `npk` 16-byte packs.  Two packs per lane with
// more waves per row measured faster on MI355X than deep per-lane unrolling
// (e.g. 4096 bf16: 2 packs x 4 waves reaches ~5.9 TB/s, 8 packs x 1 wave
// ~4.9 TB/s): more rows are in flight per CU and the per-row reduction is
// shorter.  One pack per lane goes too far (rms_norm bf16 (16384, 4096) with
// 1 pack x 8 waves: 48.3 against 44.0 us).  Rows wider than 8 packs x 16
// waves use the looped kernels.
struct VecCfg {
  int chunks, wpr;
};
inline bool pick_row_cfg(int64_t npk, VecCfg* cfg) {
  static const VecCfg table[] = {{1, 1}, {2, 1}, {2, 2}, {2, 4}, {2, 8}, {2, 16}, {4, 16}, {8, 16}};
  for (const VecCfg& c : table) {
    if (static_cast<int64_t>(c.chunks) * c.wpr * 64 >= npk) {
      *cfg = c;
      return true;
    }
  }
  return false;
}

// Instantiates MACRO(chunks, wpr) for every entry of pick_row_cfg's table.
#define NTOPS_ROW_CASES(MACRO) \
  MACRO(1, 1)                  \
  MACRO(2, 1)                  \
  MACRO(2, 2)                  \
  MACRO(2, 4)                  \
  MACRO(2, 8)                  \
  MACRO(2, 16)                 \
  MACRO(4, 16)                 \
  MACRO(8, 16)

// The packs of one row that this lane holds; zeros past the row end or for
// rows at or past `rows` (buffer loads against the row's extent: no
// branches).
template <int WPR, typename T, int CHUNKS>
__device__ __forceinline__ void load_row(Pack16<T> (&r)[CHUNKS], const T* base, int64_t stride, int64_t rows,
                                         const RowPos& p, int npk, int64_t row) {
  const bool ok = row < rows;
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(base + (ok ? row : 0) * stride, ok ? npk * 16u : 0u);
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) r[c] = buffer_load16_nt<T>(rs, pack_of<WPR>(p, c) * 16u);
}

// The V per-column parameters (weight or bias, type W) that go with one
// 16-byte pack of the row, kept in their own type from load to use
// (V * sizeof(W) bytes: one 16-byte load for W == T, two for float with a
// 16-bit T).  Loads go through a buffer resource over the parameter row
// (param_rsrc), whose extent is 0 when the parameter is absent: the loads
// then return zeros without touching memory, and no branch surrounds them.
// They keep the default cache policy: every row group re-reads them.
template <typename W, int V>
struct ParamPack {
  static constexpr int kPer = Pack16<W>::N;
  static constexpr int kLoads = V / kPer;
  static_assert(kLoads >= 1 && V % kPer == 0, "parameter type narrower than the row type");
  Pack16<W> q[kLoads];
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, int pk) {
#pragma unroll
    for (int j = 0; j < kLoads; ++j)
      q[j] = __builtin_bit_cast(Pack16<W>, __builtin_amdgcn_raw_buffer_load_b128(
                                                rs, (static_cast<uint32_t>(pk) * kLoads + j) * 16u, 0, 0));
  }
  __device__ __forceinline__ float get(int i) const { return static_cast<float>(q[i / kPer].v[i % kPer]); }
};

// Resource over a parameter row of npk packs of V elements (null: extent 0).
template <int V, typename W>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t param_rsrc(const W* w, int npk) {
  return buffer_rsrc(w, w != nullptr ? static_cast<uint32_t>(npk) * V * static_cast<uint32_t>(sizeof(W)) : 0u);
}

// Sums v[k] over the WPR waves of each of a slot's R rows (one LDS exchange
// and one barrier for all R); `red` holds R * kRowsPerBlock * WPR floats.
template <int WPR, int R>
__device__ __forceinline__ void rows_sum(float (&v)[R], float* red, const RowPos& p) {
  constexpr int RPB = RowShape<WPR>::kRowsPerBlock;
#pragma unroll
  for (int k = 0; k < R; ++k) v[k] = wave_sum(v[k]);
  if constexpr (WPR > 1) {
    if (p.lane == 0)
#pragma unroll
      for (int k = 0; k < R; ++k) red[(k * RPB + p.row_in_block) * WPR + p.wave_in_row] = v[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < R; ++k) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < WPR; ++i) s += red[(k * RPB + p.row_in_block) * WPR + i];
      v[k] = s;
    }
  }
}

// Block-wide sum for the looped (any width) kernels: 256 threads.
template <typename C>
__device__ __forceinline__ C block_sum256(C v, C* red4) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red4[wave] = v;
  __syncthreads();
  return red4[0] + red4[1] + red4[2] + red4[3];
}

template <typename C>
__device__ __forceinline__ C block_max256(C v, C* red4) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red4[wave] = v;
  __syncthreads();
  C m = red4[0];
#pragma unroll
  for (int i = 1; i < 4; ++i) m = (m > red4[i] || m != m) ? m : red4[i];
  return m;
}

}  // namespace ntops
