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

template <int WPR>
__device__ __forceinline__ RowPos row_pos() {
  RowPos p;
  p.lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
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
// shorter.  Rows wider than 8 packs x 16 waves use the looped kernels.
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

// Loads V consecutive elements of type W (16-byte aligned) as float.
template <typename W, int V>
__device__ __forceinline__ void load_as_float(const W* p, float (&out)[V]) {
  constexpr int PER = 16 / sizeof(W);
  static_assert(V % PER == 0, "V must be a multiple of the pack width");
#pragma unroll
  for (int j = 0; j < V / PER; ++j) {
    Pack16<W> pk = load16(p + j * PER);
#pragma unroll
    for (int i = 0; i < PER; ++i) out[j * PER + i] = static_cast<float>(pk.v[i]);
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
