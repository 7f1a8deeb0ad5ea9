// Rows wider than the register-resident shapes of rowcommon.h (more than
// 8 packs x 16 waves = 8192 16-byte packs: 65536 16-bit or 32768 fp32
// elements): 1024-thread blocks, one per CU, each walking rows
// blockIdx.x, blockIdx.x + gridDim.x, ...  Packs 0 .. 8191 of a row live in
// VGPRs exactly as in the 8 x 16 shape (lane t holds packs c * 1024 + t);
// the rest of the row, up to 10176 packs (159 KiB), is staged in LDS by
// direct global -> LDS loads (buffer_load_dwordx4 ... lds, 1 KiB per wave
// instruction, no VGPR round trip).  Every pass over the row then reads
// VGPRs and LDS, so HBM is read once and written once, as for narrower rows
// (the looped kernels re-read the row from L2 / HBM on every pass).
// A block's output pass over one row also loads its next row into the same
// VGPRs and LDS, piece by piece behind the stores, so the CU's reads of one
// row overlap its writes of the previous one (one row per CU at a time
// would otherwise leave HBM idle in one direction during each phase).
// Each wave reads only the LDS runs it loads itself (run j, packs
// 64 j .. 64 j + 63, by wave j % 16 in the q-loop below), so no barrier
// orders a run's refill after its last read.
// Widest row served: 18368 packs (146944 16-bit, 73472 fp32 elements);
// rows wider still take the looped kernels.
#pragma once

#include "mfma.h"
#include "rowcommon.h"

namespace ntops {

constexpr int kWideThreads = 1024;
constexpr int kWideWaves = kWideThreads / 64;
constexpr int kWideRegChunks = 8;
constexpr int kWideRegPacks = kWideRegChunks * kWideThreads;  // 8192
constexpr int kWideLdsPacks = 159 * 64;                         // 10176: 159 KiB in 1 KiB runs

inline bool wide_row_fits(int64_t npk) { return npk > kWideRegPacks && npk <= kWideRegPacks + kWideLdsPacks; }
// LDS the row's staged part takes: whole 1 KiB runs (one DMA instruction each).
inline unsigned wide_lds_bytes(int64_t npk) {
  return static_cast<unsigned>((npk - kWideRegPacks + 63) / 64 * 1024);
}

// One row: packs in VGPRs plus the staged rest in LDS (`lds`, nl packs).
template <typename T>
struct WideRow {
  Pack16<T> r[kWideRegChunks];
  const char* lds;
  int nl;
};

// One row's sources: the buffer resource of its register packs and the
// DMA resource of its staged runs (extent: the row; zeros land past it).
struct WideSrc {
  __amdgpu_buffer_rsrc_t rs;
  u32x4 dma;
};

template <typename T>
__device__ __forceinline__ WideSrc wide_src(const T* base, int npk) {
  WideSrc s;
  s.rs = buffer_rsrc(base, npk * 16u);
  const uint64_t addr = reinterpret_cast<uint64_t>(base);
  s.dma.x = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr));
  s.dma.y = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr >> 32) & 0xffffu);
  s.dma.z = static_cast<uint32_t>(npk) * 16u;
  s.dma.w = 0x00020000u;
  return s;
}

// Register chunk c of the row (this thread's pack c * 1024 + t).
template <typename T>
__device__ __forceinline__ void wide_load_chunk(WideRow<T>& w, const WideSrc& s, int c) {
  w.r[c] = buffer_load16_nt<T>(s.rs, (c * kWideThreads + threadIdx.x) * 16u);
}

// Staged run j of the row (packs kWideRegPacks + 64 j ..) into LDS at
// l0 + 1024 j, by the calling wave.
__device__ __forceinline__ void wide_dma_run(const WideSrc& s, uint32_t l0, int j) {
  const uint32_t voff = (static_cast<uint32_t>(kWideRegPacks + j * 64) + (threadIdx.x & 63)) * 16u;
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen nt lds" : : "v"(voff), "s"(s.dma), "{m0}"(l0 + j * 1024u) : "memory");
}

// Loads a block's first row (npk packs at `base`, 16-byte aligned) -- the
// staged runs by DMA into `lds`, then the VGPR packs by buffer loads -- and
// makes the row's first pass: visit(pack) for this thread's staged packs as
// soon as the DMA has landed (the register loads still in flight), then for
// its register packs.
template <typename T, typename Visit>
__device__ __forceinline__ void wide_load(WideRow<T>& w, const T* base, int npk, char* lds, Visit visit) {
  const WideSrc s = wide_src(base, npk);
  w.nl = npk - kWideRegPacks;
  w.lds = lds;
  const int runs = (w.nl + 63) / 64;
  const uint32_t l0 = lds_addr(lds);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  for (int j = wave; j < runs; j += kWideWaves) wide_dma_run(s, l0, j);
#pragma unroll
  for (int c = 0; c < kWideRegChunks; ++c) wide_load_chunk(w, s, c);
  wait_vmcnt<kWideRegChunks>();  // this wave's runs have landed
  for (int q = threadIdx.x; q < w.nl; q += kWideThreads) visit(wide_lds_pack(w, q));
  wait_vmcnt<0>();
#pragma unroll
  for (int c = 0; c < kWideRegChunks; ++c) visit(w.r[c]);
}

// Hides the row's register packs from the compiler's value tracking: the
// next pass converts them again instead of keeping every converted element
// of the previous pass live, which does not fit beside the rest of a
// 1024-thread block's state (128 VGPRs).
template <typename T>
__device__ __forceinline__ void wide_launder(WideRow<T>& w) {
#pragma unroll
  for (int c = 0; c < kWideRegChunks; ++c) {
    u32x4 u = __builtin_bit_cast(u32x4, w.r[c]);
    asm volatile("" : "+v"(u));
    w.r[c] = __builtin_bit_cast(Pack16<T>, u);
  }
}

// Staged pack q (0 <= q < nl) of the row.
template <typename T>
__device__ __forceinline__ Pack16<T> wide_lds_pack(const WideRow<T>& w, int q) {
  return __builtin_bit_cast(Pack16<T>, *reinterpret_cast<const u32x4*>(w.lds + q * 16));
}

// The output pass over the row in `w`: emit(pack, index, fetch(index)) for
// every pack of this thread, the staged runs first, then the register
// chunks.  fetch(index) loads what the output of a pack needs besides the
// pack (the weight / bias packs; an empty struct if nothing); it is issued D
// packs ahead of its use within each part, so D + 1 parameter loads per
// thread overlap instead of each waiting out an L2 round trip before its
// pack can be written.  With `more`, the block's next row (at `next`) is
// loaded into the same LDS and VGPRs as the pass goes -- each staged run
// right after this wave has read it (lgkmcnt 0: the read has returned before
// the DMA overwrites it), each register chunk right after its outputs are
// stored -- and its first pass made: visit(pack) over the staged packs once
// their DMA has landed, while the register loads are in flight, then over
// the register packs.  Returns once the next row has landed.
template <int D, typename T, typename Fetch, typename Emit, typename Visit>
__device__ __forceinline__ void wide_emit_and_load(WideRow<T>& w, bool more, const T* next, int npk, Fetch fetch,
                                                   Emit emit, Visit visit) {
  static_assert(D >= 0 && D <= 2, "prefetch depth");
  using P = decltype(fetch(0));
  const int t = threadIdx.x;
  const WideSrc s = wide_src(next, npk);
  P p1{}, p2{};
  // pack pk, the pack `stride` further on fetched D ahead (fetches past the
  // row read zeros and are not used)
  auto step = [&](const Pack16<T>& v, int pk, int stride) {
    if constexpr (D == 0) {
      emit(v, pk, fetch(pk));
    } else if constexpr (D == 1) {
      const P cur = p1;
      p1 = fetch(pk + stride);
      emit(v, pk, cur);
    } else {
      const P cur = p1;
      p1 = p2;
      p2 = fetch(pk + 2 * stride);
      emit(v, pk, cur);
    }
  };
  auto prime = [&](int pk, int stride) {
    if constexpr (D >= 1) p1 = fetch(pk);
    if constexpr (D >= 2) p2 = fetch(pk + stride);
  };
  const uint32_t l0 = lds_addr(w.lds);
  int j = __builtin_amdgcn_readfirstlane(t >> 6);
  prime(kWideRegPacks + t, kWideThreads);
  for (int q = t; q < w.nl; q += kWideThreads, j += kWideWaves) {
    step(wide_lds_pack(w, q), kWideRegPacks + q, kWideThreads);
    if (more) {
      wait_lgkmcnt0();
      wide_dma_run(s, l0, j);
    }
  }
  prime(t, kWideThreads);
#pragma unroll
  for (int c = 0; c < kWideRegChunks; ++c) {
    step(w.r[c], c * kWideThreads + t, kWideThreads);
    if (more) wide_load_chunk(w, s, c);
    // one chunk at a time: hoisting every chunk's parameter loads above the
    // stores would need more VGPRs than the 1024-thread block has
    __builtin_amdgcn_sched_barrier(0);
  }
  if (more) {
    // at most the last 2 * 8 vector-memory operations (each chunk's store
    // and load, plus any parameter loads after them) are still in flight:
    // this wave's runs have landed
    wait_vmcnt<2 * kWideRegChunks>();
    for (int q = t; q < w.nl; q += kWideThreads) visit(wide_lds_pack(w, q));
    wait_vmcnt<0>();
#pragma unroll
    for (int c = 0; c < kWideRegChunks; ++c) visit(w.r[c]);
  } else {
    wait_vmcnt<0>();
  }
}

// Blocks for n rows: one per CU (each holds a whole row), at most n.
inline unsigned wide_grid(int64_t n) {
  const int64_t cus = cu_count_cached();
  return static_cast<unsigned>(n < cus ? n : cus);
}

// Block-wide reduction of one value per thread (op commutative); `red`
// holds kWideWaves values.  Every thread gets the result, combined in wave
// order.
template <typename Op>
__device__ __forceinline__ float wide_reduce(float v, float* red, Op op) {
  v = wave_reduce(v, op);
  __syncthreads();  // red may still be read by an earlier reduction
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = red[0];
#pragma unroll
  for (int i = 1; i < kWideWaves; ++i) s = op(s, red[i]);
  return s;
}

// Sets the dynamic-LDS limit of a wide kernel (above the 64 KiB default)
// on its first launch; `done` is a static of the launching instantiation.
template <typename K>
int wide_lds_attr(K kern, bool& done) {
  if (!done) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            kWideLdsPacks * 16) != hipSuccess)
      return set_error(NTOPS_ERR_HIP, "row kernel: cannot reserve %d bytes of LDS", kWideLdsPacks * 16);
    done = true;
  }
  return NTOPS_OK;
}

}  // namespace ntops
