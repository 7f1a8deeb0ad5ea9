// Rows wider than the register-resident shapes of rowcommon.h (more than
// 8 packs x 16 waves = 8192 16-byte packs: 65536 16-bit or 32768 fp32
// elements): one 1024-thread block per row.  Packs 0 .. 8191 live in VGPRs
// exactly as in the 8 x 16 shape (lane t holds packs c * 1024 + t); the rest
// of the row, up to 10176 packs (159 KiB), is staged in LDS by direct
// global -> LDS loads (buffer_load_dwordx4 ... lds, 1 KiB per wave
// instruction, no VGPR round trip).  Every pass over the row then reads
// VGPRs and LDS, so HBM is read once and written once, as for narrower rows
// (the looped kernels re-read the row from L2 / HBM on every pass).
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

// Loads row `row` (npk packs at `base`, 16-byte aligned): the VGPR packs by
// buffer loads, the rest by DMA into `lds`; returns once the whole row is in
// VGPRs and LDS and visible to every wave of the block.
template <typename T>
__device__ __forceinline__ void wide_load(WideRow<T>& w, const T* base, int npk, char* lds) {
  const int t = threadIdx.x;
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(base, npk * 16u);
#pragma unroll
  for (int c = 0; c < kWideRegChunks; ++c) w.r[c] = buffer_load16_nt<T>(rs, (c * kWideThreads + t) * 16u);
  w.nl = npk - kWideRegPacks;
  w.lds = lds;
  // the staged part: 1 KiB run j (packs kWideRegPacks + 64 j ..) by wave j % 16
  u32x4 v;
  const uint64_t addr = reinterpret_cast<uint64_t>(base);
  v.x = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr));
  v.y = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr >> 32) & 0xffffu);
  v.z = static_cast<uint32_t>(npk) * 16u;  // num_records: past the row, zeros land in LDS
  v.w = 0x00020000u;
  const int runs = (w.nl + 63) / 64;
  const uint32_t l0 = lds_addr(lds);
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  for (int j = wave; j < runs; j += kWideWaves) {
    const uint32_t voff = (static_cast<uint32_t>(kWideRegPacks + j * 64) + (t & 63)) * 16u;
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen nt lds" : : "v"(voff), "s"(v), "{m0}"(l0 + j * 1024u) : "memory");
  }
  wait_vmcnt<0>();
  __syncthreads();
}

// Staged pack q (0 <= q < nl) of the row.
template <typename T>
__device__ __forceinline__ Pack16<T> wide_lds_pack(const WideRow<T>& w, int q) {
  return __builtin_bit_cast(Pack16<T>, *reinterpret_cast<const u32x4*>(w.lds + q * 16));
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
