// Matrix-core building blocks shared by the GEMM and attention kernels
// (gfx950, wave64): operand vector types, the 32x32x16 bf16 / f16 MFMA,
// conflict-free LDS chunk swizzles, direct global -> LDS loads, explicit
// waitcnt and barrier helpers.
#pragma once

#include "dispatch.h"

namespace ntops {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) s16x4 lds_s16x4_t;

// acc += A * B over one 32x32x16 tile.  Called as mfma32<T>(b, a, acc) with
// the B fragment first, so that lane l of the result holds row (l & 31) and
// the four consecutive columns 8q + 4(l >> 5) + 0..3 in acc[4q .. 4q + 3].
template <typename T>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (std::is_same<T, __bf16>::value)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Chunk slot of 16-byte chunk `c` of row `r` in a K-major tile whose rows
// hold BK k values (BK / 8 chunks).  Every form is an involution and gives
// zero SQ_LDS_BANK_CONFLICT for the fragment reads (ds_read_b128, lanes
// 0-31 rows r0 .. r0 + 31 at chunk c, lanes 32-63 the same rows at c + 1,
// c even); for BK = 64, c ^ ((r >> 1 + r >> 4) & 7), c ^ (r & 7) and
// c ^ ((r >> 2) & 7) each conflict on every read (256 vs 414 B per clock).
template <int BK>
__device__ __forceinline__ int kslot(int r, int c) {
  if constexpr (BK == 128)
    return c ^ (r & 15);
  else if constexpr (BK == 64)
    return c ^ ((r >> 1) & 7);
  else
    return c ^ ((r >> 2) & 3);
}
// Chunk slot of chunk `c` of k-row `k` in an M/N-major tile with 16 chunks
// (128 16-bit elements) per k-row.
__device__ __forceinline__ int mnslot(int k, int c) { return c ^ ((k & 3) << 2); }

// s_waitcnt with only the vector-memory counter constrained (<= n).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (((N >> 4) & 3) << 14) | (7 << 4) | (15 << 8));
}

// s_waitcnt lgkmcnt(0) (LDS reads returned), other counters unconstrained.
__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
}

// Workgroup barrier without a memory fence (kernels that use it order their
// LDS traffic with explicit waits); also a scheduling fence for the compiler.
__device__ __forceinline__ void block_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

constexpr uint32_t kOOB = 0x80000000u;  // buffer offset past every resource extent (< 2 GiB)

// 16-byte global -> LDS copy per lane: lane l's 16 bytes land at LDS byte
// address lds_dst + 16 * l.  Written as inline assembly so the compiler does
// not see an LDS store it would have to order against every later LDS read
// (it would wait for all outstanding loads before each K tile's first
// fragment read); the kernel orders it explicitly with vmcnt waits and the
// per-tile barrier.
__device__ __forceinline__ void dma16(u32x4 rsrc, uint32_t lds_dst, uint32_t voffset) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voffset), "s"(rsrc), "{m0}"(lds_dst)
               : "memory");
}

// 32-bit LDS address of a pointer into the block's LDS (wave-uniform).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t*)p)));
}

// Packs 8 fp32 values into an MFMA operand of 8 T elements (one rounding).
template <typename T>
__device__ __forceinline__ u32x4 pack8(const float* v) {
  T h[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = static_cast<T>(v[i]);
  return __builtin_bit_cast(u32x4, h);
}

}  // namespace ntops
