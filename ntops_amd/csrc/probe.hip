// Matrix-core rate probe: the bf16 MFMA rate this GPU sustains under a
// full-chip load, which bench.py reports as the measured ceiling of the
// matrix-bound kernels (as a plain streaming copy is for the bandwidth-bound
// ones).  The dense peak assumes the 2.4 GHz top shader clock; under a
// full matrix load the clock settles lower, so the probe is the attainable
// rate.
//
// Each wave keeps 8 independent 32x32 fp32 accumulators and 16 operand
// fragments of bf16 values in [-1, 1) (different in every lane, register and
// wave) and runs `iters` rounds of 8 v_mfma_f32_32x32x16_bf16; consecutive
// rounds pair the accumulators with different operand fragments, so the
// multiplier inputs change every instruction as they do in a GEMM.  Each
// wave then stores one checksum, so no MFMA is dead code.
#include "mfma.h"

namespace ntops {
namespace {

constexpr int kProbeAcc = 8;

__device__ __forceinline__ uint32_t probe_hash(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return x;
}

// 8 bf16 values in [-1, 1) from a hash of `seed`.
__device__ __forceinline__ u32x4 probe_operand(uint32_t seed) {
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e)
    v[e] = static_cast<float>(probe_hash(seed * 8u + e) & 0xffffu) * (2.0f / 65536.0f) - 1.0f;
  return pack8<__bf16>(v);
}

__global__ __launch_bounds__(256) void k_mfma_probe(int64_t iters, float* out) {
  const uint32_t wave = blockIdx.x * 4u + (threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  u32x4 a[kProbeAcc], b[kProbeAcc];
#pragma unroll
  for (int j = 0; j < kProbeAcc; ++j) {
    a[j] = probe_operand((wave * 64u + lane) * 32u + 2u * j);
    b[j] = probe_operand((wave * 64u + lane) * 32u + 2u * j + 1u);
  }
  f32x16 acc[kProbeAcc];
#pragma unroll
  for (int j = 0; j < kProbeAcc; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;
  for (int64_t it = 0; it < iters; it += 2) {
#pragma unroll
    for (int j = 0; j < kProbeAcc; ++j) acc[j] = mfma32<__bf16>(b[j], a[j], acc[j]);
#pragma unroll
    for (int j = 0; j < kProbeAcc; ++j)
      acc[j] = mfma32<__bf16>(b[(j + 3) % kProbeAcc], a[(j + 1) % kProbeAcc], acc[j]);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kProbeAcc; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[j][e];
  if (lane == 0) out[wave] = s;
}

}  // namespace
}  // namespace ntops

using namespace ntops;

extern "C" int ntops_mfma_rate_probe(int64_t workgroups, int64_t iters, float* out, void* stream) {
  if (workgroups < 1 || workgroups > (int64_t(1) << 20) || iters < 2 || iters > (int64_t(1) << 30) || iters % 2)
    return set_error(NTOPS_ERR_INVALID, "mfma_rate_probe: workgroups in [1, 2^20], even iters in [2, 2^30]");
  if (out == nullptr) return set_error(NTOPS_ERR_INVALID, "mfma_rate_probe: null output");
  note_kernel("mfma_probe");
  hipLaunchKernelGGL(k_mfma_probe, dim3(static_cast<unsigned>(workgroups)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), iters, out);
  return check_launch("mfma_rate_probe");
}
