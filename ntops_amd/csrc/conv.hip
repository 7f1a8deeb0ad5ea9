// conv2d: out[n, k, p, q] = bias[k] + sum_{c, r, s} x[n, c, ih, iw] * w[k, c, r, s]
// with ih = p * sh - ph + r * dh, iw = q * sw - pw + s * dw (zero outside the
// image), fp32 accumulation and one rounding of the biased sum.
//
// Reference: kernels/conv2d.py:12-104 (im2col arrangement of the padded,
// strided, dilated input over the mm tiling; bias added to the fp32 product,
// lines 102-104), torch/conv2d.py:8-53 (argument forms, output size from
// torch/pooling.py:4-19, groups == 1).
//
// Four paths:
//  * channels-last implicit GEMM (bf16 / fp16, C a multiple of 32, any
//    stride and dilation): the weights are reordered once per call to
//    wt[k][((cb * R + r) * S + s) * 32 + ci] (c = 32 cb + ci: the taps of a
//    32-channel block are consecutive in k, so the GEMM's consecutive K
//    tiles re-read the same pixels while they are in L2) and each image is
//    copied once into a
//    caller-owned workspace as a zero-padded channels-last image
//    xt[hh][ww][c] = x[c][hh - ph][ww - pw] of Hp = (P - 1) sh + (R - 1) dh + 1
//    rows of Wp = (Q - 1) sw + (S - 1) dw + 1 pixels, so that output pixel
//    (p, q) under tap (r, s) reads the C contiguous channels at
//    xt[p sh + r dh][q sw + s dw]: the GEMM's B operand is K-major with one
//    row per output pixel (its base fixed for the tile) and one scalar offset
//    per 32-channel K tile, with no bounds tests (the padding is in the copy);
//  * implicit GEMM over shifted planes (stride 1, bf16 / fp16, output rows of a multiple of 8
//    pixels): each image is copied once into a caller-owned workspace as S
//    column-shifted, zero-padded planes xs[s][c][row][q] =
//    x[c][row - ph][q + s * dw - pw] with Hp = P + (R - 1) * dh rows of Q
//    pixels, so that the unfolded row (c, r, s) is the contiguous run
//    xs[s][c][r * dh ..][0 ..) of P * Q pixels -- the GEMM's operand loader
//    computes each k-row's base from (c, r, s) instead of reading a
//    materialised unfold (3x the input instead of R * S x);
//  * GEMM path (when C * R * S and K are large enough to feed the matrix
//    cores): the input of a chunk of images is unfolded into a caller-owned
//    workspace col[n][c * R * S + r * S + s][p * Q + q] (k-rows padded to a
//    multiple of 8 pixels; CRS padded to KP, a multiple of 8, with zero
//    rows), then ntops_gemm computes, per image,
//    out_n = W (K x KP) . col_n (KP x PQ) + bias, with W shared across the
//    batch (batch stride 0) and the bias as a C operand broadcast along the
//    pixels (strides 0, 1, 0).  W is read in place when its rows are KP
//    contiguous elements at 16-byte alignment, else copied into the
//    workspace as K x KP with zero columns past CRS (e.g. a 3-channel 7 x 7
//    stem, CRS = 147).  bf16 / fp16 run on MFMA, fp32 on the IEEE FMA GEMM.
//  * direct path (small channel counts, any strides): one thread per output
//    element, fp32 accumulation.
#include <atomic>

#include "gemm.h"

namespace ntops {
namespace {

// Scratch of ntops_conv2d_noalloc: stands in for the caller's workspace (the
// shifted planes or the unfolded input of a chunk of images).  Each GPU holds
// its own copy at its own address for the life of the process; host code
// reaches it only through conv_scratch(), never through the symbol's name
// (which on the host is a stand-in, not a device address).  Every byte a call
// reads is written by the same call first (its shift / unfold / copy kernels, or the zero fill of the pad rows), so no
// clearing is needed; calls that overlap on one GPU share it and race.
constexpr int64_t kConvScratchBytes = NTOPS_CONV2D_NOALLOC_MAX_SCRATCH;
static __device__ __align__(256) char scratch[kConvScratchBytes];

// Device address of this device's scratch (looked up once per device with
// that device current), or nullptr with the error recorded.
void* conv_scratch() {
  static std::atomic<void*> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    set_error(NTOPS_ERR_HIP, "conv2d_noalloc: no current HIP device");
    return nullptr;
  }
  void* p = cache[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error(NTOPS_ERR_HIP, "conv2d_noalloc: scratch address lookup failed: %s", hipGetErrorString(e));
      return nullptr;
    }
    cache[dev].store(p, std::memory_order_release);
  }
  return p;
}

struct ConvArgs {
  const void* x;
  const void* w;
  const void* bias;
  void* out;
  int64_t xs[4], ws[4], os[4], bs;
  int N, C, H, W, K, R, S, P, Q;
  int sh, sw, ph, pw, dh, dw;
};

// Output plane rows of pq pixels from rows of ld pixels (image i, channel
// k: src[(i K + k) ld + p] -> dst[i os0 + k os1 + p]), one element per
// thread per step of a grid-stride loop (the grid is capped by grid_for).
template <typename T>
__global__ __launch_bounds__(256) void k_conv_rows_out(const T* src, int64_t ld, T* dst, int64_t os0,
                                                       int64_t os1, int64_t K, int64_t pq, int64_t total) {
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t p = e % pq, r = e / pq;  // r = i K + k
    const int64_t i = r / K, k = r - i * K;
    dst[i * os0 + k * os1 + p] = src[r * ld + p];
  }
}

template <typename T>
__global__ __launch_bounds__(256) void k_conv_direct(ConvArgs a, int64_t total) {
  using O = typename OpMath<T>::T_;
  const T* x = static_cast<const T*>(a.x);
  const T* w = static_cast<const T*>(a.w);
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    // i -> (n, k, p, q) with q fastest, so neighbouring threads read
    // neighbouring input pixels and share one weight
    const int q = static_cast<int>(i % a.Q);
    int64_t t = i / a.Q;
    const int p = static_cast<int>(t % a.P);
    t /= a.P;
    const int k = static_cast<int>(t % a.K);
    const int n = static_cast<int>(t / a.K);
    float acc = 0.f;
    const T* xn = x + n * a.xs[0];
    const T* wk = w + k * a.ws[0];
    for (int c = 0; c < a.C; ++c) {
      for (int r = 0; r < a.R; ++r) {
        const int ih = p * a.sh - a.ph + r * a.dh;
        if (ih < 0 || ih >= a.H) continue;
        for (int s = 0; s < a.S; ++s) {
          const int iw = q * a.sw - a.pw + s * a.dw;
          if (iw < 0 || iw >= a.W) continue;
          acc += static_cast<float>(xn[c * a.xs[1] + ih * a.xs[2] + iw * a.xs[3]]) *
                 static_cast<float>(wk[c * a.ws[1] + r * a.ws[2] + s * a.ws[3]]);
        }
      }
    }
    if (a.bias) acc += static_cast<float>(static_cast<const T*>(a.bias)[k * a.bs]);
    static_cast<T*>(a.out)[n * a.os[0] + k * a.os[1] + p * a.os[2] + q * a.os[3]] = static_cast<T>(acc);
  }
}

// col[b][kg][pix] for images n0 .. n0 + nb - 1 (b = n - n0), pixel rows of
// ld elements (pixels PQ .. ld - 1 are zero).  One thread per 8 pixels of one
// (b, kg) row: a 16-byte (or 32-byte for fp32) run of the output row.
template <typename T>
__global__ __launch_bounds__(256) void k_im2col(ConvArgs a, T* col, int n0, int nb, int64_t ld, int64_t kp) {
  const int crs = a.C * a.R * a.S;
  const int64_t chunks = ld / 8;
  const int64_t total = static_cast<int64_t>(nb) * crs * chunks;
  const T* x = static_cast<const T*>(a.x);
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t ch = i % chunks;
    const int64_t row = i / chunks;  // b * crs + kg
    const int kg = static_cast<int>(row % crs);
    const int b = static_cast<int>(row / crs);
    const int s = kg % a.S;
    const int r = (kg / a.S) % a.R;
    const int c = kg / (a.R * a.S);
    const T* xc = x + (n0 + b) * a.xs[0] + c * a.xs[1];
    T v[8];
    const int pq0 = static_cast<int>(ch * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int pq = pq0 + e;
      T val = static_cast<T>(0.f);
      if (pq < a.P * a.Q) {
        const int p = pq / a.Q, q = pq - (pq / a.Q) * a.Q;
        const int ih = p * a.sh - a.ph + r * a.dh;
        const int iw = q * a.sw - a.pw + s * a.dw;
        if (ih >= 0 && ih < a.H && iw >= 0 && iw < a.W) val = xc[ih * a.xs[2] + iw * a.xs[3]];
      }
      v[e] = val;
    }
    T* dst = col + (static_cast<int64_t>(b) * kp + kg) * ld + pq0;
    if constexpr (sizeof(T) == 2) {
      *reinterpret_cast<u32x4*>(dst) = __builtin_bit_cast(u32x4, v);
    } else {
      reinterpret_cast<u32x4*>(dst)[0] = u32x4{__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                                               __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3])};
      reinterpret_cast<u32x4*>(dst)[1] = u32x4{__builtin_bit_cast(uint32_t, v[4]), __builtin_bit_cast(uint32_t, v[5]),
                                               __builtin_bit_cast(uint32_t, v[6]), __builtin_bit_cast(uint32_t, v[7])};
    }
  }
}

// Stages rows row0 .. row0 + nrows - 1 of x[n][c] (W elements each) into
// LDS: 16-byte loads when the rows are contiguous, 16-byte aligned runs of a
// multiple of 8 elements, else one element per load.
template <typename T>
__device__ __forceinline__ void stage_rows(const ConvArgs& a, const T* xc, T* plane, int row0, int nrows) {
  constexpr int V = 16 / sizeof(T);
  xc += static_cast<int64_t>(row0) * a.xs[2];
  if (a.xs[3] == 1 && a.W % V == 0 && a.xs[2] % V == 0 && (reinterpret_cast<uintptr_t>(xc) & 15u) == 0) {
    const int wv = a.W / V;
    for (int i = threadIdx.x; i < nrows * wv; i += blockDim.x) {
      const int ih = i / wv, c8 = i - (i / wv) * wv;
      *reinterpret_cast<u32x4*>(plane + ih * a.W + c8 * V) = *reinterpret_cast<const u32x4*>(xc + ih * a.xs[2] + c8 * V);
    }
  } else {
    for (int i = threadIdx.x; i < nrows * a.W; i += blockDim.x) {
      const int ih = i / a.W, iw = i - (i / a.W) * a.W;
      plane[i] = xc[ih * a.xs[2] + iw * a.xs[3]];
    }
  }
}

// The whole H x W plane x[n][c].
template <typename T>
__device__ __forceinline__ void stage_plane(const ConvArgs& a, const T* xc, T* plane) {
  stage_rows<T>(a, xc, plane, 0, a.H);
}

// Same output as k_im2col, one workgroup per (image, channel): the input
// plane is staged in LDS once (read from HBM once, any strides), then every
// tap's unfolded row is written from LDS with 16-byte stores, neighbouring
// threads writing neighbouring pixel runs.  Used when the plane fits in
// kPlaneLds bytes (the launch reserves exactly the plane, so small planes
// leave room for many workgroups per CU).
constexpr int kPlaneLds = 64 * 1024;

template <typename T>
__global__ __launch_bounds__(256) void k_im2col_plane(ConvArgs a, T* col, int n0, int nb, int64_t ld,
                                                      int64_t kp) {
  extern __shared__ __attribute__((aligned(16))) char sm[];  // H * W elements
  T* plane = reinterpret_cast<T*>(sm);
  const int64_t id = block_id();  // (image, channel) plane; blocks_2d grid
  if (id >= static_cast<int64_t>(nb) * a.C) return;  // the tail of the grid (the whole block)
  const int b = static_cast<int>(id / a.C);
  const int c = static_cast<int>(id - static_cast<int64_t>(b) * a.C);
  stage_plane<T>(a, static_cast<const T*>(a.x) + (n0 + b) * a.xs[0] + c * a.xs[1], plane);
  __syncthreads();
  const int rs = a.R * a.S;
  const int pq = a.P * a.Q;
  const int nch = static_cast<int>(ld / 8);
  T* dst0 = col + (static_cast<int64_t>(b) * kp + static_cast<int64_t>(c) * rs) * ld;
  for (int j = threadIdx.x; j < nch; j += blockDim.x) {
    // the 8 pixels of run j: output (p, q) computed once, then reused for
    // every tap
    int p = (8 * j) / a.Q;
    int q = 8 * j - p * a.Q;
    int hbase[8], wbase[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool in = 8 * j + e < pq;
      hbase[e] = in ? p * a.sh - a.ph : -0x40000000;  // out-of-range pixels never land in the plane
      wbase[e] = q * a.sw - a.pw;
      if (++q == a.Q) {
        q = 0;
        ++p;
      }
    }
    for (int r = 0; r < a.R; ++r) {
      for (int s = 0; s < a.S; ++s) {
        T v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int ih = hbase[e] + r * a.dh;
          const int iw = wbase[e] + s * a.dw;
          const bool ok = static_cast<unsigned>(ih) < static_cast<unsigned>(a.H) &&
                          static_cast<unsigned>(iw) < static_cast<unsigned>(a.W);
          v[e] = ok ? plane[ih * a.W + iw] : static_cast<T>(0.f);
        }
        T* dst = dst0 + static_cast<int64_t>(r * a.S + s) * ld + 8 * j;
        if constexpr (sizeof(T) == 2) {
          *reinterpret_cast<u32x4*>(dst) = __builtin_bit_cast(u32x4, v);
        } else {
          reinterpret_cast<u32x4*>(dst)[0] = u32x4{__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                                                   __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3])};
          reinterpret_cast<u32x4*>(dst)[1] = u32x4{__builtin_bit_cast(uint32_t, v[4]), __builtin_bit_cast(uint32_t, v[5]),
                                                   __builtin_bit_cast(uint32_t, v[6]), __builtin_bit_cast(uint32_t, v[7])};
        }
      }
    }
  }
}

// Same output as k_im2col for planes too large for k_im2col_plane's LDS: one
// workgroup per (image, channel, band of kBandRuns 8-pixel runs of the
// unfolded row); it stages only the input rows its band's output rows read
// (kBandRuns * 8 pixels = a few output rows, so a 3-channel 224 x 224 stem
// with stride 2 and a 7 x 7 kernel stages 17 rows, 7.4 KiB), then writes
// every tap's 16-byte runs from LDS -- lane l of the block on run l % 64,
// taps l / 64, l / 64 + 4, ... -- so neighbouring lanes store neighbouring
// runs.  The launch reserves band_lds_rows(a) rows of W elements.
constexpr int kBandRuns = 64;

template <typename T>
__global__ __launch_bounds__(256) void k_im2col_band(ConvArgs a, T* col, int n0, int nb, int64_t ld, int64_t kp,
                                                     int nbands) {
  extern __shared__ __attribute__((aligned(16))) char sm[];
  T* band = reinterpret_cast<T*>(sm);
  const int64_t id = block_id();  // ((image, channel), band); blocks_2d grid
  if (id >= static_cast<int64_t>(nb) * a.C * nbands) return;  // the tail of the grid (the whole block)
  const int64_t plane_id = id / nbands;
  const int bi = static_cast<int>(id - plane_id * nbands);
  const int b = static_cast<int>(plane_id / a.C);
  const int c = static_cast<int>(plane_id - static_cast<int64_t>(b) * a.C);
  const int pq = a.P * a.Q;
  const int nch = static_cast<int>(ld / 8);
  const int j0 = bi * kBandRuns;
  const int j1 = min(nch, j0 + kBandRuns);
  // output rows of the band's pixels, and the input rows they read
  const int p_lo = (8 * j0) / a.Q;
  const int p_hi = (min(8 * j1, pq) - 1) / a.Q;
  const int ih0 = max(0, p_lo * a.sh - a.ph);
  const int ih1 = min(a.H - 1, p_hi * a.sh - a.ph + (a.R - 1) * a.dh);
  if (ih1 >= ih0)
    stage_rows<T>(a, static_cast<const T*>(a.x) + (n0 + b) * a.xs[0] + c * a.xs[1], band, ih0, ih1 - ih0 + 1);
  __syncthreads();
  const int rs = a.R * a.S;
  T* dst0 = col + (static_cast<int64_t>(b) * kp + static_cast<int64_t>(c) * rs) * ld;
  const int j = j0 + (threadIdx.x & (kBandRuns - 1));
  if (j >= j1) return;
  int p = (8 * j) / a.Q;
  int q = 8 * j - p * a.Q;
  int hbase[8], wbase[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const bool in = 8 * j + e < pq;
    hbase[e] = in ? p * a.sh - a.ph : -0x40000000;  // out-of-range pixels never land in the band
    wbase[e] = q * a.sw - a.pw;
    if (++q == a.Q) {
      q = 0;
      ++p;
    }
  }
  for (int t = threadIdx.x / kBandRuns; t < rs; t += 256 / kBandRuns) {
    const int r = t / a.S, sx = t - r * a.S;
    T v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int ih = hbase[e] + r * a.dh;
      const int iw = wbase[e] + sx * a.dw;
      const bool ok = static_cast<unsigned>(ih) < static_cast<unsigned>(a.H) &&
                      static_cast<unsigned>(iw) < static_cast<unsigned>(a.W);
      v[e] = ok ? band[(ih - ih0) * a.W + iw] : static_cast<T>(0.f);
    }
    T* dst = dst0 + static_cast<int64_t>(t) * ld + 8 * j;
    if constexpr (sizeof(T) == 2) {
      *reinterpret_cast<u32x4*>(dst) = __builtin_bit_cast(u32x4, v);
    } else {
      reinterpret_cast<u32x4*>(dst)[0] = u32x4{__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                                               __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3])};
      reinterpret_cast<u32x4*>(dst)[1] = u32x4{__builtin_bit_cast(uint32_t, v[4]), __builtin_bit_cast(uint32_t, v[5]),
                                               __builtin_bit_cast(uint32_t, v[6]), __builtin_bit_cast(uint32_t, v[7])};
    }
  }
}

// Input rows a band of k_im2col_band may stage: its kBandRuns * 8 pixels
// span at most (kBandRuns * 8 - 1) / Q + 2 output rows.
int64_t band_lds_rows(const ConvArgs& a) {
  const int64_t prow = (kBandRuns * 8 - 1) / a.Q + 2;
  return std::min<int64_t>(a.H, (prow - 1) * a.sh + static_cast<int64_t>(a.R - 1) * a.dh + 1);
}

// xs[b][s][c][row][q] for images n0 .. n0 + nb - 1 (stride-1 convolutions):
// one thread per 8 consecutive q of one (b, s, c, row).
template <typename T>
__global__ __launch_bounds__(256) void k_conv_shift(ConvArgs a, T* xs, int n0, int nb, int hp) {
  const int q8 = a.Q / 8;
  const int64_t total = static_cast<int64_t>(nb) * a.S * a.C * hp * q8;
  const T* x = static_cast<const T*>(a.x);
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int qc = static_cast<int>(i % q8);
    int64_t t = i / q8;
    const int row = static_cast<int>(t % hp);
    t /= hp;
    const int c = static_cast<int>(t % a.C);
    t /= a.C;
    const int s = static_cast<int>(t % a.S);
    const int b = static_cast<int>(t / a.S);
    const int ih = row - a.ph;
    const int iw0 = qc * 8 + s * a.dw - a.pw;
    const T* xr = x + (n0 + b) * a.xs[0] + c * a.xs[1] + static_cast<int64_t>(ih) * a.xs[2];
    const bool row_ok = ih >= 0 && ih < a.H;
    T v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int iw = iw0 + e;
      v[e] = (row_ok && iw >= 0 && iw < a.W) ? xr[iw * a.xs[3]] : static_cast<T>(0.f);
    }
    *reinterpret_cast<u32x4*>(xs + i * 8) = __builtin_bit_cast(u32x4, v);
  }
}

// Same output as k_conv_shift, one workgroup per (image, channel) with the
// input plane staged in LDS (read from HBM once); a thread then writes the
// same 8-pixel run of every shifted plane.
template <typename T>
__global__ __launch_bounds__(256) void k_conv_shift_plane(ConvArgs a, T* xs, int n0, int nb, int hp) {
  extern __shared__ __attribute__((aligned(16))) char sm[];  // H * W elements
  T* plane = reinterpret_cast<T*>(sm);
  const int64_t id = block_id();  // (image, channel) plane; blocks_2d grid
  if (id >= static_cast<int64_t>(nb) * a.C) return;  // the tail of the grid (the whole block)
  const int b = static_cast<int>(id / a.C);
  const int c = static_cast<int>(id - static_cast<int64_t>(b) * a.C);
  stage_plane<T>(a, static_cast<const T*>(a.x) + (n0 + b) * a.xs[0] + c * a.xs[1], plane);
  __syncthreads();
  const int q8 = a.Q / 8;
  const int64_t plane_elems = static_cast<int64_t>(hp) * a.Q;
  const int64_t s_stride = static_cast<int64_t>(a.C) * plane_elems;  // between shifted planes
  T* dst0 = xs + (static_cast<int64_t>(b) * a.S * a.C + c) * plane_elems;
  for (int j = threadIdx.x; j < hp * q8; j += blockDim.x) {
    const int row = j / q8;
    const int q0 = (j - row * q8) * 8;
    const int ih = row - a.ph;
    const bool row_ok = static_cast<unsigned>(ih) < static_cast<unsigned>(a.H);
    T* dst = dst0 + static_cast<int64_t>(row) * a.Q + q0;
    for (int s = 0; s < a.S; ++s) {
      const int iw0 = q0 + s * a.dw - a.pw;
      T v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int iw = iw0 + e;
        v[e] = (row_ok && static_cast<unsigned>(iw) < static_cast<unsigned>(a.W)) ? plane[ih * a.W + iw]
                                                                                  : static_cast<T>(0.f);
      }
      *reinterpret_cast<u32x4*>(dst + s * s_stride) = __builtin_bit_cast(u32x4, v);
    }
  }
}

// Padded channels-last copy of images n0 .. n0 + nb - 1:
// xt[b][hh][ww][c] = x[n0 + b][c][hh - ph][ww - pw], zero outside the image.
// One thread per pixel and 8 channels: 8 loads of one channel row each
// (neighbouring threads read neighbouring pixels of it) and one 16-byte
// store of the channels.
template <typename T>
__global__ __launch_bounds__(256) void k_conv_to_cl(ConvArgs a, T* xt, int n0, int nb, int hp, int wp) {
  const int c8 = a.C / 8;
  const int64_t total = static_cast<int64_t>(nb) * hp * c8 * wp;
  const T* x = static_cast<const T*>(a.x);
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int ww = static_cast<int>(i % wp);
    int64_t t = i / wp;
    const int j = static_cast<int>(t % c8);
    t /= c8;
    const int hh = static_cast<int>(t % hp);
    const int b = static_cast<int>(t / hp);
    const int ih = hh - a.ph, iw = ww - a.pw;
    T v[8];
    if (static_cast<unsigned>(ih) < static_cast<unsigned>(a.H) && static_cast<unsigned>(iw) < static_cast<unsigned>(a.W)) {
      const T* src = x + (n0 + b) * a.xs[0] + static_cast<int64_t>(j * 8) * a.xs[1] + ih * a.xs[2] + iw * a.xs[3];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = src[e * a.xs[1]];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = static_cast<T>(0.f);
    }
    *reinterpret_cast<u32x4*>(xt + ((static_cast<int64_t>(b) * hp + hh) * wp + ww) * a.C + j * 8) =
        __builtin_bit_cast(u32x4, v);
  }
}

// Weights in the channels-last GEMM's k order (32-channel blocks, then
// taps, then the block's channels): wt[k][((cb * R + r) * S + s) * 32 + ci]
// = w[k][32 cb + ci][r][s].  Item i (of K C R S / 8) is 8 channels: 8
// loads, one 16-byte store.
template <typename T>
__device__ __forceinline__ void conv_weight_pack(const ConvArgs& a, T* wt, int64_t i) {
  const T* w = static_cast<const T*>(a.w);
  const int ci8 = static_cast<int>(i % 4) * 8;  // the 8 channels' offset in the block
  int64_t t = i / 4;
  const int s = static_cast<int>(t % a.S);
  t /= a.S;
  const int r = static_cast<int>(t % a.R);
  t /= a.R;
  const int cb = static_cast<int>(t % (a.C / 32));
  const int k = static_cast<int>(t / (a.C / 32));
  const T* src = w + k * a.ws[0] + static_cast<int64_t>(cb * 32 + ci8) * a.ws[1] + r * a.ws[2] + s * a.ws[3];
  T v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = src[e * a.ws[1]];
  *reinterpret_cast<u32x4*>(wt + i * 8) = __builtin_bit_cast(u32x4, v);
}

// Same output as k_conv_to_cl for 16-byte aligned input rows of a multiple
// of 8 pixels that fit the padded row (pw + W <= wp).  A wave moves 64
// channels x 64 consecutive pixels of the channel planes: lane 8 j + g loads
// 8 pixels (one 16-byte run, inside one image row) of each of the channels
// 8 j .. 8 j + 7 -- eight lanes read 128 contiguous bytes of a plane --,
// transposes the 8 x 8 block in registers and stores 8 channels of each of
// its 8 pixels -- eight lanes write 128 contiguous bytes of a pixel.  Waves
// past the interior zero the border (rows above and below it, columns beside
// it), 16 bytes per lane.  (32, 256, 56, 56) bf16: 18.9 us, 5.6 TB/s, where
// lanes taking neighbouring channel groups of one pixel group ran 25.0 us.
// With wt set, the launch's first waves also reorder the weights
// (conv_weight_pack), which a launch of their own left serialised ahead of
// the copy.
template <typename T>
__global__ __launch_bounds__(256) void k_conv_to_cl8(ConvArgs a, T* xt, int n0, int nb, int hp, int wp, T* wt) {
  const int lane = threadIdx.x & 63;
  const int64_t witems = wt != nullptr ? static_cast<int64_t>(a.K) * a.C * a.R * a.S / 8 : 0;
  const int64_t wwaves = (witems + 63) / 64;
  const int64_t hw = static_cast<int64_t>(a.H) * a.W;
  const int cb = (a.C + 63) / 64;                        // 64-channel blocks
  const int64_t pb = (hw + 63) / 64;                     // 64-pixel blocks
  const int64_t units = static_cast<int64_t>(nb) * cb * pb;
  const int top = min(a.ph, hp);                         // zero rows above the interior
  const int mid = max(0, min(hp, a.ph + a.H) - a.ph);    // interior rows
  const int bot = hp - top - mid;                        // zero rows below it
  const int side = wp - a.W;                             // zero columns per interior row
  const int64_t border = static_cast<int64_t>(top + bot) * wp + static_cast<int64_t>(mid) * side;
  const int c8 = a.C / 8;
  const int64_t pads = static_cast<int64_t>(nb) * border * c8;
  const int64_t waves = wwaves + units + (pads + 63) / 64;
  const T* x = static_cast<const T*>(a.x);
  for (int64_t v = blockIdx.x * 4ll + (threadIdx.x >> 6); v < waves; v += static_cast<int64_t>(gridDim.x) * 4) {
    if (v < wwaves) {
      const int64_t i = v * 64 + lane;
      if (i < witems) conv_weight_pack(a, wt, i);
      continue;
    }
    const int64_t u = v - wwaves;
    if (u < units) {
      const int64_t g = u % pb;
      const int64_t t = u / pb;
      const int c0 = static_cast<int>(t % cb) * 64 + (lane >> 3) * 8;
      const int b = static_cast<int>(t / cb);
      const int64_t p0 = g * 64 + (lane & 7) * 8;
      if (c0 >= a.C || p0 >= hw) continue;
      const int ih = static_cast<int>(p0 / a.W), iw = static_cast<int>(p0 % a.W);
      const int hh = a.ph + ih;
      if (hh >= hp) continue;  // input row the convolution never reads
      const T* src = x + (n0 + b) * a.xs[0] + c0 * a.xs[1] + ih * a.xs[2] + iw;
      u32x4 in[8];  // in[e]: pixels 0..7 of channel c0 + e, two per word
#pragma unroll
      for (int e = 0; e < 8; ++e) in[e] = *reinterpret_cast<const u32x4*>(src + e * a.xs[1]);
      u32x4 out[8];  // out[f] word k: channels 2k (low half) and 2k + 1 (high half) of pixel f
#pragma unroll
      for (int f = 0; f < 8; ++f)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t lo = in[2 * k][f / 2], hi = in[2 * k + 1][f / 2];
          out[f][k] = (f & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
        }
      T* dst = xt + ((static_cast<int64_t>(b) * hp + hh) * wp + a.pw + iw) * a.C + c0;
#pragma unroll
      for (int f = 0; f < 8; ++f) *reinterpret_cast<u32x4*>(dst + static_cast<int64_t>(f) * a.C) = out[f];
    } else {
      const int64_t k = (u - units) * 64 + lane;
      if (k >= pads) continue;
      const int j = static_cast<int>(k % c8);
      int64_t q = k / c8;
      const int b = static_cast<int>(q / border);
      q %= border;
      int hh, ww;
      if (q < static_cast<int64_t>(top) * wp) {
        hh = static_cast<int>(q / wp);
        ww = static_cast<int>(q % wp);
      } else if ((q -= static_cast<int64_t>(top) * wp) < static_cast<int64_t>(bot) * wp) {
        hh = top + mid + static_cast<int>(q / wp);
        ww = static_cast<int>(q % wp);
      } else {
        q -= static_cast<int64_t>(bot) * wp;
        hh = a.ph + static_cast<int>(q / side);
        const int c = static_cast<int>(q % side);
        ww = c < a.pw ? c : a.W + c;  // columns [0, pw) and [pw + W, wp)
      }
      *reinterpret_cast<u32x4*>(xt + ((static_cast<int64_t>(b) * hp + hh) * wp + ww) * a.C + j * 8) =
          u32x4{0u, 0u, 0u, 0u};
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void k_conv_weights_cl(ConvArgs a, T* wt) {
  const int64_t total = static_cast<int64_t>(a.K) * a.C * a.R * a.S / 8;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    conv_weight_pack(a, wt, i);
}

// Rows crs .. kp - 1 of each of nb unfolded images (the zero rows that pad
// the GEMM's reduction depth to a multiple of 8), one 16-byte chunk per
// thread per step (rows of ld elements are whole 16-byte chunks).
template <typename T>
__global__ __launch_bounds__(256) void k_conv_col_zero_rows(T* col, int64_t nb, int64_t crs, int64_t kp, int64_t ld) {
  const int64_t per_row = ld * static_cast<int64_t>(sizeof(T)) / 16;
  const int64_t per_img = (kp - crs) * per_row;
  const int64_t total = nb * per_img;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t b = i / per_img, rem = i - b * per_img;
    char* row0 = reinterpret_cast<char*>(col + (b * kp + crs) * ld);
    *reinterpret_cast<u32x4*>(row0 + rem * 16) = u32x4{0u, 0u, 0u, 0u};
  }
}

// W (any strides) as a row-major K x kp matrix whose columns crs .. kp - 1
// are zero: the GEMM's A operand when the weight rows cannot be read in
// place.
template <typename T>
__global__ __launch_bounds__(256) void k_conv_weights_rows(ConvArgs a, T* wp, int64_t kp) {
  const int rs = a.R * a.S;
  const int64_t crs = static_cast<int64_t>(a.C) * rs;
  const int64_t total = static_cast<int64_t>(a.K) * kp;
  const T* w = static_cast<const T*>(a.w);
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t k = i / kp, j = i - k * kp;
    T v = static_cast<T>(0.f);
    if (j < crs) {
      const int c = static_cast<int>(j / rs), t = static_cast<int>(j - static_cast<int64_t>(c) * rs);
      const int r = t / a.S, sx = t - r * a.S;
      v = w[k * a.ws[0] + c * a.ws[1] + r * a.ws[2] + sx * a.ws[3]];
    }
    wp[i] = v;
  }
}

unsigned grid_for(int64_t work, int per_block) {
  int64_t g = (work + per_block - 1) / per_block;
  if (g > 65536) g = 65536;  // grid-stride loops cover the rest
  return static_cast<unsigned>(g < 1 ? 1 : g);
}

// Pixels per unfolded row (a multiple of 8, so rows stay 16-byte aligned).
int64_t col_ld(const ConvArgs& a) { return (static_cast<int64_t>(a.P) * a.Q + 7) / 8 * 8; }

// Unfolded rows per image: C R S padded to a multiple of 8 (the GEMM's
// K-major operand needs 16-byte rows); the pad rows are zero.
int64_t col_rows(const ConvArgs& a) { return (static_cast<int64_t>(a.C) * a.R * a.S + 7) / 8 * 8; }

// Whether W can be the GEMM's A operand in place: rows of C R S contiguous
// elements, a row stride of a multiple of 8 elements, 16-byte aligned.
bool w_rows_ok(const ConvArgs& a) {
  return a.ws[3] == 1 && a.ws[2] == a.S && a.ws[1] == static_cast<int64_t>(a.R) * a.S && a.ws[0] % 8 == 0 &&
         (reinterpret_cast<uintptr_t>(a.w) & 15u) == 0;
}

// Whether the unfold path copies W into the workspace (K x col_rows, zero
// columns past C R S).
bool unfold_stages_w(const ConvArgs& a) {
  return col_rows(a) != static_cast<int64_t>(a.C) * a.R * a.S || !w_rows_ok(a);
}

// Whether the GEMM path applies: enough reduction depth, output channels and
// output pixels to feed the matrix cores, and pixel planes of the output
// that are contiguous.
bool use_gemm(const ConvArgs& a, int dt) {
  const int64_t crs = static_cast<int64_t>(a.C) * a.R * a.S;
  const int64_t pq = static_cast<int64_t>(a.P) * a.Q;
  const bool out_plane = a.os[3] == 1 && a.os[2] == a.Q;
  return dt != NTOPS_F64 && crs >= 64 && a.K >= 32 && pq >= 16 && out_plane &&
         col_rows(a) * col_ld(a) <= 0x7fffffffLL;
}

int64_t col_bytes_per_image(const ConvArgs& a, int dt) { return col_rows(a) * col_ld(a) * dtype_size(dt); }

// Output planes whose pixel count is not a multiple of 8 are computed at
// the unfold's padded width (the matrix-core GEMM's N-major operand and
// vector stores need it) into the workspace, then copied out: bytes per
// image of that staging (0 when the plane is written directly).
int64_t padded_out_bytes_per_image(const ConvArgs& a, int dt) {
  const int64_t pq = static_cast<int64_t>(a.P) * a.Q;
  return pq % 8 ? static_cast<int64_t>(a.K) * col_ld(a) * dtype_size(dt) : 0;
}

// Rows of each shifted plane of the implicit path.
int64_t shift_rows(const ConvArgs& a) { return static_cast<int64_t>(a.P) + static_cast<int64_t>(a.R - 1) * a.dh; }

// Whether the implicit GEMM applies (on top of use_gemm): stride 1, 16-bit
// data, output rows of a multiple of 8 pixels, W readable in place with
// C R S a multiple of 8, operands inside the 2 GiB
// buffer range, and an output whose channel and image strides are multiples
// of 4 elements at an 8-byte aligned address (the epilogue's store width);
// anything else takes the unfold + GEMM path.
bool use_implicit(const ConvArgs& a, int dt) {
  const int64_t elems = static_cast<int64_t>(a.S) * a.C * shift_rows(a) * a.Q;
  const int64_t crs = static_cast<int64_t>(a.C) * a.R * a.S;
  const bool out_ok = a.os[1] % 4 == 0 && a.os[0] % 4 == 0 && (reinterpret_cast<uintptr_t>(a.out) & 7u) == 0;
  return (dt == NTOPS_BF16 || dt == NTOPS_F16) && a.sh == 1 && a.sw == 1 && a.Q % 8 == 0 && crs % 8 == 0 &&
         w_rows_ok(a) && elems * 2 < (int64_t(1) << 31) && (256 * a.ws[0] + crs) * 2 < (int64_t(1) << 31) &&
         out_ok;
}

// Rows and pixels per row of the channels-last padded copy.
int64_t cl_rows(const ConvArgs& a) { return static_cast<int64_t>(a.P - 1) * a.sh + static_cast<int64_t>(a.R - 1) * a.dh + 1; }
int64_t cl_cols(const ConvArgs& a) { return static_cast<int64_t>(a.Q - 1) * a.sw + static_cast<int64_t>(a.S - 1) * a.dw + 1; }

// Waves of k_conv_to_cl8 for nb images: the weight items (if any), 64 per
// wave, 64-channel x 64-pixel blocks of the input, then the border's
// 16-byte chunks, 64 per wave.
int64_t cl8_waves(const ConvArgs& a, int64_t nb, int64_t hp, int64_t wp, bool weights) {
  const int64_t hw = static_cast<int64_t>(a.H) * a.W;
  const int64_t mid = std::max<int64_t>(0, std::min<int64_t>(hp, a.ph + a.H) - a.ph);  // interior rows
  const int64_t border = (hp - mid) * wp + mid * (wp - a.W);
  const int64_t witems = weights ? static_cast<int64_t>(a.K) * a.C * a.R * a.S / 8 : 0;
  return (witems + 63) / 64 + nb * ((a.C + 63) / 64) * ((hw + 63) / 64) + (nb * border * (a.C / 8) + 63) / 64;
}

// Whether the channels-last implicit GEMM applies (on top of use_gemm):
// 16-bit data, C a multiple of the GEMM's 32-channel K tile, P * Q a
// multiple of 4 with the output channel and image strides multiples of 4
// elements at an 8-byte aligned address (the epilogue's store width), and
// each padded image and the weight matrix inside the 2 GiB buffer range.
bool use_channels_last(const ConvArgs& a, int dt) {
  const int64_t crs = static_cast<int64_t>(a.C) * a.R * a.S;
  const int64_t pq = static_cast<int64_t>(a.P) * a.Q;
  const bool out_ok = a.os[1] % 4 == 0 && a.os[0] % 4 == 0 && (reinterpret_cast<uintptr_t>(a.out) & 7u) == 0;
  return (dt == NTOPS_BF16 || dt == NTOPS_F16) && a.C % 32 == 0 && pq % 4 == 0 && out_ok &&
         cl_rows(a) * cl_cols(a) * a.C * 2 < (int64_t(1) << 31) && 257 * crs * 2 < (int64_t(1) << 31) &&
         crs <= 0x7fffffffLL && pq <= 0x7fffffffLL;
}

// Workspace bytes after the unfold path's images through which its fp32
// GEMM over nb images splits K (what ntops_gemm_workspace asks for; 0 for
// 16-bit data and the implicit paths): a batch of per-image products with
// few output channels and pixels fills few tiles otherwise.
int64_t split_bytes(const ConvArgs& a, int dt, int64_t nb) {
  if (dt != NTOPS_F32 || use_channels_last(a, dt) || use_implicit(a, dt)) return 0;
  const int64_t pq = static_cast<int64_t>(a.P) * a.Q;
  const int64_t cols = padded_out_bytes_per_image(a, dt) > 0 ? col_ld(a) : pq;
  const int64_t w = ntops_gemm_workspace(dt, nb, a.K, cols, col_rows(a));
  return w > 0 ? (w + 511) / 256 * 256 : 0;  // (room to start it 256-aligned)
}

// Workspace bytes per image of the chosen GEMM path.
int64_t ws_bytes_per_image(const ConvArgs& a, int dt) {
  if (use_channels_last(a, dt)) return cl_rows(a) * cl_cols(a) * a.C * dtype_size(dt);
  if (use_implicit(a, dt)) return static_cast<int64_t>(a.S) * a.C * shift_rows(a) * a.Q * dtype_size(dt);
  return col_bytes_per_image(a, dt) + padded_out_bytes_per_image(a, dt);
}

// Workspace bytes the chosen GEMM path needs once per call, ahead of the
// images' (the channels-last path's reordered weights, or the unfold path's
// K x col_rows copy of W; rounded up to 256).
int64_t ws_bytes_fixed(const ConvArgs& a, int dt) {
  if (use_channels_last(a, dt))
    return (static_cast<int64_t>(a.K) * a.C * a.R * a.S * dtype_size(dt) + 255) / 256 * 256;
  if (use_implicit(a, dt) || !unfold_stages_w(a)) return 0;
  return (static_cast<int64_t>(a.K) * col_rows(a) * dtype_size(dt) + 255) / 256 * 256;
}

int fill_args(ConvArgs& a, int64_t N, int64_t C, int64_t H, int64_t W, int64_t K, int64_t R, int64_t S,
              int64_t P, int64_t Q, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw) {
  const int64_t v[] = {N, C, H, W, K, R, S, P, Q, sh, sw, ph, pw, dh, dw};
  for (int64_t x : v)
    if (x < 0 || x > 0x7fffffffLL) return set_error(NTOPS_ERR_INVALID, "conv2d: size or parameter out of range");
  if (sh < 1 || sw < 1 || dh < 1 || dw < 1) return set_error(NTOPS_ERR_INVALID, "conv2d: stride and dilation must be >= 1");
  a.N = static_cast<int>(N);
  a.C = static_cast<int>(C);
  a.H = static_cast<int>(H);
  a.W = static_cast<int>(W);
  a.K = static_cast<int>(K);
  a.R = static_cast<int>(R);
  a.S = static_cast<int>(S);
  a.P = static_cast<int>(P);
  a.Q = static_cast<int>(Q);
  a.sh = static_cast<int>(sh);
  a.sw = static_cast<int>(sw);
  a.ph = static_cast<int>(ph);
  a.pw = static_cast<int>(pw);
  a.dh = static_cast<int>(dh);
  a.dw = static_cast<int>(dw);
  return NTOPS_OK;
}

}  // namespace
}  // namespace ntops

using namespace ntops;

extern "C" int64_t ntops_conv2d_workspace(int dtype, int64_t N, int64_t C, int64_t H, int64_t W, int64_t K,
                                          int64_t R, int64_t S, int64_t P, int64_t Q, int64_t stride_h,
                                          int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t dil_h,
                                          int64_t dil_w, const int64_t* w_strides, const int64_t* out_strides) {
  ConvArgs a{};
  if (fill_args(a, N, C, H, W, K, R, S, P, Q, stride_h, stride_w, pad_h, pad_w, dil_h, dil_w) != NTOPS_OK) return 0;
  if (!w_strides || !out_strides || dtype_size(dtype) == 0) return 0;
  for (int i = 0; i < 4; ++i) {
    a.ws[i] = w_strides[i];
    a.os[i] = out_strides[i];
  }
  a.w = nullptr;  // alignment is checked again on the call
  a.out = nullptr;
  if (!use_gemm(a, dtype)) return 0;
  return ws_bytes_fixed(a, dtype) + ws_bytes_per_image(a, dtype) * N + split_bytes(a, dtype, N);
}

extern "C" int ntops_conv2d(int dtype, int64_t N, int64_t C, int64_t H, int64_t W, int64_t K, int64_t R,
                            int64_t S, int64_t P, int64_t Q, int64_t stride_h, int64_t stride_w, int64_t pad_h,
                            int64_t pad_w, int64_t dil_h, int64_t dil_w, const void* x, const int64_t* x_strides,
                            const void* w, const int64_t* w_strides, const void* bias, int64_t bias_stride,
                            void* out, const int64_t* out_strides, void* workspace, int64_t workspace_bytes,
                            void* stream) {
  ConvArgs a{};
  int rc = fill_args(a, N, C, H, W, K, R, S, P, Q, stride_h, stride_w, pad_h, pad_w, dil_h, dil_w);
  if (rc != NTOPS_OK) return rc;
  if (N == 0 || K == 0 || P == 0 || Q == 0) return NTOPS_OK;
  if (!x || !w || !out || !x_strides || !w_strides || !out_strides)
    return set_error(NTOPS_ERR_INVALID, "conv2d: null pointer");
  if (workspace_bytes < 0) return set_error(NTOPS_ERR_INVALID, "conv2d: negative workspace size");
  a.x = x;
  a.w = w;
  a.bias = bias;
  a.out = out;
  a.bs = bias_stride;
  for (int i = 0; i < 4; ++i) {
    a.xs[i] = x_strides[i];
    a.ws[i] = w_strides[i];
    a.os[i] = out_strides[i];
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t per_image = dtype_size(dtype) ? ws_bytes_per_image(a, dtype) : 0;
  const int64_t fixed = dtype_size(dtype) ? ws_bytes_fixed(a, dtype) : 0;
  const bool gemm = dtype_size(dtype) && use_gemm(a, dtype) && workspace && per_image > 0 &&
                    workspace_bytes >= fixed + per_image && (reinterpret_cast<uintptr_t>(workspace) & 15u) == 0;
  if (!gemm) {
    return dispatch_float16_32(dtype, "conv2d", [&](auto tag) {
      using T = decltype(tag);
      const int64_t total = N * K * P * Q;
      hipLaunchKernelGGL(k_conv_direct<T>, dim3(grid_for(total, 256)), dim3(256), 0, st, a, total);
      return check_launch("conv2d");
    });
  }
  const int64_t crs = C * R * S;
  if (use_channels_last(a, dtype)) {
    // channels-last implicit GEMM: weights reordered into the workspace's
    // first `fixed` bytes, then chunks of images that fit the rest
    const int64_t hp = cl_rows(a), wp = cl_cols(a);
    const int64_t img = hp * wp * C;  // elements of one padded image
    const int64_t nb_max = std::min<int64_t>(N, (workspace_bytes - fixed) / per_image);
    void* wt = workspace;
    void* xt = static_cast<char*>(workspace) + fixed;
    // 16-byte input rows: the block copy, which also reorders the weights
    // (with the first chunk); otherwise the element copy after a weight launch
    const bool rows16 = a.xs[3] == 1 && a.xs[2] % 8 == 0 && a.xs[1] % 8 == 0 && a.xs[0] % 8 == 0 &&
                        W % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && pad_w + W <= wp;
    if (!rows16) {
      rc = dispatch_float16_32(dtype, "conv2d", [&](auto tag) {
        using T = decltype(tag);
        if constexpr (sizeof(T) != 2) {
          return set_error(NTOPS_ERR_INVALID, "conv2d: the channels-last path needs 16-bit data");
        } else {
          hipLaunchKernelGGL(k_conv_weights_cl<T>, dim3(grid_for(K * crs / 8, 256)), dim3(256), 0, st, a,
                             static_cast<T*>(wt));
          return check_launch("conv2d");
        }
      });
      if (rc != NTOPS_OK) return rc;
    }
    for (int64_t n0 = 0; n0 < N; n0 += nb_max) {
      const int64_t nb = std::min(nb_max, N - n0);
      rc = dispatch_float16_32(dtype, "conv2d", [&](auto tag) {
        using T = decltype(tag);
        if constexpr (sizeof(T) != 2) {
          return set_error(NTOPS_ERR_INVALID, "conv2d: the channels-last path needs 16-bit data");
        } else {
          if (rows16)
            hipLaunchKernelGGL(k_conv_to_cl8<T>, dim3(grid_for(cl8_waves(a, nb, hp, wp, n0 == 0) * 64, 256)),
                               dim3(256), 0, st, a, static_cast<T*>(xt), static_cast<int>(n0), static_cast<int>(nb),
                               static_cast<int>(hp), static_cast<int>(wp), n0 == 0 ? static_cast<T*>(wt) : nullptr);
          else
            hipLaunchKernelGGL(k_conv_to_cl<T>, dim3(grid_for(nb * hp * (C / 8) * wp, 256)), dim3(256), 0, st, a,
                               static_cast<T*>(xt), static_cast<int>(n0), static_cast<int>(nb), static_cast<int>(hp),
                               static_cast<int>(wp));
          return check_launch("conv2d");
        }
      });
      if (rc != NTOPS_OK) return rc;
      void* dst = static_cast<char*>(out) + n0 * out_strides[0] * dtype_size(dtype);
      rc = gemm_conv_channels_last(dtype, static_cast<int>(nb), static_cast<int>(K), static_cast<int>(P * Q),
                                   static_cast<int>(crs), wt, xt, img, static_cast<int>(R), static_cast<int>(S),
                                   static_cast<int>(C), static_cast<int>(Q), static_cast<int>(stride_h),
                                   static_cast<int>(stride_w), static_cast<int>(wp), static_cast<int>(dil_h),
                                   static_cast<int>(dil_w), bias, bias_stride, dst, out_strides[0], out_strides[1], st);
      if (rc != NTOPS_OK) return rc;
    }
    return NTOPS_OK;
  }
  if (use_implicit(a, dtype)) {
    // implicit GEMM, in chunks of images that fit the workspace
    const int64_t hp = shift_rows(a);
    const int64_t plane = hp * Q;  // elements of one shifted plane of one channel
    const int64_t nb_max = std::min<int64_t>(N, workspace_bytes / per_image);
    for (int64_t n0 = 0; n0 < N; n0 += nb_max) {
      const int64_t nb = std::min(nb_max, N - n0);
      rc = dispatch_float16_32(dtype, "conv2d", [&](auto tag) {
        using T = decltype(tag);
        if constexpr (sizeof(T) != 2) {
          return set_error(NTOPS_ERR_INVALID, "conv2d: the implicit path needs 16-bit data");
        } else {
          if (H * W * static_cast<int64_t>(sizeof(T)) <= kPlaneLds)
            hipLaunchKernelGGL(k_conv_shift_plane<T>, blocks_2d(nb * C), dim3(256),
                               static_cast<unsigned>(H * W * sizeof(T)), st, a, static_cast<T*>(workspace),
                               static_cast<int>(n0), static_cast<int>(nb), static_cast<int>(hp));
          else
            hipLaunchKernelGGL(k_conv_shift<T>, dim3(grid_for(nb * S * C * hp * (Q / 8), 256)), dim3(256), 0, st, a,
                               static_cast<T*>(workspace), static_cast<int>(n0), static_cast<int>(nb),
                               static_cast<int>(hp));
          return check_launch("conv2d");
        }
      });
      if (rc != NTOPS_OK) return rc;
      void* dst = static_cast<char*>(out) + n0 * out_strides[0] * dtype_size(dtype);
      rc = gemm_implicit_conv(dtype, static_cast<int>(nb), static_cast<int>(K), static_cast<int>(P * Q),
                              static_cast<int>(crs), w, w_strides[0], workspace, S * C * plane, static_cast<int>(R),
                              static_cast<int>(S), C * plane, plane, dil_h * Q, bias, bias_stride, dst,
                              out_strides[0], out_strides[1], st);
      if (rc != NTOPS_OK) return rc;
    }
    return NTOPS_OK;
  }
  // GEMM path, in chunks of images that fit the workspace: [W copy (if
  // staged)][unfolded images][padded output planes (if P Q % 8 != 0)]
  const int64_t ld = col_ld(a);
  const int64_t kp = col_rows(a);
  const bool stage_w = unfold_stages_w(a);
  void* col = static_cast<char*>(workspace) + fixed;
  const int64_t nb_max = std::min<int64_t>(N, (workspace_bytes - fixed) / per_image);
  const void* wa = stage_w ? workspace : w;
  const int64_t a_str[3] = {0, stage_w ? kp : w_strides[0], 1};
  const int64_t b_str[3] = {kp * ld, ld, 1};
  const int64_t c_str[3] = {0, bias_stride, 0};
  const int64_t d_str[3] = {out_strides[0], out_strides[1], 1};
  const int es = dtype_size(dtype);
  // planes of P Q % 8 != 0 pixels: the GEMM writes rows of ld pixels into
  // the workspace after the unfold, then k_conv_rows_out copies them out
  const bool padded = padded_out_bytes_per_image(a, dtype) > 0;
  void* staged = static_cast<char*>(col) + nb_max * kp * ld * es;
  const int64_t s_str[3] = {K * ld, ld, 1};
  if (stage_w || kp != crs) {
    // the W copy, and the zero pad rows of every image slot of a chunk
    // (the unfold never writes them)
    rc = dispatch_float16_32(dtype, "conv2d", [&](auto tag) {
      using T = decltype(tag);
      if (stage_w)
        hipLaunchKernelGGL(k_conv_weights_rows<T>, dim3(grid_for(K * kp, 256)), dim3(256), 0, st, a,
                           static_cast<T*>(workspace), kp);
      if (kp != crs)
        hipLaunchKernelGGL(k_conv_col_zero_rows<T>, dim3(grid_for(nb_max * (kp - crs) * ld * es / 16, 256)),
                           dim3(256), 0, st, static_cast<T*>(col), nb_max, crs, kp, ld);
      return check_launch("conv2d");
    });
    if (rc != NTOPS_OK) return rc;
  }
  for (int64_t n0 = 0; n0 < N; n0 += nb_max) {
    const int64_t nb = std::min(nb_max, N - n0);
    rc = dispatch_float16_32(dtype, "conv2d", [&](auto tag) {
      using T = decltype(tag);
      const int64_t band_bytes = band_lds_rows(a) * W * static_cast<int64_t>(sizeof(T));
      const int nbands = static_cast<int>((ld / 8 + kBandRuns - 1) / kBandRuns);
      if (static_cast<int64_t>(H) * W * static_cast<int64_t>(sizeof(T)) <= kPlaneLds)
        hipLaunchKernelGGL(k_im2col_plane<T>, blocks_2d(nb * C), dim3(256),
                           static_cast<unsigned>(H * W * sizeof(T)), st, a, static_cast<T*>(col),
                           static_cast<int>(n0), static_cast<int>(nb), ld, kp);
      else if (band_bytes <= kPlaneLds)
        hipLaunchKernelGGL(k_im2col_band<T>, blocks_2d(nb * C * nbands), dim3(256), static_cast<unsigned>(band_bytes),
                           st, a, static_cast<T*>(col), static_cast<int>(n0), static_cast<int>(nb), ld, kp, nbands);
      else
        hipLaunchKernelGGL(k_im2col<T>, dim3(grid_for(nb * crs * (ld / 8), 256)), dim3(256), 0, st, a,
                           static_cast<T*>(col), static_cast<int>(n0), static_cast<int>(nb), ld, kp);
      return check_launch("conv2d");
    });
    if (rc != NTOPS_OK) return rc;
    void* dst = static_cast<char*>(out) + n0 * out_strides[0] * es;
    // what the chunk leaves of the workspace serves the GEMM's split over K
    const int64_t used = (fixed + nb_max * per_image + 255) / 256 * 256;
    void* part = used < workspace_bytes ? static_cast<char*>(workspace) + used : nullptr;
    rc = ntops_gemm_ws(dtype, nb, K, padded ? ld : P * Q, kp, wa, a_str, col, b_str, bias, bias ? c_str : nullptr,
                       1.0, bias ? 1.0 : 0.0, padded ? staged : dst, padded ? s_str : d_str, part,
                       part ? workspace_bytes - used : 0, stream);
    if (rc != NTOPS_OK) return rc;
    if (padded) {
      rc = dispatch_float16_32(dtype, "conv2d", [&](auto tag) {
        using T = decltype(tag);
        const int64_t total = nb * K * P * Q;
        hipLaunchKernelGGL(k_conv_rows_out<T>, dim3(grid_for(total, 256)), dim3(256), 0, st,
                           static_cast<const T*>(staged), ld, static_cast<T*>(dst), out_strides[0],
                           out_strides[1], K, P * Q, total);
        return check_launch("conv2d");
      });
      if (rc != NTOPS_OK) return rc;
    }
  }
  return NTOPS_OK;
}

extern "C" int ntops_conv2d_noalloc(int dtype, int64_t N, int64_t C, int64_t H, int64_t W, int64_t K, int64_t R,
                                    int64_t S, int64_t P, int64_t Q, int64_t stride_h, int64_t stride_w,
                                    int64_t pad_h, int64_t pad_w, int64_t dil_h, int64_t dil_w, const void* x,
                                    const int64_t* x_strides, const void* w, const int64_t* w_strides,
                                    const void* bias, int64_t bias_stride, void* out, const int64_t* out_strides,
                                    void* stream) {
  // Bytes one image takes on the workspace path (0 when the problem runs
  // without one); images are processed in chunks that fit the scratch.
  const int64_t per_image = ntops_conv2d_workspace(dtype, 1, C, H, W, K, R, S, P, Q, stride_h, stride_w, pad_h,
                                                   pad_w, dil_h, dil_w, w_strides, out_strides);
  if (per_image > kConvScratchBytes)
    return set_error(NTOPS_ERR_UNSUPPORTED,
                     "conv2d_noalloc: one image needs %lld bytes of scratch, more than the %lld-byte maximum",
                     static_cast<long long>(per_image), static_cast<long long>(kConvScratchBytes));
  void* ws = nullptr;
  if (per_image > 0 && N > 0 && K > 0 && P > 0 && Q > 0) {
    ws = conv_scratch();
    if (ws == nullptr) return NTOPS_ERR_HIP;
  }
  return ntops_conv2d(dtype, N, C, H, W, K, R, S, P, Q, stride_h, stride_w, pad_h, pad_w, dil_h, dil_w, x,
                      x_strides, w, w_strides, bias, bias_stride, out, out_strides, ws, ws ? kConvScratchBytes : 0,
                      stream);
}
