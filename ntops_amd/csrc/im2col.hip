// im2col: out[n][(c * kh + r) * kw + s][p * ow + q] =
//     x[n][c][p * sh - ph + r * dh][q * sw - pw + s * dw]   (zero outside the image)
//
// Reference: kernels/im2col.py:10-80 (input padded on both sides, tiled into
// kh x kw windows with strides and dilation in floor mode, each window's
// (c, r, s) elements along the output's middle axis), torch/im2col.py:44-135
// (argument forms, output size, checks).
//
// Pure data movement: the kernels are templated on the element size (1, 2, 4
// or 8 bytes) and move every dtype as its bits.  A thread owns a run of 8
// consecutive output pixels (p, q) of one (image, channel) and writes that run
// into each of the kh * kw tap rows; the run's pixel positions are computed
// once and reused for every tap.
//  * plane kernel (the (image, channel) plane fits in 64 KiB): one workgroup
//    per plane stages it in LDS with neighbouring threads loading
//    neighbouring elements, so the input is read from HBM once and the taps
//    gather from LDS;
//  * direct kernel (larger planes): a grid-stride loop over (image, channel,
//    run) items whose taps gather from global memory (L2).
// When every output row starts on a multiple of the run's byte size (capped
// at 16 bytes), whole runs are written with full-width non-temporal vector
// stores (the output is written once and is kh * kw times the input: on the
// (32, 256, 56, 56) 3x3 bf16 unfold they move 86 instead of 99 us);
// otherwise (and for a row's last, partial run) element by element.
//  * stride-1 kernel (16-bit elements, stride and dilation 1, output rows a
//    multiple of 8 pixels, vector stores): the plane is staged in LDS with
//    its zero padding around it, so a run's 8 + kw - 1 input elements under
//    kernel row r are one aligned 32-byte LDS read and the kw taps are
//    register selections (even taps) or 16-bit funnel shifts (odd taps) of
//    it -- no per-element bounds tests or gathers.
#include "dispatch.h"

namespace ntops {
namespace {

struct Im2colArgs {
  const void* x;
  void* out;
  int64_t xs[4];
  int64_t os[3];
  int N, C, H, W;
  int kh, kw, dh, dw, ph, pw, sh, sw;
  int oh, ow, L, runs;
};

template <int ES> struct Bits;
template <> struct Bits<1> { using U = uint8_t; };
template <> struct Bits<2> { using U = uint16_t; };
template <> struct Bits<4> { using U = uint32_t; };
template <> struct Bits<8> { using U = uint64_t; };

constexpr int kRun = 8;
constexpr int kIm2colPlaneLds = 64 * 1024;

// Row and column bases of the run's 8 pixels: hb = p * sh - ph (a sentinel
// far outside the image past the last pixel), wb = q * sw - pw.
__device__ __forceinline__ void run_bases(const Im2colArgs& a, int j0, int (&hb)[kRun], int (&wb)[kRun]) {
  int p = j0 / a.ow;
  int q = j0 - p * a.ow;
#pragma unroll
  for (int e = 0; e < kRun; ++e) {
    hb[e] = j0 + e < a.L ? p * a.sh - a.ph : -0x40000000;
    wb[e] = q * a.sw - a.pw;
    if (++q == a.ow) {
      q = 0;
      ++p;
    }
  }
}

template <int ES, bool VEC>
__device__ __forceinline__ void store_run(const Im2colArgs& a, char* row, int j0,
                                          const typename Bits<ES>::U (&v)[kRun]) {
  using U = typename Bits<ES>::U;
  if constexpr (VEC) {
    if (j0 + kRun <= a.L) {
      char* dst = row + static_cast<int64_t>(j0) * ES;
      if constexpr (ES == 1) {
        __builtin_nontemporal_store(__builtin_bit_cast(uint64_t, v), reinterpret_cast<uint64_t*>(dst));
      } else {
        struct Chunks {
          u32x4 c[ES * kRun / 16];
        };
        const Chunks ch = __builtin_bit_cast(Chunks, v);
#pragma unroll
        for (int i = 0; i < ES * kRun / 16; ++i) __builtin_nontemporal_store(ch.c[i], reinterpret_cast<u32x4*>(dst) + i);
      }
      return;
    }
  }
  U* dst = reinterpret_cast<U*>(row);
#pragma unroll
  for (int e = 0; e < kRun; ++e)
    if (j0 + e < a.L) dst[static_cast<int64_t>(j0 + e) * a.os[2]] = v[e];
}

// Writes the run starting at output pixel j0 of plane (n, c) into every tap
// row; `at(ih, iw)` returns the input element (only called inside the image).
template <int ES, bool VEC, typename At>
__device__ __forceinline__ void write_taps(const Im2colArgs& a, int n, int c, int j0, At at) {
  using U = typename Bits<ES>::U;
  int hb[kRun], wb[kRun];
  run_bases(a, j0, hb, wb);
  char* out = static_cast<char*>(a.out) + (static_cast<int64_t>(n) * a.os[0] +
                                           static_cast<int64_t>(c) * a.kh * a.kw * a.os[1]) * ES;
  for (int r = 0; r < a.kh; ++r) {
    for (int s = 0; s < a.kw; ++s) {
      U v[kRun];
#pragma unroll
      for (int e = 0; e < kRun; ++e) {
        const int ih = hb[e] + r * a.dh;
        const int iw = wb[e] + s * a.dw;
        const bool in = static_cast<unsigned>(ih) < static_cast<unsigned>(a.H) &&
                        static_cast<unsigned>(iw) < static_cast<unsigned>(a.W);
        v[e] = in ? at(ih, iw) : U(0);
      }
      store_run<ES, VEC>(a, out + static_cast<int64_t>(r * a.kw + s) * a.os[1] * ES, j0, v);
    }
  }
}

template <int ES, bool VEC>
__global__ __launch_bounds__(256) void k_im2col_lds(Im2colArgs a) {
  using U = typename Bits<ES>::U;
  extern __shared__ __attribute__((aligned(16))) char sm[];
  U* plane = reinterpret_cast<U*>(sm);
  const int64_t id = block_id();  // (image, channel) plane; blocks_2d grid
  if (id >= static_cast<int64_t>(a.N) * a.C) return;  // the tail of the grid (the whole block)
  const int n = static_cast<int>(id / a.C);
  const int c = static_cast<int>(id - static_cast<int64_t>(n) * a.C);
  const U* x = static_cast<const U*>(a.x) + n * a.xs[0] + c * a.xs[1];
  const int hw = a.H * a.W;
  for (int i = threadIdx.x; i < hw; i += blockDim.x) {
    const int ih = i / a.W, iw = i - (i / a.W) * a.W;
    plane[i] = x[ih * a.xs[2] + iw * a.xs[3]];
  }
  __syncthreads();
  for (int run = threadIdx.x; run < a.runs; run += blockDim.x)
    write_taps<ES, VEC>(a, n, c, run * kRun, [&](int ih, int iw) { return plane[ih * a.W + iw]; });
}

template <int ES, bool VEC>
__global__ __launch_bounds__(256) void k_im2col_direct(Im2colArgs a, int64_t items) {
  using U = typename Bits<ES>::U;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < items;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int run = static_cast<int>(i % a.runs);
    const int64_t nc = i / a.runs;
    const int n = static_cast<int>(nc / a.C);
    const int c = static_cast<int>(nc - static_cast<int64_t>(n) * a.C);
    const U* x = static_cast<const U*>(a.x) + n * a.xs[0] + c * a.xs[1];
    write_taps<ES, VEC>(a, n, c, run * kRun,
                        [&](int ih, int iw) { return x[ih * a.xs[2] + iw * a.xs[3]]; });
  }
}


// Stride 1, dilation 1, ES == 2, ow % 8 == 0, KW <= 9, VEC stores.  LDS holds
// the plane zero-padded: row ih + ph, column iw + pw, `pitch` (a multiple of
// 8, >= ow + 8) elements per row, H + 2 ph rows.  Output pixel (p, q) under
// tap (r, s) is padded element (p + r, q + s), so the run at (p, q0) reads
// padded row p + r, columns q0 .. q0 + 15 (two 16-byte reads; q0 and pitch
// are multiples of 8) and tap s takes elements s .. s + 7 of them.
template <int KW>
__global__ __launch_bounds__(512) void k_im2col_s1(Im2colArgs a, int pitch, int vec_in) {
  extern __shared__ __attribute__((aligned(16))) char sm[];
  uint16_t* plane = reinterpret_cast<uint16_t*>(sm);
  const int64_t id = block_id();  // (image, channel) plane; blocks_2d grid
  if (id >= static_cast<int64_t>(a.N) * a.C) return;  // the tail of the grid (the whole block)
  const int n = static_cast<int>(id / a.C);
  const int c = static_cast<int>(id - static_cast<int64_t>(n) * a.C);
  const int hp = a.H + 2 * a.ph;
  for (int i = threadIdx.x; i < hp * pitch / 8; i += blockDim.x) reinterpret_cast<u32x4*>(sm)[i] = u32x4{0u, 0u, 0u, 0u};
  __syncthreads();
  const uint16_t* x = static_cast<const uint16_t*>(a.x) + n * a.xs[0] + c * a.xs[1];
  if (vec_in) {  // unit column stride, rows of a multiple of 8 elements, 16-byte aligned
    const int w8 = a.W / 8;
    for (int i = threadIdx.x; i < a.H * w8; i += blockDim.x) {
      const int ih = i / w8, iw = (i - ih * w8) * 8;
      const u32x4 v = *reinterpret_cast<const u32x4*>(x + ih * a.xs[2] + iw);
      // 2-byte stores kept apart (relaxed atomic stores are not merged): with
      // pw odd the destination is only 2-byte aligned, and merged they would
      // form a misaligned 16-byte LDS store
      uint16_t* d = plane + (ih + a.ph) * pitch + iw + a.pw;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        __hip_atomic_store(d + 2 * k, static_cast<uint16_t>(v[k]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        __hip_atomic_store(d + 2 * k + 1, static_cast<uint16_t>(v[k] >> 16), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
  } else {
    for (int i = threadIdx.x; i < a.H * a.W; i += blockDim.x) {
      const int ih = i / a.W, iw = i - ih * a.W;
      plane[(ih + a.ph) * pitch + iw + a.pw] = x[ih * a.xs[2] + iw * a.xs[3]];
    }
  }
  __syncthreads();
  char* out = static_cast<char*>(a.out) + (static_cast<int64_t>(n) * a.os[0] +
                                           static_cast<int64_t>(c) * a.kh * KW * a.os[1]) * 2;
  for (int run = threadIdx.x; run < a.runs; run += blockDim.x) {
    const int j0 = run * kRun;
    const int p = j0 / a.ow, q0 = j0 - p * a.ow;
    for (int r = 0; r < a.kh; ++r) {
      const u32x4* src = reinterpret_cast<const u32x4*>(plane + (p + r) * pitch + q0);
      const u32x4 lo = src[0], hi = src[1];
      const uint32_t d[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};  // elements 2k, 2k + 1
#pragma unroll
      for (int s = 0; s < KW; ++s) {
        u32x4 o;
#pragma unroll
        for (int k = 0; k < 4; ++k)
          o[k] = (s & 1) ? __builtin_amdgcn_alignbit(d[s / 2 + k + 1], d[s / 2 + k], 16) : d[s / 2 + k];
        __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(out + (static_cast<int64_t>(r * KW + s) * a.os[1] + j0) * 2));
      }
    }
  }
}

// Row pitch (elements) of the stride-1 kernel's padded plane, or 0 when the
// problem is not one it handles (including a padded plane over 64 KiB).
int s1_pitch(const Im2colArgs& a) {
  if (a.sh != 1 || a.sw != 1 || a.dh != 1 || a.dw != 1 || a.ow % kRun != 0 || a.kw > 9) return 0;
  const int64_t w = std::max<int64_t>(static_cast<int64_t>(a.W) + 2 * a.pw, static_cast<int64_t>(a.ow) + 8);
  const int64_t pitch = (w + 7) / 8 * 8;
  if ((static_cast<int64_t>(a.H) + 2 * a.ph) * pitch * 2 > kIm2colPlaneLds) return 0;
  return static_cast<int>(pitch);
}

template <int KW>
int launch_s1(const Im2colArgs& a, int pitch, hipStream_t st) {
  const bool vec_in = a.xs[3] == 1 && a.W % 8 == 0 && a.xs[2] % 8 == 0 && a.xs[1] % 8 == 0 && a.xs[0] % 8 == 0 &&
                      (reinterpret_cast<uintptr_t>(a.x) & 15u) == 0;
  const int threads = static_cast<int>(std::min<int64_t>(512, (std::max(a.runs, 64) + 63) / 64 * 64));
  const unsigned lds = static_cast<unsigned>((static_cast<int64_t>(a.H) + 2 * a.ph) * pitch * 2);
  note_kernel("im2col_s1 kw%d", KW);
  hipLaunchKernelGGL(k_im2col_s1<KW>, blocks_2d(static_cast<int64_t>(a.N) * a.C), dim3(threads),
                     lds, st, a, pitch, vec_in ? 1 : 0);
  return check_launch("im2col");
}

int run_s1(const Im2colArgs& a, int pitch, hipStream_t st) {
  switch (a.kw) {
    case 1: return launch_s1<1>(a, pitch, st);
    case 2: return launch_s1<2>(a, pitch, st);
    case 3: return launch_s1<3>(a, pitch, st);
    case 4: return launch_s1<4>(a, pitch, st);
    case 5: return launch_s1<5>(a, pitch, st);
    case 6: return launch_s1<6>(a, pitch, st);
    case 7: return launch_s1<7>(a, pitch, st);
    case 8: return launch_s1<8>(a, pitch, st);
    default: return launch_s1<9>(a, pitch, st);
  }
}

template <int ES, bool VEC>
int launch_im2col(const Im2colArgs& a, hipStream_t st) {
  const int64_t planes = static_cast<int64_t>(a.N) * a.C;
  const int64_t plane_bytes = static_cast<int64_t>(a.H) * a.W * ES;
  if constexpr (ES == 2 && VEC) {
    const int pitch = s1_pitch(a);
    if (pitch > 0) return run_s1(a, pitch, st);
  }
  if (plane_bytes <= kIm2colPlaneLds) {
    note_kernel("im2col_lds es%d %s", ES, VEC ? "vec" : "scalar");
    hipLaunchKernelGGL((k_im2col_lds<ES, VEC>), blocks_2d(planes), dim3(256),
                       static_cast<unsigned>(plane_bytes), st, a);
    return check_launch("im2col");
  }
  const int64_t items = planes * a.runs;
  int64_t grid = (items + 255) / 256;
  if (grid > 65536) grid = 65536;
  note_kernel("im2col_direct es%d %s", ES, VEC ? "vec" : "scalar");
  hipLaunchKernelGGL((k_im2col_direct<ES, VEC>), dim3(static_cast<unsigned>(grid)), dim3(256), 0, st, a, items);
  return check_launch("im2col");
}

template <int ES>
int run_im2col(const Im2colArgs& a, hipStream_t st) {
  // Whole runs can be stored as one vector when every row (and the base)
  // starts on the run's byte size, capped at 16 bytes.
  constexpr int kAlign = ES * kRun < 16 ? ES * kRun : 16;
  const bool vec = a.os[2] == 1 && (a.os[1] * ES) % kAlign == 0 && (a.os[0] * ES) % kAlign == 0 &&
                   (reinterpret_cast<uintptr_t>(a.out) % kAlign) == 0;
  return vec ? launch_im2col<ES, true>(a, st) : launch_im2col<ES, false>(a, st);
}

}  // namespace
}  // namespace ntops

using namespace ntops;

extern "C" int ntops_im2col(int dtype, int64_t N, int64_t C, int64_t H, int64_t W, int64_t kernel_h,
                            int64_t kernel_w, int64_t dil_h, int64_t dil_w, int64_t pad_h, int64_t pad_w,
                            int64_t stride_h, int64_t stride_w, const void* x, const int64_t* x_strides,
                            void* out, const int64_t* out_strides, void* stream) {
  const int es = dtype_size(dtype);
  if (es == 0) return set_error(NTOPS_ERR_UNSUPPORTED, "im2col: unknown dtype %d", dtype);
  const int64_t v[] = {N, C, H, W, kernel_h, kernel_w, dil_h, dil_w, pad_h, pad_w, stride_h, stride_w};
  for (int64_t s : v)
    if (s < 0 || s > 0x7fffffffLL) return set_error(NTOPS_ERR_INVALID, "im2col: size or parameter out of range");
  if (kernel_h < 1 || kernel_w < 1) return set_error(NTOPS_ERR_INVALID, "im2col: kernel_size should be greater than zero");
  if (dil_h < 1 || dil_w < 1) return set_error(NTOPS_ERR_INVALID, "im2col: dilation should be greater than zero");
  if (stride_h < 1 || stride_w < 1) return set_error(NTOPS_ERR_INVALID, "im2col: stride should be greater than zero");
  const int64_t oh = (H + 2 * pad_h - dil_h * (kernel_h - 1) - 1) / stride_h + 1;
  const int64_t ow = (W + 2 * pad_w - dil_w * (kernel_w - 1) - 1) / stride_w + 1;
  // (the numerators may be negative: C division truncates toward zero, so
  // test them directly rather than the quotients)
  if (H + 2 * pad_h - dil_h * (kernel_h - 1) - 1 < 0 || W + 2 * pad_w - dil_w * (kernel_w - 1) - 1 < 0 || oh < 1 ||
      ow < 1)
    return set_error(NTOPS_ERR_INVALID, "im2col: the output size must be at least one");
  // keeps every row / column position (and the past-the-end sentinel plus a
  // tap offset) inside int32
  if (H + 2 * pad_h > (int64_t(1) << 30) || W + 2 * pad_w > (int64_t(1) << 30) || oh * ow > 0x7fffffffLL - kRun ||
      C * kernel_h * kernel_w > 0x7fffffffLL)
    return set_error(NTOPS_ERR_UNSUPPORTED, "im2col: sizes exceed the int32 index range");
  if (N == 0 || C == 0) return NTOPS_OK;
  if (x == nullptr || out == nullptr || x_strides == nullptr || out_strides == nullptr)
    return set_error(NTOPS_ERR_INVALID, "im2col: null pointer");
  Im2colArgs a{};
  a.x = x;
  a.out = out;
  for (int i = 0; i < 4; ++i) a.xs[i] = x_strides[i];
  for (int i = 0; i < 3; ++i) a.os[i] = out_strides[i];
  a.N = static_cast<int>(N);
  a.C = static_cast<int>(C);
  a.H = static_cast<int>(H);
  a.W = static_cast<int>(W);
  a.kh = static_cast<int>(kernel_h);
  a.kw = static_cast<int>(kernel_w);
  a.dh = static_cast<int>(dil_h);
  a.dw = static_cast<int>(dil_w);
  a.ph = static_cast<int>(pad_h);
  a.pw = static_cast<int>(pad_w);
  a.sh = static_cast<int>(stride_h);
  a.sw = static_cast<int>(stride_w);
  a.oh = static_cast<int>(oh);
  a.ow = static_cast<int>(ow);
  a.L = static_cast<int>(oh * ow);
  a.runs = (a.L + kRun - 1) / kRun;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (es) {
    case 1: return run_im2col<1>(a, st);
    case 2: return run_im2col<2>(a, st);
    case 4: return run_im2col<4>(a, st);
    default: return run_im2col<8>(a, st);
  }
}
