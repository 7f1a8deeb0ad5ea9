// GEMM family (mm / bmm / addmm): out = alpha * (A @ B) + beta * C.
//
// Reference: kernels/mm.py:54-65 (fp32 accumulator over K tiles, output
// rounded to the input dtype), kernels/bmm.py:26-39 (batch tile of 1),
// kernels/addmm.py:64-67 (beta * input + alpha * mm).
//
// MFMA path (bf16 / fp16 with 16-byte aligned, unit-stride operands):
//  * macro tile BM x BN x 64, WM x WN wavefronts, each wave owns a
//    (BM/WM) x (BN/WN) sub-tile built from 32x32 v_mfma_f32_32x32x16_{bf16,f16}
//    tiles with fp32 accumulators;
//  * both operands are staged in LDS as [row][k] (row = m for A, n for B),
//    128 B per row, 16-byte chunks XOR-swizzled by ((row>>1)+(row>>4))&7 so
//    fragment reads (ds_read_b128) are conflict-free;
//  * a K-major operand is copied chunk-for-chunk; an M/N-major operand (e.g.
//    B of a row-major K x N matrix) is loaded as 4(k) x 8(n) blocks and
//    transposed in registers on its way into LDS;
//  * two LDS stages: global loads of tile k+1 are in flight while tile k is
//    multiplied; one barrier per K tile;
//  * the MFMA is issued with B as its first operand, so each lane ends up
//    holding 4 consecutive output columns of one row: the epilogue applies
//    alpha / beta in fp32, rounds once and writes 8-byte stores;
//  * tiles are assigned XCD-aware: consecutive workgroups land on different
//    XCDs (round-robin dispatch), so the tile order is remapped to give each
//    XCD a contiguous, M-grouped range of tiles sharing A and B panels in its
//    own L2.
// Generic path (fp32, or any other strides): 64x64 LDS-tiled FMA kernel with
// fp32 accumulation (IEEE; gfx950 has no reduced-precision fp32 MFMA input).
#include "dispatch.h"

namespace ntops {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <typename T>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (std::is_same<T, __bf16>::value)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

struct GemmArgs {
  const void* A;
  const void* B;
  const void* C;
  void* D;
  int64_t sa_b, sa_m, sa_k;
  int64_t sb_b, sb_k, sb_n;
  int64_t sc_b, sc_m, sc_n;
  int64_t sd_b, sd_m, sd_n;
  int M, N, K, batch;
  float alpha, beta;
  int use_c;
};

constexpr int kBK = 64;
constexpr int kRowBytes = kBK * 2;  // one LDS row of 64 16-bit k values

__device__ __forceinline__ int swz(int row) { return ((row >> 1) + (row >> 4)) & 7; }
__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * kRowBytes + ((chunk ^ swz(row)) << 4);
}

// Maps a linear workgroup id to (batch, tile_m, tile_n).
__device__ __forceinline__ void tile_of(int pid, int nblocks, int tm_count, int tn_count,
                                        int& bat, int& tm, int& tn) {
  // Workgroups are dispatched round-robin over the 8 XCDs; make the ids an
  // XCD sees consecutive in tile order.
  if ((nblocks & 7) == 0) pid = (pid & 7) * (nblocks >> 3) + (pid >> 3);
  const int per_batch = tm_count * tn_count;
  bat = pid / per_batch;
  const int t = pid - bat * per_batch;
  constexpr int kGroupM = 8;
  const int group_size = kGroupM * tn_count;
  const int g = t / group_size;
  const int first_m = g * kGroupM;
  const int gm = min(tm_count - first_m, kGroupM);
  const int r = t - g * group_size;
  tm = first_m + r % gm;
  tn = r / gm;
}

// ---- global -> register staging ------------------------------------------
// K-major operand: R rows x 64 k, 16-byte chunks (8 per row).
template <int R, int NT, bool EVEN>
struct KMajorLoader {
  static constexpr int kChunks = R * 8 / NT;
  u32x4 v[kChunks];
  __device__ __forceinline__ void load(const uint16_t* base, int64_t s_row, int row0, int rows,
                                       int k0, int K, int t) {
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int c = t + i * NT;
      const int r = c >> 3, kc = c & 7;
      const int gr = row0 + r, gk = k0 + kc * 8;
      if (EVEN || (gr < rows && gk < K))
        v[i] = *reinterpret_cast<const u32x4*>(base + gr * s_row + gk);
      else
        v[i] = u32x4{0, 0, 0, 0};
    }
  }
  __device__ __forceinline__ void store(char* lds, int t) const {
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int c = t + i * NT;
      const int r = c >> 3, kc = c & 7;
      *reinterpret_cast<u32x4*>(lds + lds_off(r, kc)) = v[i];
    }
  }
};

// M/N-major operand: 64 k x R (contiguous) columns, loaded as 4(k) x 8(col)
// blocks and transposed to [col][k] in registers.
template <int R, int NT, bool EVEN>
struct MNMajorLoader {
  static constexpr int kItems = 16 * (R / 8) / NT;
  u32x4 v[kItems][4];
  __device__ __forceinline__ static void item(int it, int& ng, int& kg) {
    ng = (it & 7) + 8 * ((it >> 3) >> 4);
    kg = (it >> 3) & 15;
  }
  __device__ __forceinline__ void load(const uint16_t* base, int64_t s_k, int col0, int cols,
                                       int k0, int K, int t) {
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
      int ng, kg;
      item(t + i * NT, ng, kg);
      const int gc = col0 + ng * 8;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gk = k0 + kg * 4 + r;
        if (EVEN || (gc < cols && gk < K))
          v[i][r] = *reinterpret_cast<const u32x4*>(base + gk * s_k + gc);
        else
          v[i][r] = u32x4{0, 0, 0, 0};
      }
    }
  }
  __device__ __forceinline__ void store(char* lds, int t) const {
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
      int ng, kg;
      item(t + i * NT, ng, kg);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        // column 2d takes the low halves, column 2d+1 the high halves.
        u32x2 lo, hi;
        lo.x = (v[i][0][d] & 0xffffu) | (v[i][1][d] << 16);
        lo.y = (v[i][2][d] & 0xffffu) | (v[i][3][d] << 16);
        hi.x = (v[i][0][d] >> 16) | (v[i][1][d] & 0xffff0000u);
        hi.y = (v[i][2][d] >> 16) | (v[i][3][d] & 0xffff0000u);
        const int c0 = ng * 8 + 2 * d;
        const int kb = kg * 8;  // byte offset of these 4 k values in the row
        *reinterpret_cast<u32x2*>(lds + lds_off(c0, kb >> 4) + (kb & 8)) = lo;
        *reinterpret_cast<u32x2*>(lds + lds_off(c0 + 1, kb >> 4) + (kb & 8)) = hi;
      }
    }
  }
};

template <int R, int NT, bool KMAJ, bool EVEN>
using Loader = typename std::conditional<KMAJ, KMajorLoader<R, NT, EVEN>, MNMajorLoader<R, NT, EVEN>>::type;

// ---- MFMA kernel -----------------------------------------------------------
template <typename T, int BM, int BN, int WM, int WN, bool AK, bool BK_, bool EVEN>
__global__ __launch_bounds__(WM* WN * 64) void k_gemm_mfma(GemmArgs g) {
  constexpr int NT = WM * WN * 64;
  constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  constexpr int TM = WTM / 32, TN = WTN / 32;  // 32x32 MFMA tiles per wave
  constexpr int kStage = (BM + BN) * kRowBytes;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const int tm_count = (g.M + BM - 1) / BM, tn_count = (g.N + BN - 1) / BN;
  int bat, tmi, tni;
  tile_of(blockIdx.x, gridDim.x, tm_count, tn_count, bat, tmi, tni);
  const int m0 = tmi * BM, n0 = tni * BN;

  const uint16_t* A = static_cast<const uint16_t*>(g.A) + bat * g.sa_b;
  const uint16_t* B = static_cast<const uint16_t*>(g.B) + bat * g.sb_b;
  // Pointers at the tile origin (row/col offsets folded in).
  const uint16_t* Ab = AK ? A + static_cast<int64_t>(m0) * g.sa_m : A + m0;
  const uint16_t* Bb = BK_ ? B + static_cast<int64_t>(n0) * g.sb_n : B + n0;
  const int a_rows = g.M - m0, b_cols = g.N - n0;

  Loader<BM, NT, AK, EVEN> la;
  Loader<BN, NT, BK_, EVEN> lb;

  auto load_tile = [&](int k0) {
    if constexpr (AK)
      la.load(Ab, g.sa_m, 0, a_rows, k0, g.K, t);
    else
      la.load(Ab, g.sa_k, 0, a_rows, k0, g.K, t);
    if constexpr (BK_)
      lb.load(Bb, g.sb_n, 0, b_cols, k0, g.K, t);
    else
      lb.load(Bb, g.sb_k, 0, b_cols, k0, g.K, t);
  };
  auto store_tile = [&](int stage) {
    char* base = smem + stage * kStage;
    la.store(base, t);
    lb.store(base + BM * kRowBytes, t);
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int ktiles = (g.K + kBK - 1) / kBK;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  const int frow = lane & 31, fchunk = lane >> 5;
  for (int kt = 0; kt < ktiles; ++kt) {
    const int stage = kt & 1;
    const bool more = kt + 1 < ktiles;
    if (more) load_tile((kt + 1) * kBK);
    const char* sa = smem + stage * kStage;
    const char* sb = sa + BM * kRowBytes;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      u32x4 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const u32x4*>(sa + lds_off(wm * WTM + i * 32 + frow, ks * 2 + fchunk));
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bf[j] = *reinterpret_cast<const u32x4*>(sb + lds_off(wn * WTN + j * 32 + frow, ks * 2 + fchunk));
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma32<T>(bf[j], af[i], acc[i][j]);
    }
    if (more) store_tile(stage ^ 1);
    __syncthreads();
  }

  // Epilogue.  With B as the first MFMA operand, lane l of tile (i, j) holds
  // output row  m = l & 31  and columns  n = 8q + 4(l >> 5) + 0..3  in
  // acc[i][j][4q .. 4q+3].
  T* D = static_cast<T*>(g.D) + bat * g.sd_b;
  const T* Cp = g.use_c ? static_cast<const T*>(g.C) + bat * g.sc_b : nullptr;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm * WTM + i * 32 + (lane & 31);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * WTN + j * 32 + q * 8 + (lane >> 5) * 4;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = g.alpha * acc[i][j][4 * q + e];
        if (EVEN || (m < g.M && n + 3 < g.N)) {
          if (Cp != nullptr) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              v[e] += g.beta * static_cast<float>(Cp[m * g.sc_m + (n + e) * g.sc_n]);
          }
          T o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = static_cast<T>(v[e]);
          *reinterpret_cast<u32x2*>(D + static_cast<int64_t>(m) * g.sd_m + n) =
              __builtin_bit_cast(u32x2, o);
        } else if (m < g.M) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (n + e < g.N) {
              float r = v[e];
              if (Cp != nullptr) r += g.beta * static_cast<float>(Cp[m * g.sc_m + (n + e) * g.sc_n]);
              D[static_cast<int64_t>(m) * g.sd_m + n + e] = static_cast<T>(r);
            }
          }
        }
      }
    }
  }
}

// ---- generic kernel (any dtype among F32/F16/BF16, any strides) -------------
template <typename T>
__global__ __launch_bounds__(256) void k_gemm_generic(GemmArgs g) {
  constexpr int BT = 64, KT = 16;
  __shared__ float As[KT][BT + 1];
  __shared__ float Bs[KT][BT + 1];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int tiles_n = (g.N + BT - 1) / BT;
  const int tiles_m = (g.M + BT - 1) / BT;
  const int per_batch = tiles_m * tiles_n;
  const int bat = blockIdx.x / per_batch;
  const int t = blockIdx.x - bat * per_batch;
  const int m0 = (t / tiles_n) * BT, n0 = (t % tiles_n) * BT;
  const T* A = static_cast<const T*>(g.A) + bat * g.sa_b;
  const T* B = static_cast<const T*>(g.B) + bat * g.sb_b;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < g.K; k0 += KT) {
    for (int e = threadIdx.x; e < KT * BT; e += 256) {
      const int kk = e / BT, mm = e % BT;
      const int gm = m0 + mm, gk = k0 + kk;
      As[kk][mm] = (gm < g.M && gk < g.K) ? static_cast<float>(A[gm * g.sa_m + gk * g.sa_k]) : 0.f;
      const int gn = n0 + mm;
      Bs[kk][mm] = (gn < g.N && gk < g.K) ? static_cast<float>(B[gk * g.sb_k + gn * g.sb_n]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
  T* D = static_cast<T*>(g.D) + bat * g.sd_b;
  const T* Cp = g.use_c ? static_cast<const T*>(g.C) + bat * g.sc_b : nullptr;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + ty * 4 + i;
    if (m >= g.M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tx * 4 + j;
      if (n >= g.N) continue;
      float v = g.alpha * acc[i][j];
      if (Cp != nullptr) v += g.beta * static_cast<float>(Cp[m * g.sc_m + n * g.sc_n]);
      D[m * g.sd_m + n * g.sd_n] = static_cast<T>(v);
    }
  }
}

// ---- host dispatch ---------------------------------------------------------
template <typename T, int BM, int BN, int WM, int WN, bool AK, bool BKM, bool EVEN>
int launch_mfma(const GemmArgs& g, hipStream_t st) {
  constexpr int NT = WM * WN * 64;
  constexpr int kLds = 2 * (BM + BN) * kRowBytes;
  auto kern = k_gemm_mfma<T, BM, BN, WM, WN, AK, BKM, EVEN>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLds) != hipSuccess)
      return set_error(NTOPS_ERR_HIP, "gemm: cannot reserve %d bytes of LDS", kLds);
    attr_set = true;
  }
  const int64_t tiles = static_cast<int64_t>((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN) * g.batch;
  if (tiles > 0x7fffffffLL) return set_error(NTOPS_ERR_UNSUPPORTED, "gemm: too many tiles");
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(tiles)), dim3(NT), kLds, st, g);
  return check_launch("gemm");
}

template <typename T, bool AK, bool BKM>
int pick_tile(const GemmArgs& g, hipStream_t st) {
  const int64_t big_tiles = static_cast<int64_t>((g.M + 255) / 256) * ((g.N + 255) / 256) * g.batch;
  if (big_tiles >= 240) {
    const bool even = g.M % 256 == 0 && g.N % 256 == 0 && g.K % kBK == 0;
    if (even) return launch_mfma<T, 256, 256, 2, 4, AK, BKM, true>(g, st);
    return launch_mfma<T, 256, 256, 2, 4, AK, BKM, false>(g, st);
  }
  const bool even = g.M % 128 == 0 && g.N % 128 == 0 && g.K % kBK == 0;
  if (even) return launch_mfma<T, 128, 128, 2, 2, AK, BKM, true>(g, st);
  return launch_mfma<T, 128, 128, 2, 2, AK, BKM, false>(g, st);
}

template <typename T>
int run_gemm(GemmArgs g, hipStream_t st) {
  if constexpr (!std::is_same<T, float>::value) {
    const auto al = [](const void* p) { return aligned16(p); };
    // A: K-major (row-major M x K) or M-major (column-major).
    const bool a_k = g.sa_k == 1 && g.sa_m % 8 == 0 && g.K % 8 == 0;
    const bool a_m = g.sa_m == 1 && g.sa_k % 8 == 0 && g.M % 8 == 0 && !a_k;
    const bool b_k = g.sb_k == 1 && g.sb_n % 8 == 0 && g.K % 8 == 0;
    const bool b_n = g.sb_n == 1 && g.sb_k % 8 == 0 && g.N % 8 == 0 && !b_k;
    const bool d_ok = g.sd_n == 1 && g.sd_m % 4 == 0 && g.sd_b % 4 == 0 &&
                      (reinterpret_cast<uintptr_t>(g.D) & 7u) == 0 && g.N % 4 == 0;
    const bool batch_ok = (g.batch == 1) || (g.sa_b % 8 == 0 && g.sb_b % 8 == 0);
    const bool fits = static_cast<int64_t>(g.M) * g.sd_m < (int64_t(1) << 31) &&
                      static_cast<int64_t>(g.M) * (a_k ? g.sa_m : 1) < (int64_t(1) << 31) &&
                      static_cast<int64_t>(g.K) * (a_k ? 1 : g.sa_k) < (int64_t(1) << 31) &&
                      static_cast<int64_t>(g.N) * (b_k ? g.sb_n : 1) < (int64_t(1) << 31) &&
                      static_cast<int64_t>(g.K) * (b_k ? 1 : g.sb_k) < (int64_t(1) << 31) &&
                      (!g.use_c || (static_cast<int64_t>(g.M) * (g.sc_m < 0 ? -g.sc_m : g.sc_m) +
                                        static_cast<int64_t>(g.N) * (g.sc_n < 0 ? -g.sc_n : g.sc_n) <
                                    (int64_t(1) << 31)));
    if ((a_k || a_m) && (b_k || b_n) && d_ok && batch_ok && fits && al(g.A) && al(g.B)) {
      if (a_k && b_n) return pick_tile<T, true, false>(g, st);
      if (a_k && b_k) return pick_tile<T, true, true>(g, st);
      if (a_m && b_n) return pick_tile<T, false, false>(g, st);
      return pick_tile<T, false, true>(g, st);
    }
  }
  const int64_t tiles = static_cast<int64_t>((g.M + 63) / 64) * ((g.N + 63) / 64) * g.batch;
  if (tiles > 0x7fffffffLL) return set_error(NTOPS_ERR_UNSUPPORTED, "gemm: too many tiles");
  hipLaunchKernelGGL((k_gemm_generic<T>), dim3(static_cast<unsigned>(tiles)), dim3(256), 0, st, g);
  return check_launch("gemm");
}

}  // namespace
}  // namespace ntops

using namespace ntops;

extern "C" int ntops_gemm(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K,
                          const void* A, const int64_t* a_strides, const void* B,
                          const int64_t* b_strides, const void* C, const int64_t* c_strides,
                          double alpha, double beta, void* out, const int64_t* out_strides,
                          void* stream) {
  if (batch < 0 || M < 0 || N < 0 || K < 0) return set_error(NTOPS_ERR_INVALID, "gemm: negative size");
  if (batch > 0x7fffffffLL || M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL)
    return set_error(NTOPS_ERR_UNSUPPORTED, "gemm: size exceeds int32");
  if (batch == 0 || M == 0 || N == 0) return NTOPS_OK;
  if (out == nullptr || out_strides == nullptr || a_strides == nullptr || b_strides == nullptr)
    return set_error(NTOPS_ERR_INVALID, "gemm: null pointer");
  if (K > 0 && (A == nullptr || B == nullptr)) return set_error(NTOPS_ERR_INVALID, "gemm: null operand");
  GemmArgs g;
  g.A = A;
  g.B = B;
  g.D = out;
  g.sa_b = a_strides[0];
  g.sa_m = a_strides[1];
  g.sa_k = a_strides[2];
  g.sb_b = b_strides[0];
  g.sb_k = b_strides[1];
  g.sb_n = b_strides[2];
  g.sd_b = out_strides[0];
  g.sd_m = out_strides[1];
  g.sd_n = out_strides[2];
  g.M = static_cast<int>(M);
  g.N = static_cast<int>(N);
  g.K = static_cast<int>(K);
  g.batch = static_cast<int>(batch);
  g.alpha = static_cast<float>(alpha);
  g.beta = static_cast<float>(beta);
  g.use_c = (C != nullptr && beta != 0.0) ? 1 : 0;
  g.C = C;
  if (g.use_c) {
    if (c_strides == nullptr) return set_error(NTOPS_ERR_INVALID, "gemm: null C strides");
    g.sc_b = c_strides[0];
    g.sc_m = c_strides[1];
    g.sc_n = c_strides[2];
  } else {
    g.sc_b = g.sc_m = g.sc_n = 0;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  return dispatch_float16_32(dtype, "gemm", [&](auto tag) {
    using T = decltype(tag);
    return run_gemm<T>(g, st);
  });
}
