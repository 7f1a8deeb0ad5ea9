// GEMM family (mm / bmm / addmm): out = alpha * (A @ B) + beta * C.
//
// Reference: kernels/mm.py:54-65 (fp32 accumulator over K tiles, output
// rounded to the input dtype), kernels/bmm.py:26-39 (batch tile of 1),
// kernels/addmm.py:64-67 (beta * input + alpha * mm).
//
// MFMA path (bf16 / fp16 operands with one unit-stride axis each):
//  * macro tile BM x BN x BK (256 x 256 x 32 for large problems, 128 x 128 x
//    32 otherwise), WM x WN wavefronts; each wave owns a (BM/WM) x (BN/WN)
//    sub-tile of 32x32 v_mfma_f32_32x32x16_{bf16,f16} tiles with fp32
//    accumulators;
//  * operands go global -> LDS directly (buffer_load_dwordx4 ... lds): no
//    VGPR staging, no LDS write instructions.  A lane's LDS destination is
//    fixed (M0 + 16 * lane), so the swizzle is applied on the global side:
//    each lane fetches the chunk that belongs at its LDS slot;
//  * K-major operand tile: [row][BK k], 16-byte chunks XOR-swizzled per row
//    (kslot) so the fragment reads (ds_read_b128) are bank-conflict free;
//  * M/N-major operand tile: [BK k][R], chunk c of row k at slot
//    c ^ (4 * (k % 4)); fragments are read with ds_read_b64_tr_b16, which
//    transposes 4(k) x 16 blocks inside each 16-lane group so every lane
//    receives 4 consecutive k of one column (two reads per 32x32x16 operand);
//    the swizzle makes those reads conflict free;
//  * STAGES LDS stages with prefetch distance STAGES - 1, ordered by explicit
//    vmcnt waits and raw s_barrier (the DMA is issued from inline assembly so
//    the compiler does not serialise every LDS read behind it);
//  * ping-pong schedule: the two waves that share a SIMD are in opposite
//    phases -- one reads a K tile's fragments and issues DMA while the other
//    runs the MFMAs of the tile it read before -- so the matrix core is fed
//    across the per-tile barriers;
//  * B is the MFMA's first operand, so each lane holds 4 consecutive output
//    columns of one row; the epilogue applies alpha / beta in fp32, rounds
//    once, stages the wave's tile in LDS and writes full 128-byte row
//    segments with 16-byte stores (8-byte direct stores when the output is
//    not 16-byte aligned);
//  * tiles are assigned XCD-aware: workgroup ids are dispatched round-robin
//    over the 8 XCDs, so ids are remapped to give each XCD a contiguous,
//    M-grouped range of tiles that share A and B panels in its L2;
//  * edges: buffer loads with a per-tile resource; out-of-range chunks get an
//    offset past the resource's extent and read as zero.
// Skinny path (M <= 64, K-major A): 16/32/64-column blocks whose waves
// split K, operands straight to registers in the v_mfma_f32_16x16x32 layout
// (fp32: v_mfma_f32_16x16x4_f32).
// Short-K path (K <= 128, M and N multiples of 128): a persistent kernel
// built around the output stream.
// fp32 tile path (K-major A): v_mfma_f32_16x16x4_f32 wave tiles of 64 x 64,
// 32-deep K tiles shared by the block through two LDS buffers, or (N-major B
// filling the GPU) operands from L2 per wave.
// Generic path (any other strides): 64x64 LDS-tiled FMA kernel with fp32
// accumulation (IEEE; gfx950 has no reduced-precision fp32 MFMA input).
#include "gemm.h"
#include "mfma.h"

namespace ntops {
namespace {

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
  int c_mode;  // epilogue's C access (kCNone / kCStrided / kCVec4 / kCRow), set by set_c_mode
  int staged;  // out is 16-byte aligned with unit column stride and N % 8 == 0
  int ragged;  // out rows are not 8-byte aligned runs with unit column stride: element stores
  int shifted;  // unit column stride, rows not 16-byte aligned: full-tile kernels store shifted 16-byte chunks
  // Split-K (the SPLITK instantiation): block row blockIdx.y takes k in
  // [blockIdx.y * kchunk, min(K, (blockIdx.y + 1) * kchunk)) and writes its
  // fp32 partial tile to part + blockIdx.y * part_stride (rows of N).
  float* part;          // the workspace (null: no split-K)
  int64_t part_bytes;   // its size
  int64_t part_stride;  // M * N
  int kchunk;
  // Implicit convolution operand (used only by the CONV instantiation): B's
  // k-row kg = (c * R + r) * S + s starts at element
  // s * cv_per_s + c * cv_per_c + r * cv_per_r of the batch's B buffer, and
  // its N elements are contiguous from there.
  int cv_rs, cv_r, cv_s;
  int cv_ds, cv_dr, cv_dc;  // BK k-rows expressed as (s, r, c) steps: BK = (dc * R + dr) * S + ds
  int64_t cv_per_s, cv_per_c, cv_per_r;
  // Channels-last convolution operand (CONV == 2): B is K-major with one row
  // per output pixel n of the batch's image, p = n / cl_q, q = n % cl_q,
  // starting at element (p * cl_sh * cl_wp + q * cl_sw) * cl_c of the
  // batch's zero-padded (rows of cl_wp pixels, cl_c channels each) image.
  // k runs over 32-channel blocks, then taps, then the block's channels:
  // k = ((cb * cv_r + r) * cv_s + s) * 32 + ci adds (r * cl_dh * cl_wp +
  // s * cl_dw) * cl_c + 32 * cb + ci, so one K tile is one (block, tap) and
  // the R * S tiles of a block, which read overlapping pixels, follow each
  // other (the reuse stays within L2).
  int cl_q, cl_sh, cl_sw, cl_wp, cl_c, cl_dh, cl_dw;
};


// Waits until at most `younger` tiles' worth of this wave's DMA loads
// (loads_per_tile each) are still in flight.
__device__ __forceinline__ void wait_tile(int younger, int loads_per_tile) {
  const int n = younger * loads_per_tile;
  if (n >= 12)
    wait_vmcnt<12>();
  else if (n >= 8)
    wait_vmcnt<8>();
  else if (n >= 6)
    wait_vmcnt<6>();
  else if (n >= 4)
    wait_vmcnt<4>();
  else if (n >= 2)
    wait_vmcnt<2>();
  else
    wait_vmcnt<0>();
}

// Maps a linear workgroup id to (batch, tile_m, tile_n).
__device__ __forceinline__ void tile_of(int pid, int nblocks, int tm_count, int tn_count,
                                        int& bat, int& tm, int& tn) {
  if ((nblocks & 7) == 0) pid = (pid & 7) * (nblocks >> 3) + (pid >> 3);
  const int per_batch = tm_count * tn_count;
  bat = pid / per_batch;
  const int t = pid - bat * per_batch;
  constexpr int kGroupM = 4;  // 4 measured ~0.7 % over 8 and 2 on mm, 16 ~2.5 % below
  const int group_size = kGroupM * tn_count;
  const int g = t / group_size;
  const int first_m = g * kGroupM;
  const int gm = min(tm_count - first_m, kGroupM);
  const int r = t - g * group_size;
  tm = first_m + r % gm;
  tn = r / gm;
}


// One operand's global -> LDS stream for a tile of R rows/columns x BK k.
// The tile is R * BK * 2 bytes: R * BK / 512 one-KiB load instructions,
// spread evenly over the NW waves of the block.
// CONV: 0 a plain operand; 1 the shifted-plane convolution operand (N-major,
// per-lane k-row bases); 2 the channels-last convolution operand (K-major,
// per-lane pixel bases plus one scalar offset per K tile).
template <int R, bool KMAJ, int NW, bool EVEN, int BK, int CONV = 0>
struct TileLoader {
  static_assert(CONV != 1 || !KMAJ, "the shifted-plane convolution operand is N-major");
  static_assert(CONV != 2 || KMAJ, "the channels-last convolution operand is K-major");
  static constexpr int kInst = R * BK / 512 / NW;
  static_assert(kInst * NW * 512 == R * BK, "tile must split evenly over the waves");
  static constexpr int kCprK = BK / 8;  // chunks per row (K-major)
  static constexpr int kCprMN = R / 8;  // chunks per k-row (M/N-major)
  u32x4 rsrc;             // buffer resource (V#) of the operand tile
  uint32_t voff[kInst];   // byte offset of this lane's chunk at k0 = 0
  int lim_row[kInst];     // K-major: tile row; M/N-major: k-row
  int lim_col[kInst];     // K-major: k of the chunk; M/N-major: column of the chunk
  uint32_t k_stride_bytes;
  int lds_base;           // first instruction's LDS offset inside the operand tile
  // implicit convolution (CONV): this lane's k-row of each instruction for
  // the next tile to issue, as (c, r, s) -- advanced by BK per tile
  int cv_c[CONV == 1 ? kInst : 1], cv_r[CONV == 1 ? kInst : 1], cv_s[CONV == 1 ? kInst : 1];
  // channels-last convolution (CONV == 2): the tap (r, s) and first channel
  // c0 of the next K tile to issue
  int cl_r = 0, cl_s = 0, cl_c0 = 0;

  // base: element pointer at the tile origin; ld: row stride (K-major) or
  // k-row stride (M/N-major), in elements; extent_bytes: readable bytes.
  __device__ __forceinline__ void init(const uint16_t* base, int64_t ld, int64_t extent_bytes,
                                       int wave, int lane) {
    const uint64_t addr = reinterpret_cast<uint64_t>(base);
    rsrc.x = static_cast<uint32_t>(addr);
    rsrc.y = static_cast<uint32_t>(addr >> 32) & 0xffffu;  // stride 0, no swizzle
    rsrc.z = static_cast<uint32_t>(extent_bytes);           // num_records (bytes)
    rsrc.w = 0x00020000u;                                   // 32-bit data format
    rsrc.x = __builtin_amdgcn_readfirstlane(rsrc.x);
    rsrc.y = __builtin_amdgcn_readfirstlane(rsrc.y);
    rsrc.z = __builtin_amdgcn_readfirstlane(rsrc.z);
    lds_base = wave * kInst * 1024;
    if constexpr (KMAJ) {
      k_stride_bytes = 2;
      constexpr int rows_per_inst = 1024 / (BK * 2);
#pragma unroll
      for (int i = 0; i < kInst; ++i) {
        const int q = wave * kInst + i;
        const int row = q * rows_per_inst + lane / kCprK;
        const int c = kslot<BK>(row, lane % kCprK);
        voff[i] = static_cast<uint32_t>(row * ld * 2 + c * 16);
        lim_row[i] = row;
        lim_col[i] = c * 8;
      }
    } else {
      k_stride_bytes = static_cast<uint32_t>(ld * 2);
      constexpr int rows_per_inst = 64 / kCprMN;
#pragma unroll
      for (int i = 0; i < kInst; ++i) {
        const int q = wave * kInst + i;
        const int krow = q * rows_per_inst + lane / kCprMN;
        const int c = mnslot(krow, lane % kCprMN);
        voff[i] = static_cast<uint32_t>((CONV == 1 ? 0 : krow * ld * 2) + c * 16);
        lim_row[i] = krow;
        lim_col[i] = c * 8;
      }
    }
  }

  // Channels-last convolution: each instruction's row is output pixel
  // n0 + row; its offset becomes that pixel's element in the padded image
  // (rows past the image's last pixel keep a valid offset and are rejected
  // by lim_row when !EVEN).
  __device__ __forceinline__ void conv_cl_init(const GemmArgs& g, int n0) {
    if constexpr (CONV == 2) {
#pragma unroll
      for (int i = 0; i < kInst; ++i) {
        const int n = min(n0 + lim_row[i], g.N - 1);
        const int p = n / g.cl_q, q = n - p * g.cl_q;
        const int64_t pix = (static_cast<int64_t>(p) * g.cl_sh * g.cl_wp + static_cast<int64_t>(q) * g.cl_sw) * g.cl_c;
        voff[i] = static_cast<uint32_t>(pix * 2 + lim_col[i] * 2);
      }
    }
  }

  // Implicit convolution: the (c, r, s) of each instruction's k-row at
  // k0 = 0 (k-row kg = (c * R + r) * S + s).
  __device__ __forceinline__ void conv_init(const GemmArgs& g) {
    if constexpr (CONV == 1) {
#pragma unroll
      for (int i = 0; i < kInst; ++i) {
        const int kg = lim_row[i];
        cv_c[i] = kg / g.cv_rs;
        const int rs = kg - cv_c[i] * g.cv_rs;
        cv_r[i] = rs / g.cv_s;
        cv_s[i] = rs - cv_r[i] * g.cv_s;
      }
    }
  }

  // Moves the resource to another tile origin with the same leading
  // dimension and extent (the per-lane offsets stay valid).
  __device__ __forceinline__ void rebase(const uint16_t* base) {
    const uint64_t addr = reinterpret_cast<uint64_t>(base);
    rsrc.x = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr));
    rsrc.y = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr >> 32) & 0xffffu);
  }

  // Issues the loads of the K tile starting at k0 into LDS at the 32-bit
  // LDS address `lds` (this operand's tile in one LDS stage; the kernels
  // form it from the LDS base once: a generic -> LDS pointer cast per load
  // instruction carries a null test, 3-4 scalar instructions each).
  // `valid` is the number of valid tile rows (K-major) or tile columns
  // (M/N-major); K bounds the k axis.
  // CONV: tiles must be issued in order k0 = 0, BK, 2 BK, ... (each call
  // advances the (c, r, s) state by BK k-rows).
  __device__ __forceinline__ void issue(uint32_t lds, int k0, int valid, int K, const GemmArgs* cv = nullptr) {
    // channels-last: the tile's (channel block, tap) offset in bytes, then
    // advance to the next K tile's: the next tap, after the last tap the
    // next block
    uint32_t cl_off = 0;
    if constexpr (CONV == 2) {
      static_assert(BK == 32, "one K tile is one 32-channel block under one tap");
      cl_off = static_cast<uint32_t>(((cl_r * cv->cl_dh * cv->cl_wp + cl_s * cv->cl_dw) * cv->cl_c + cl_c0) * 2);
      if (++cl_s >= cv->cv_s) {
        cl_s = 0;
        if (++cl_r >= cv->cv_r) {
          cl_r = 0;
          cl_c0 += BK;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < kInst; ++i) {
      uint32_t off;
      if constexpr (CONV == 1) {
        // row base of k-row (c, r, s), then advance it by BK k-rows
        const int64_t base = cv_s[i] * cv->cv_per_s + cv_c[i] * cv->cv_per_c + cv_r[i] * cv->cv_per_r;
        off = voff[i] + static_cast<uint32_t>(base * 2);
        cv_s[i] += cv->cv_ds;
        const int cs = cv_s[i] >= cv->cv_s ? 1 : 0;
        cv_s[i] -= cs * cv->cv_s;
        cv_r[i] += cv->cv_dr + cs;
        const int cr = cv_r[i] >= cv->cv_r ? 1 : 0;
        cv_r[i] -= cr * cv->cv_r;
        cv_c[i] += cv->cv_dc + cr;
      } else if constexpr (CONV == 2) {
        off = voff[i] + cl_off;
      } else {
        off = voff[i] + static_cast<uint32_t>(k0) * k_stride_bytes;
      }
      if constexpr (!EVEN) {
        bool ok;
        if constexpr (KMAJ)
          ok = lim_row[i] < valid && k0 + lim_col[i] < K;
        else
          ok = k0 + lim_row[i] < K && lim_col[i] < valid;
        off = ok ? off : kOOB;
      }
      dma16(rsrc, lds + static_cast<uint32_t>(lds_base + i * 1024), off);
    }
  }
};

// Fragment of one 32-row (m or n) x 16 k operand slice for lane `lane`:
// lane l holds row (l & 31), k = 8 * (l >> 5) + 0..7.
template <int R, bool KMAJ, int BK>
__device__ __forceinline__ u32x4 load_frag(const char* tile, int row0, int ks, int lane) {
  if constexpr (KMAJ) {
    const int r = row0 + (lane & 31);
    const int c = ks * 2 + (lane >> 5);
    return *reinterpret_cast<const u32x4*>(tile + r * (BK * 2) + kslot<BK>(r, c) * 16);
  } else {
    // ds_read_b64_tr_b16: within each 16-lane group, source lane i reads
    // 4 elements of k-row kb + i/4 at columns nb + 4 (i % 4) .. +3; output
    // lane j receives column nb + j at k-rows kb .. kb + 3.
    const int i = lane & 15;
    const int n = row0 + ((lane >> 4) & 1) * 16 + (i & 3) * 4;
    const int c = n >> 3, half = (n >> 2) & 1;
    s16x4 v[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k = ks * 16 + (lane >> 5) * 8 + h * 4 + (i >> 2);
      const char* p = tile + k * (R * 2) + mnslot(k, c) * 16 + half * 8;
      v[h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p));
    }
    u32x4 r;
    r.x = static_cast<uint16_t>(v[0][0]) | (static_cast<uint32_t>(static_cast<uint16_t>(v[0][1])) << 16);
    r.y = static_cast<uint16_t>(v[0][2]) | (static_cast<uint32_t>(static_cast<uint16_t>(v[0][3])) << 16);
    r.z = static_cast<uint16_t>(v[1][0]) | (static_cast<uint32_t>(static_cast<uint16_t>(v[1][1])) << 16);
    r.w = static_cast<uint16_t>(v[1][2]) | (static_cast<uint32_t>(static_cast<uint16_t>(v[1][3])) << 16);
    return r;
  }
}

// ---- epilogue --------------------------------------------------------------
// With B as the first MFMA operand, lane l of 32x32 tile (i, j) holds output
// row  m = l & 31  and columns  n = 8q + 4(l >> 5) + 0..3  in
// acc[i][j][4q .. 4q+3].  alpha / beta are applied in fp32 and each value is
// rounded once.  (mw, nw) is the wave tile's origin in the output; D and Cp
// already point at the batch's matrices.  The C access mode CM is a template
// parameter so the C test is not a branch per element:
//   kCNone     no C;
//   kCStrided  one load per element (any strides);
//   kCVec4     unit column stride, rows and batches 8-byte aligned: a lane's
//              4 consecutive columns in one 8-byte load (addmm's bias row
//              and full C matrices);
//   kCRow      column stride 0: one value per row (conv2d's bias).
constexpr int kCNone = 0, kCStrided = 1, kCVec4 = 2, kCRow = 3;

// beta * C at (m, n .. n + 3) in fp32 (zeros where `ok` is false, i.e.
// past the output's edge: no load is issued there).
template <typename T, int CM>
__device__ __forceinline__ void c_values(const GemmArgs& g, const T* Cp, int m, int n, bool ok, float (&c)[4]) {
  if constexpr (CM == kCVec4) {
    u32x2 raw = {0u, 0u};
    if (ok) raw = *reinterpret_cast<const u32x2*>(Cp + static_cast<int64_t>(m) * g.sc_m + n);
    const T* t = reinterpret_cast<const T*>(&raw);
#pragma unroll
    for (int e = 0; e < 4; ++e) c[e] = g.beta * static_cast<float>(t[e]);
  } else if constexpr (CM == kCRow) {
    const float v = ok ? g.beta * static_cast<float>(Cp[static_cast<int64_t>(m) * g.sc_m]) : 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) c[e] = v;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      c[e] = (CM == kCStrided && ok) ? g.beta * static_cast<float>(Cp[m * g.sc_m + (n + e) * g.sc_n]) : 0.f;
  }
}

template <typename T, int CM, int TM, int TN>
__device__ __forceinline__ float final_value(const GemmArgs& g, const f32x16 (&acc)[TM][TN], const float (&c)[4],
                                             int i, int j, int q, int e) {
  float v = g.alpha * acc[i][j][4 * q + e];
  if constexpr (CM != kCNone) v += c[e];
  return v;
}

// Staged store: the wave writes its rounded WTM x WTN tile into its own LDS
// region `ep` (rows of WTN * 2 bytes, 16-byte chunk c of row r at slot
// c ^ ((r >> 1) & 7)), reads it back row by row (stage_tile), then streams
// it out with 16-byte stores, 8 lanes per 128-byte row segment, so every L2
// write request is a full line instead of 16 bytes (store_rows: exactly
// WTM / 8 store instructions when EVEN).
template <typename T, int CM, int TM, int TN, int WTM, int WTN, bool EVEN>
__device__ __forceinline__ void stage_tile(const GemmArgs& g, const f32x16 (&acc)[TM][TN], char* ep,
                                           const T* Cp, int mw, int nw, int lane,
                                           u32x4 (&rows)[WTM / 8]) {
  static_assert(WTN * 2 == 128, "staged epilogue assumes 64-column wave tiles");
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int r = i * 32 + (lane & 31);
    const int m = mw + r;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = j * 32 + q * 8 + (lane >> 5) * 4;
        const int n = nw + col;
        T o[4];
        // N % 4 == 0 on this path, so columns n .. n + 3 are all in or all out
        float cv[4];
        c_values<T, CM>(g, Cp, m, n, EVEN || (m < g.M && n < g.N), cv);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool ok = EVEN || (m < g.M && n + e < g.N);
          o[e] = static_cast<T>(ok ? final_value<T, CM>(g, acc, cv, i, j, q, e) : 0.f);
        }
        const int c = col >> 3, half = (col >> 2) & 1;
        *reinterpret_cast<u32x2*>(ep + r * 128 + ((c ^ ((r >> 1) & 7)) << 4) + half * 8) =
            __builtin_bit_cast(u32x2, o);
      }
    }
  }
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int r0 = 0; r0 < WTM; r0 += 8) {
    const int r = r0 + (lane >> 3), c = lane & 7;
    rows[r0 / 8] = *reinterpret_cast<const u32x4*>(ep + r * 128 + ((c ^ ((r >> 1) & 7)) << 4));
  }
}

template <typename T, int WTM, bool EVEN, bool NT>
__device__ __forceinline__ void store_rows(const GemmArgs& g, const u32x4 (&rows)[WTM / 8], T* D,
                                           int mw, int nw, int lane) {
#pragma unroll
  for (int r0 = 0; r0 < WTM; r0 += 8) {
    const int r = r0 + (lane >> 3), c = lane & 7;
    const int m = mw + r;
    const int n = nw + c * 8;
    if (EVEN || (m < g.M && n < g.N)) {
      u32x4* dst = reinterpret_cast<u32x4*>(D + static_cast<int64_t>(m) * g.sd_m + n);
      if constexpr (NT)
        __builtin_nontemporal_store(rows[r0 / 8], dst);
      else
        *dst = rows[r0 / 8];
    }
  }
}

// Staged rows of a 16-bit output whose rows start anywhere (2-byte aligned):
// each wave-tile row segment is 64 columns = 128 bytes at byte address G0 with
// s = G0 % 16.  Lane c of the row's 8 lanes (holding columns 8c .. 8c + 7)
// writes the aligned 16-byte chunk that starts 16 (c + 1) - s bytes into the
// segment (c < 7): the top s bytes of its own chunk and the low 16 - s of the
// next lane's; lane 0 also writes the segment's first (16 - s) / 2 columns and
// lane 7 its last s / 2, element by element.  Every store stays inside the
// segment.  Full tiles only (EVEN): no column of a segment lies past N.
template <typename T, int WTM, bool NT>
__device__ __forceinline__ void store_rows_shifted(const GemmArgs& g, const u32x4 (&rows)[WTM / 8], T* D,
                                                   int mw, int nw, int lane) {
  static_assert(sizeof(T) == 2, "16-bit outputs");
#pragma unroll
  for (int r0 = 0; r0 < WTM; r0 += 8) {
    const int r = r0 + (lane >> 3), c = lane & 7;
    const u32x4 cur = rows[r0 / 8];
    u32x4 nxt;
    nxt.x = static_cast<uint32_t>(__shfl_down(static_cast<int>(cur.x), 1, 8));
    nxt.y = static_cast<uint32_t>(__shfl_down(static_cast<int>(cur.y), 1, 8));
    nxt.z = static_cast<uint32_t>(__shfl_down(static_cast<int>(cur.z), 1, 8));
    nxt.w = static_cast<uint32_t>(__shfl_down(static_cast<int>(cur.w), 1, 8));
    T* seg = D + static_cast<int64_t>(mw + r) * g.sd_m + nw;
    const uint32_t s = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(seg)) & 15u;
    if (s == 0) {
      u32x4* dst = reinterpret_cast<u32x4*>(seg + 8 * c);
      if constexpr (NT)
        __builtin_nontemporal_store(cur, dst);
      else
        *dst = cur;
      continue;
    }
    // (cur | nxt) >> 8 * (16 - s) bits, as 64-bit halves
    const uint64_t x0 = cur.x | (static_cast<uint64_t>(cur.y) << 32), x1 = cur.z | (static_cast<uint64_t>(cur.w) << 32);
    const uint64_t x2 = nxt.x | (static_cast<uint64_t>(nxt.y) << 32), x3 = nxt.z | (static_cast<uint64_t>(nxt.w) << 32);
    const uint32_t sh = 8u * (16u - s);  // 16 .. 112 bits
    uint64_t o0, o1;
    if (sh < 64) {
      o0 = (x0 >> sh) | (x1 << (64 - sh));
      o1 = (x1 >> sh) | (x2 << (64 - sh));
    } else if (sh == 64) {
      o0 = x1;
      o1 = x2;
    } else {
      const uint32_t k = sh - 64;
      o0 = (x1 >> k) | (x2 << (64 - k));
      o1 = (x2 >> k) | (x3 << (64 - k));
    }
    char* base = reinterpret_cast<char*>(seg) - s;  // the 16-byte aligned address below G0
    if (c < 7) {
      const u32x4 v = {static_cast<uint32_t>(o0), static_cast<uint32_t>(o0 >> 32), static_cast<uint32_t>(o1),
                       static_cast<uint32_t>(o1 >> 32)};
      u32x4* dst = reinterpret_cast<u32x4*>(base + 16 * (c + 1));
      if constexpr (NT)
        __builtin_nontemporal_store(v, dst);
      else
        *dst = v;
    }
    auto elem = [&](uint32_t e) -> uint16_t {
      const uint32_t d = e < 2 ? cur.x : e < 4 ? cur.y : e < 6 ? cur.z : cur.w;
      return static_cast<uint16_t>(d >> (16 * (e & 1)));
    };
    uint16_t* seg16 = reinterpret_cast<uint16_t*>(seg);
    if (c == 0)
      for (uint32_t e = 0; e < (16u - s) / 2; ++e) seg16[e] = elem(e);
    if (c == 7)
      for (uint32_t e = 8 - s / 2; e < 8; ++e) seg16[56 + e] = elem(e);
  }
}

template <typename T, int CM, int TM, int TN, int WTM, int WTN, bool EVEN, bool NT>
__device__ __forceinline__ void store_tile_shifted(const GemmArgs& g, const f32x16 (&acc)[TM][TN],
                                                   char* ep, T* D, const T* Cp, int mw, int nw, int lane) {
  u32x4 rows[WTM / 8];
  stage_tile<T, CM, TM, TN, WTM, WTN, EVEN>(g, acc, ep, Cp, mw, nw, lane, rows);
  store_rows_shifted<T, WTM, NT>(g, rows, D, mw, nw, lane);
}

template <typename T, int CM, int TM, int TN, int WTM, int WTN, bool EVEN, bool NT>
__device__ __forceinline__ void store_tile_staged(const GemmArgs& g, const f32x16 (&acc)[TM][TN],
                                                  char* ep, T* D, const T* Cp, int mw, int nw,
                                                  int lane) {
  u32x4 rows[WTM / 8];
  stage_tile<T, CM, TM, TN, WTM, WTN, EVEN>(g, acc, ep, Cp, mw, nw, lane, rows);
  store_rows<T, WTM, EVEN, NT>(g, rows, D, mw, nw, lane);
}

// Direct store: 8-byte stores of each lane's 4 consecutive columns (any
// output row stride that keeps 8-byte alignment), element stores at the edge.
template <typename T, int CM, int TM, int TN, bool EVEN>
__device__ __forceinline__ void store_tile_direct(const GemmArgs& g, const f32x16 (&acc)[TM][TN],
                                                  T* D, const T* Cp, int mw, int nw, int lane) {
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = mw + i * 32 + (lane & 31);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = nw + j * 32 + q * 8 + (lane >> 5) * 4;
        if (g.ragged) {
          // rows of any stride, N of any width: element stores, C read per element
          if (m < g.M) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (n + e < g.N) {
                float cv[4] = {0.f, 0.f, 0.f, 0.f};
                if constexpr (CM != kCNone)
                  cv[e] = g.beta * static_cast<float>(Cp[m * g.sc_m + (n + e) * g.sc_n]);
                D[static_cast<int64_t>(m) * g.sd_m + static_cast<int64_t>(n + e) * g.sd_n] =
                    static_cast<T>(final_value<T, CM>(g, acc, cv, i, j, q, e));
              }
            }
          }
          continue;
        }
        if (!EVEN && m < g.M && n < g.N && n + 3 >= g.N) {
          // the last, partial 4-column group of a row (N % 4 != 0)
#pragma unroll
          for (int e = 0; e < 3; ++e) {
            if (n + e < g.N) {
              float cv[4] = {0.f, 0.f, 0.f, 0.f};
              if constexpr (CM != kCNone)
                cv[e] = g.beta * static_cast<float>(Cp[m * g.sc_m + (n + e) * g.sc_n]);
              D[static_cast<int64_t>(m) * g.sd_m + n + e] = static_cast<T>(final_value<T, CM>(g, acc, cv, i, j, q, e));
            }
          }
          continue;
        }
        if (EVEN || (m < g.M && n + 3 < g.N)) {
          float cv[4];
          c_values<T, CM>(g, Cp, m, n, true, cv);
          T o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = static_cast<T>(final_value<T, CM>(g, acc, cv, i, j, q, e));
          *reinterpret_cast<u32x2*>(D + static_cast<int64_t>(m) * g.sd_m + n) =
              __builtin_bit_cast(u32x2, o);
        }
      }
    }
  }
}

// Output stores marked non-temporal (streamed past L2) per kernel: both
// kernels write their output once (mm 8192 x 14336 bf16: 767 -> 762 us,
// conv2d's implicit GEMM 155.5 -> 152.6 us with them).
constexpr bool kStreamOutMfma = true;
constexpr bool kStreamOutPanel = true;

// ---- MFMA kernel -----------------------------------------------------------
// STAGES LDS stages, prefetch distance STAGES - 1: the loads of tile
// kt + STAGES - 1 are issued right after the barrier that opens tile kt, so
// an operand fetch that misses L2 has STAGES - 1 tiles of MFMA work to land.
template <typename T, int BM, int BN, int WM, int WN, int BK, int STAGES, bool AK, bool BKM, bool EVEN,
          int CONV = 0, bool SPLITK = false>
__global__ __launch_bounds__(WM* WN * 64) void k_gemm_mfma(GemmArgs g) {
  static_assert(!SPLITK || CONV == 0, "split-K takes plain operands");
  constexpr int NW = WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  constexpr int TM = WTM / 32, TN = WTN / 32;  // 32x32 MFMA tiles per wave
  constexpr int kATile = BM * BK * 2, kBTile = BN * BK * 2;
  constexpr int kStage = kATile + kBTile;
  using LA = TileLoader<BM, AK, NW, EVEN, BK>;
  using LB = TileLoader<BN, BKM, NW, EVEN, BK, CONV>;
  constexpr int kLoadsPerTile = LA::kInst + LB::kInst;  // per wave
  static_assert(STAGES >= 2 && STAGES <= 5, "stages");
  extern __shared__ __attribute__((aligned(1024))) char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;

  const int tm_count = (g.M + BM - 1) / BM, tn_count = (g.N + BN - 1) / BN;
  int bat, tmi, tni;
  tile_of(blockIdx.x, gridDim.x, tm_count, tn_count, bat, tmi, tni);
  const int m0 = tmi * BM, n0 = tni * BN;
  const int m_valid = min(g.M - m0, BM), n_valid = min(g.N - n0, BN);

  const uint16_t* A = static_cast<const uint16_t*>(g.A) + bat * g.sa_b;
  const uint16_t* B = static_cast<const uint16_t*>(g.B) + bat * g.sb_b;

  LA la;
  LB lb;
  if constexpr (AK)
    la.init(A + static_cast<int64_t>(m0) * g.sa_m, g.sa_m,
            (static_cast<int64_t>(m_valid - 1) * g.sa_m + g.K) * 2, wave, lane);
  else
    la.init(A + m0, g.sa_k, (static_cast<int64_t>(g.K - 1) * g.sa_k + m_valid) * 2, wave, lane);
  if constexpr (CONV == 1) {
    lb.init(B + n0, 0, (g.sb_b - n0) * 2, wave, lane);  // the batch's whole buffer
    lb.conv_init(g);
  } else if constexpr (CONV == 2) {
    lb.init(B, 0, g.sb_b * 2, wave, lane);  // the batch's whole padded image
    lb.conv_cl_init(g, n0);
  }
  else if constexpr (BKM)
    lb.init(B + static_cast<int64_t>(n0) * g.sb_n, g.sb_n,
            (static_cast<int64_t>(n_valid - 1) * g.sb_n + g.K) * 2, wave, lane);
  else
    lb.init(B + n0, g.sb_k, (static_cast<int64_t>(g.K - 1) * g.sb_k + n_valid) * 2, wave, lane);

  const uint32_t smem_addr = lds_addr(smem);
  // this block's k range (split-K: one slice of K per block row)
  const int k_lo = SPLITK ? static_cast<int>(blockIdx.y) * g.kchunk : 0;
  const int k_len = SPLITK ? min(g.K - k_lo, g.kchunk) : g.K;
  auto issue = [&](int stage, int k0) {
    const uint32_t base = smem_addr + static_cast<uint32_t>(stage * kStage);
    la.issue(base, k_lo + k0, m_valid, g.K);
    lb.issue(base + kATile, k_lo + k0, n_valid, g.K, &g);
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int ktiles = (k_len + BK - 1) / BK;
  constexpr int KS = BK / 16;
  // Ping-pong: the block's waves form two groups with one wave per SIMD in
  // each (waves are placed round-robin over the 4 SIMDs).  In every phase one
  // group reads a K tile's fragments from LDS and issues the DMA of a later
  // tile while the other group runs the MFMAs of the tile it read in the
  // previous phase; a block barrier separates phases.  Group 1 runs one phase
  // behind group 0, so each SIMD always has one wave feeding the matrix core.
  const int grp = wave / (NW / 2);

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < ktiles) issue(s, s * BK);
  wait_tile(min(STAGES - 2, ktiles - 1), kLoadsPerTile);
  block_barrier();

  // Group 1 starts one phase late: its first barrier pairs with the barrier
  // group 0 reaches after reading tile 0.  Both groups then run the same
  // loop (read tile k | barrier | MFMAs of tile k | barrier); group 0 ends
  // with one extra barrier so every wave executes the same number.
  if (grp == 1) block_barrier();
  u32x4 af[KS][TM], bf[KS][TN];
  // One K tile.  STEADY: tile k + STAGES - 1 exists, so the refill is
  // unconditional and the wait for tile k + 1 a constant (the loop over
  // these tiles carries no per-tile branches); the last STAGES - 1 tiles
  // take the general form.
  auto tile = [&](int k, auto steady_tag) {
    constexpr bool STEADY = decltype(steady_tag)::value;
    // memory phase: refill the stage of tile k - 1 with tile k + STAGES - 1,
    // then read all of tile k's fragments.
    if (STEADY || k + STAGES - 1 < ktiles) issue((k + STAGES - 1) % STAGES, (k + STAGES - 1) * BK);
    const char* sa = smem + (k % STAGES) * kStage;
    const char* sb = sa + kATile;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int i = 0; i < TM; ++i) af[ks][i] = load_frag<BM, AK, BK>(sa, wm * WTM + i * 32, ks, lane);
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[ks][j] = load_frag<BN, BKM, BK>(sb, wn * WTN + j * 32, ks, lane);
    }
    // The fragments are in registers before the stage can be refilled, and
    // this wave's share of tile k + 1 has landed before the barrier that
    // opens the next memory phase of either group.
    wait_lgkmcnt0();
    if constexpr (STEADY)
      wait_vmcnt<(STAGES - 2) * kLoadsPerTile>();
    else if (k + 1 < ktiles)
      wait_tile(min(STAGES - 2, ktiles - 2 - k), kLoadsPerTile);
    block_barrier();
    // MFMA phase, at raised wave priority so the SIMD's arbiter issues the
    // matrix wave ahead of its memory-phase partner (+0.8 % on mm).
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma32<T>(bf[ks][j], af[ks][i], acc[i][j]);
    __builtin_amdgcn_s_setprio(0);
    block_barrier();
  };
  int k = 0;
  for (; k + STAGES - 1 < ktiles; ++k) tile(k, std::true_type{});
  for (; k < ktiles; ++k) tile(k, std::false_type{});
  if (grp == 0) block_barrier();

  const int mw = m0 + wm * WTM, nw = n0 + wn * WTN;
  if constexpr (SPLITK) {
    // the fp32 partial tile: lane l holds row (l & 31) and 4 consecutive
    // columns per (i, j, q), one 16-byte store each (N % 4 == 0, so the 4
    // columns are all in or all out)
    float* P = g.part + static_cast<int64_t>(blockIdx.y) * g.part_stride;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int m = mw + i * 32 + (lane & 31);
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = nw + j * 32 + q * 8 + (lane >> 5) * 4;
          if (EVEN || (m < g.M && n < g.N)) {
            const f32x4 v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
            *reinterpret_cast<f32x4*>(P + static_cast<int64_t>(m) * g.N + n) = v;
          }
        }
    }
    return;
  }
  T* D = static_cast<T*>(g.D) + bat * g.sd_b;
  const T* Cp = g.use_c ? static_cast<const T*>(g.C) + bat * g.sc_b : nullptr;
  char* ep = smem + wave * (WTM * WTN * 2);
  auto store = [&](auto cm_tag) {
    constexpr int CM = decltype(cm_tag)::value;
    if (g.staged)
      store_tile_staged<T, CM, TM, TN, WTM, WTN, EVEN, kStreamOutMfma>(g, acc, ep, D, Cp, mw, nw, lane);
    else if (EVEN && WTN == 64 && g.shifted)
      store_tile_shifted<T, CM, TM, TN, WTM, WTN, EVEN, kStreamOutMfma>(g, acc, ep, D, Cp, mw, nw, lane);
    else
      store_tile_direct<T, CM, TM, TN, EVEN>(g, acc, D, Cp, mw, nw, lane);
  };
  switch (Cp == nullptr ? kCNone : g.c_mode) {
    case kCNone: store(std::integral_constant<int, kCNone>{}); break;
    case kCVec4: store(std::integral_constant<int, kCVec4>{}); break;
    case kCRow: store(std::integral_constant<int, kCRow>{}); break;
    default: store(std::integral_constant<int, kCStrided>{}); break;
  }
}

// ---- short-K persistent kernel ---------------------------------------------
// For K <= 128 (bmm with a head-sized K) a 128 x 128 tile's whole K panel is
// one DMA per operand (32 KiB each), and the kernel is bound by writing the
// output, not by the MFMAs.
//
// Blocks of 4 waves (2 x 2 wave tiles of 64 x 64) hold one A panel and one
// B panel (64 KiB of LDS), two blocks per CU, persistent, with no
// synchronisation between blocks: the output stores of one block drain
// while the other computes, instead of every store burst being gated by
// block barriers shared with MFMA work.  A block runs tile after tile: the
// tile's MFMAs; the epilogue staged through the A panel it has just finished
// with; then the next tile's DMA, queued ahead of this tile's stores.
//
// Work is walked in units of `seg` consecutive tiles down one tile column
// (same batch and 128-column block of B): the unit's B panel is loaded once
// and only the A panel per tile.  Units are dealt so that each XCD takes a
// contiguous range, i.e. the blocks working at the same time on one batch
// hold neighbouring tile columns and write whole output rows together.
// Measured on MI355X for bmm (32, 2048 x 128)(128 x 2048) this column order
// writes ~7 % faster than walking tile rows (each output row then written in
// 256-byte pieces at far-apart times), and the pair of barrier-free blocks
// ~2 % faster than one 8-wave block whose two 4-wave halves alternate MFMA
// and epilogue phases between block barriers.  Temporal (L2-allocating)
// output stores are ~25 % slower than streaming ones here.
//
// Requires M % 128 == 0, N % 128 == 0, K % 8 == 0, seg | M / 128 and the
// staged (16-byte aligned, unit column stride) output; k >= K reads as zero.
constexpr int kPanelK = 128;
constexpr int kPanelTile = 128 * kPanelK * 2;  // one operand panel
constexpr int kPanelLds = 2 * kPanelTile;      // 64 KiB
constexpr int kPanelBlocksPerCu = 2;

template <typename T, bool AK, bool BKM>
__global__ __launch_bounds__(256, 2) void k_gemm_panel(GemmArgs g, int seg) {
  constexpr int BM = 128, BN = 128, NW = 4;
  constexpr int WTM = 64, WTN = 64, TM = 2, TN = 2, KS = kPanelK / 16;
  using LA = TileLoader<BM, AK, NW, false, kPanelK>;
  using LB = TileLoader<BN, BKM, NW, false, kPanelK>;
  constexpr int kStores = WTM / 8;  // store instructions per wave per tile
  constexpr int kOffA = 0, kOffB = kPanelTile;
  extern __shared__ __attribute__((aligned(1024))) char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int tm_count = g.M / BM, tn_count = g.N / BN;
  const int upc = tm_count / seg;  // units per tile column
  const int units = g.batch * tn_count * upc;
  const int G = gridDim.x;
  const int u0 = blockIdx.x;
  if (u0 >= units) return;
  const int n = ((units - 1 - u0) / G + 1) * seg;  // tiles of this block

  const uint16_t* A0 = static_cast<const uint16_t*>(g.A);
  const uint16_t* B0 = static_cast<const uint16_t*>(g.B);
  LA la;
  LB lb;
  if constexpr (AK)
    la.init(A0, g.sa_m, (static_cast<int64_t>(BM - 1) * g.sa_m + g.K) * 2, wave, lane);
  else
    la.init(A0, g.sa_k, (static_cast<int64_t>(g.K - 1) * g.sa_k + BM) * 2, wave, lane);
  if constexpr (BKM)
    lb.init(B0, g.sb_n, (static_cast<int64_t>(BN - 1) * g.sb_n + g.K) * 2, wave, lane);
  else
    lb.init(B0, g.sb_k, (static_cast<int64_t>(g.K - 1) * g.sb_k + BN) * 2, wave, lane);

  struct Coord {
    int bat, m0, n0;
    bool first;  // first tile of its unit: loads the unit's B panel
  };
  // Tile i of this block: unit k = i / seg (global unit u0 + k * G, remapped
  // so each XCD walks a contiguous range of units), tile j = i % seg of it.
  auto coord = [&](int i) {
    Coord c;
    const int k = i / seg, j = i - k * seg;
    int u = u0 + k * G;
    if ((units & 7) == 0 && (G & 7) == 0) u = (u & 7) * (units >> 3) + (u >> 3);
    const int col = u / upc, s = u - col * upc;
    c.bat = col / tn_count;
    c.n0 = (col - c.bat * tn_count) * BN;
    c.m0 = (s * seg + j) * BM;
    c.first = j == 0;
    return c;
  };
  const uint32_t smem_addr = lds_addr(smem);
  auto issue = [&](const Coord& c) {
    la.rebase(A0 + c.bat * g.sa_b + (AK ? static_cast<int64_t>(c.m0) * g.sa_m : c.m0));
    la.issue(smem_addr + kOffA, 0, BM, g.K);
    if (c.first) {
      lb.rebase(B0 + c.bat * g.sb_b + (BKM ? static_cast<int64_t>(c.n0) * g.sb_n : c.n0));
      lb.issue(smem_addr + kOffB, 0, BN, g.K);
    }
  };

  issue(coord(0));
  f32x16 acc[TM][TN];
  for (int t = 0; t < n; ++t) {
    const Coord c = coord(t);
    // Tile t's operands have landed (only tile t - 1's stores may still be
    // in flight), in every wave's share.
    if (t == 0)
      wait_vmcnt<0>();
    else
      wait_vmcnt<kStores>();
    block_barrier();
    const char* sa = smem + kOffA;
    const char* sb = smem + kOffB;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = load_frag<BM, AK, kPanelK>(sa, wm * WTM + i * 32, ks, lane);
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = load_frag<BN, BKM, kPanelK>(sb, wn * WTN + j * 32, ks, lane);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma32<T>(bf[j], af[i], acc[i][j]);
    }
    wait_lgkmcnt0();
    // Every wave is done reading the A panel: it becomes the staging area.
    block_barrier();
    T* D = static_cast<T*>(g.D) + c.bat * g.sd_b;
    char* ep = smem + kOffA + wave * (WTM * WTN * 2);
    const int mw = c.m0 + wm * WTM, nw = c.n0 + wn * WTN;
    u32x4 rows[WTM / 8];
    if (g.use_c)
      stage_tile<T, kCStrided, TM, TN, WTM, WTN, true>(g, acc, ep, static_cast<const T*>(g.C) + c.bat * g.sc_b,
                                                        mw, nw, lane, rows);
    else
      stage_tile<T, kCNone, TM, TN, WTM, WTN, true>(g, acc, ep, nullptr, mw, nw, lane, rows);
    wait_lgkmcnt0();
    // Every wave holds its rows: the panels may be refilled.  The next
    // tile's DMA is queued ahead of this tile's stores.
    block_barrier();
    if (t + 1 < n) issue(coord(t + 1));
    store_rows<T, WTM, true, kStreamOutPanel>(g, rows, D, mw, nw, lane);
  }
  wait_vmcnt<0>();
}

// ---- skinny kernel (M <= 64) -------------------------------------------------
// Decode-shaped products (a few rows of A against a large B) are bound by
// streaming B once.  A block owns 16 J output columns of one batch and all
// of M (MB blocks of 16 rows); its NW waves split K in 32-wide steps (wave w
// takes steps w, w + NW, ...), so each column's B is read front to back by
// the block, and merge their fp32 partial sums through LDS at the end.
// Each A fragment serves J B fragments.
// Operands go straight from global memory to registers in the layout of
// v_mfma_f32_16x16x32 (lane l: row / column l & 15, k = 8 (l >> 4) .. + 7):
// A and K-major B with one 16-byte buffer load per lane; M/N-major B
// loaded as 16-byte row pieces and transposed through a J KiB per-wave LDS
// area with ds_read_b64_tr_b16.  U steps are loaded before their MFMAs so
// each wave keeps U * (MB + J) 16-byte loads in flight (refilling each
// step's registers as soon as they are consumed measured no faster).  Blocks
// are mapped so that consecutive n-slices share an XCD: for an M/N-major B
// each block reads 32 J bytes of every k-row, and its neighbours' pieces of
// the same 128-byte lines then come from the same L2 (16-column slices,
// 16 x 14336 x 4096 NN: 75 -> 40 us).  Out-of-range rows, columns and k
// read as zero (buffer offsets past the extent).
// Requires A K-major, K % 8 == 0; M/N-major B also N % 8 == 0.
constexpr int kSkinnyMaxM = 64;
// Rows up to which K-major products take the skinny kernel: past 32 its
// blocks' re-reads of A (every block reads all of it) cost more than the
// tile kernels' idle matrix rows (M = 64, N = 128256, K = 4096: 410 against
// 245-275 µs on the 256 x 256 tiles) -- unless the 128 x 128 tiles would not
// fill the GPU (and the product does not split K).
constexpr int kSkinnyRouteM = 32;
// Rows above which a product with a workspace takes the split-K tiles
// instead of the skinny kernel (whose blocks each re-read all of A).
constexpr int kSplitKMinM = 16;
// Widest column slice (in 16-column groups) for MB 16-row blocks of A: the
// partial-sum exchange (4 * J * MB KiB of LDS) stays within 32 KiB.
constexpr int kSkinnyMaxJ(int mb) { return mb <= 2 ? 4 : 2; }

template <typename T>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (std::is_same<T, __bf16>::value)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <typename T, bool BKM, int MB, int J, int NW>
__global__ __launch_bounds__(64 * NW) void k_gemm_skinny(GemmArgs g) {
  constexpr int U = MB + J <= 3 ? 8 : 4, NB = 16 * J;
  __shared__ float red[NW][J][MB][4][64];
  __shared__ __attribute__((aligned(16))) uint16_t trs[BKM ? 1 : NW][32 * NB];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Consecutive n-slices on one XCD (workgroups are dealt round-robin over
  // the 8 XCDs), so neighbouring pieces of an M/N-major B row share an L2.
  int bx = blockIdx.x;
  if ((gridDim.x & 7) == 0) bx = (bx & 7) * (gridDim.x >> 3) + (bx >> 3);
  const int n0 = bx * NB;
  const int bat = blockIdx.y;
  const int nv = min(NB, g.N - n0);
  const int r16 = lane & 15, kq = (lane >> 4) * 8;

  const uint16_t* A = static_cast<const uint16_t*>(g.A) + bat * g.sa_b;
  const uint16_t* B = static_cast<const uint16_t*>(g.B) + bat * g.sb_b;
  const __amdgpu_buffer_rsrc_t ra =
      buffer_rsrc(A, static_cast<uint32_t>((static_cast<int64_t>(g.M - 1) * g.sa_m + g.K) * 2));
  const __amdgpu_buffer_rsrc_t rb =
      BKM ? buffer_rsrc(B + static_cast<int64_t>(n0) * g.sb_n,
                        static_cast<uint32_t>((static_cast<int64_t>(nv - 1) * g.sb_n + g.K) * 2))
          : buffer_rsrc(B + n0, static_cast<uint32_t>((static_cast<int64_t>(g.K - 1) * g.sb_k + nv) * 2));
  // Per-lane byte offsets at k0 = 0.  K-major B: load j covers columns
  // 16 j + (l & 15).  M/N-major B: load j covers k-rows j * 32 / J +
  // l / (2 J), 16-byte chunk l % (2 J) of the slice's row piece.
  uint32_t a_off[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) a_off[mb] = static_cast<uint32_t>(((mb * 16 + r16) * g.sa_m + kq) * 2);
  uint32_t b_off[J];
  bool b_col_ok[J];
  int b_krow[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    if constexpr (BKM) {
      b_off[j] = static_cast<uint32_t>(((16 * j + r16) * g.sb_n + kq) * 2);
      b_col_ok[j] = 16 * j + r16 < nv;
      b_krow[j] = kq;
    } else {
      b_krow[j] = j * (32 / J) + lane / (2 * J);
      b_off[j] = static_cast<uint32_t>((b_krow[j] * g.sb_k + 8 * (lane % (2 * J))) * 2);
      b_col_ok[j] = 8 * (lane % (2 * J)) < nv;
    }
  }
  const uint32_t b_kstep = BKM ? 2u : static_cast<uint32_t>(g.sb_k * 2);  // bytes per k

  f32x4 acc[J][MB];
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[j][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int s0 = wave; s0 * 32 < g.K; s0 += NW * U) {
    u32x4 bq[U][J], aq[U][MB];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k0 = (s0 + NW * u) * 32;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const bool b_ok = b_col_ok[j] && k0 + b_krow[j] < g.K;
        bq[u][j] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       rb, b_ok ? b_off[j] + static_cast<uint32_t>(k0) * b_kstep : kOOB, 0, 0));
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const bool a_ok = mb * 16 + r16 < g.M && k0 + kq < g.K;
        aq[u][mb] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, a_ok ? a_off[mb] + k0 * 2u : kOOB, 0, 0));
      }
    }
    // All U steps' loads are issued before the first MFMA needs one.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      u32x4 bf[J];
      if constexpr (BKM) {
#pragma unroll
        for (int j = 0; j < J; ++j) bf[j] = bq[u][j];
      } else {
        // Store the 32 x NB step tile row-major (load j's 64 lanes write
        // bytes j KiB + 16 l), read each 16-column group back transposed.
#pragma unroll
        for (int j = 0; j < J; ++j) *reinterpret_cast<u32x4*>(&trs[wave][j * 512 + lane * 8]) = bq[u][j];
#pragma unroll
        for (int j = 0; j < J; ++j) {
          s16x4 v[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int k = kq + 4 * h + (r16 >> 2);
            v[h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s16x4_t*)(&trs[wave][k * NB + 16 * j + 4 * (r16 & 3)]));
          }
          bf[j].x = static_cast<uint16_t>(v[0][0]) | (static_cast<uint32_t>(static_cast<uint16_t>(v[0][1])) << 16);
          bf[j].y = static_cast<uint16_t>(v[0][2]) | (static_cast<uint32_t>(static_cast<uint16_t>(v[0][3])) << 16);
          bf[j].z = static_cast<uint16_t>(v[1][0]) | (static_cast<uint32_t>(static_cast<uint16_t>(v[1][1])) << 16);
          bf[j].w = static_cast<uint16_t>(v[1][2]) | (static_cast<uint32_t>(static_cast<uint16_t>(v[1][3])) << 16);
        }
      }
#pragma unroll
      for (int j = 0; j < J; ++j)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[j][mb] = mfma16<T>(aq[u][mb], bf[j], acc[j][mb]);
    }
  }
  // Lane l holds rows 4 (l >> 4) + r of each 16-row block, column
  // 16 j + (l & 15) of the slice.
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][j][mb][r][lane] = acc[j][mb][r];
  __syncthreads();
  T* D = static_cast<T*>(g.D) + bat * g.sd_b;
  const T* Cp = g.use_c ? static_cast<const T*>(g.C) + bat * g.sc_b : nullptr;
  for (int q = wave; q < J * MB; q += NW) {
    const int j = q / MB, mb = q - j * MB;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = mb * 16 + (lane >> 4) * 4 + r, n = n0 + 16 * j + r16;
      if (m < g.M && n < g.N) {
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) v += red[w][j][mb][r][lane];
        v *= g.alpha;
        if (Cp != nullptr) v += g.beta * static_cast<float>(Cp[m * g.sc_m + n * g.sc_n]);
        D[static_cast<int64_t>(m) * g.sd_m + static_cast<int64_t>(n) * g.sd_n] = static_cast<T>(v);
      }
    }
  }
}

template <typename T, bool BKM, int MB>
int launch_skinny_mb(const GemmArgs& g, hipStream_t st, int j) {
  const unsigned by = static_cast<unsigned>(g.batch);
  note_kernel("gemm_skinny m%d n%d %s", 16 * MB, 16 * j, BKM ? "B:K" : "B:N");
  if constexpr (kSkinnyMaxJ(MB) >= 4)
    if (j == 4) {
      hipLaunchKernelGGL((k_gemm_skinny<T, BKM, MB, 4, 4>), dim3((g.N + 63) / 64, by), dim3(256), 0, st, g);
      return check_launch("gemm");
    }
  if (j == 2)
    hipLaunchKernelGGL((k_gemm_skinny<T, BKM, MB, 2, 4>), dim3((g.N + 31) / 32, by), dim3(256), 0, st, g);
  else
    hipLaunchKernelGGL((k_gemm_skinny<T, BKM, MB, 1, 4>), dim3((g.N + 15) / 16, by), dim3(256), 0, st, g);
  return check_launch("gemm");
}

// Column-slice width 16 j: the widest that still gives three quarters of
// the CUs a block.  Wider slices read whole 128-byte lines of an N-major B
// row (32 columns: half lines) and more columns per A fragment: N = 14336,
// K = 4096 runs 25-26 us in 224 64-column blocks against 34-39 us in 448
// 32-column ones (N-major B; K-major at 16 rows 28 against 31.5), while one
// block per CU stays better than fewer (N = 4096: 256 16-column blocks).
// (16-wave blocks splitting K finer for the few-block shapes, e.g.
// 16 x 4096 x 14336, measured no faster than 4-wave ones.)
int skinny_j(int64_t M, int64_t N, int64_t batch) {
  const int mb = static_cast<int>((M + 15) / 16);
  const int cus = cu_count_cached() > 0 ? cu_count_cached() : 256;
  for (int c : {4, 2})
    if (c <= kSkinnyMaxJ(mb) && (N + 16 * c - 1) / (16 * c) * batch * 4 >= 3 * cus) return c;
  return 1;
}

template <typename T, bool BKM>
int launch_skinny(const GemmArgs& g, hipStream_t st) {
  const int mb = (g.M + 15) / 16;
  const int j = skinny_j(g.M, g.N, g.batch);
  if (mb == 1) return launch_skinny_mb<T, BKM, 1>(g, st, j);
  if (mb == 2) return launch_skinny_mb<T, BKM, 2>(g, st, j);
  if (mb == 3) return launch_skinny_mb<T, BKM, 3>(g, st, j);
  return launch_skinny_mb<T, BKM, 4>(g, st, j);
}

// fp32 variant of the skinny kernel: v_mfma_f32_16x16x4_f32 (IEEE fp32
// products, fp32 accumulation) in 16-wide K steps.  A lane's 16-byte load
// holds 4 consecutive k of one row, k0 + 4 (l >> 4) + e, and element e of
// every operand feeds MFMA e of the step, so the four MFMAs cover the
// step's 16 k values in a fixed permutation shared by A and B.  An M/N-major
// B goes through a per-wave LDS tile [16 k][16 J n] read back per column.
template <bool BKM, int MB, int J>
__global__ __launch_bounds__(256) void k_gemm_skinny_f32(GemmArgs g) {
  constexpr int NW = 4, U = MB + J <= 3 ? 8 : 4, NB = 16 * J;
  __shared__ float red[NW][J][MB][4][64];
  __shared__ __attribute__((aligned(16))) float trs[BKM ? 1 : NW][16 * NB];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int bx = blockIdx.x;
  if ((gridDim.x & 7) == 0) bx = (bx & 7) * (gridDim.x >> 3) + (bx >> 3);
  const int n0 = bx * NB;
  const int bat = blockIdx.y;
  const int nv = min(NB, g.N - n0);
  const int r16 = lane & 15, kq = (lane >> 4) * 4;

  const float* A = static_cast<const float*>(g.A) + bat * g.sa_b;
  const float* B = static_cast<const float*>(g.B) + bat * g.sb_b;
  const __amdgpu_buffer_rsrc_t ra =
      buffer_rsrc(A, static_cast<uint32_t>((static_cast<int64_t>(g.M - 1) * g.sa_m + g.K) * 4));
  const __amdgpu_buffer_rsrc_t rb =
      BKM ? buffer_rsrc(B + static_cast<int64_t>(n0) * g.sb_n,
                        static_cast<uint32_t>((static_cast<int64_t>(nv - 1) * g.sb_n + g.K) * 4))
          : buffer_rsrc(B + n0, static_cast<uint32_t>((static_cast<int64_t>(g.K - 1) * g.sb_k + nv) * 4));
  uint32_t a_off[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) a_off[mb] = static_cast<uint32_t>(((mb * 16 + r16) * g.sa_m + kq) * 4);
  uint32_t b_off[J];
  bool b_col_ok[J];
  int b_krow[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    if constexpr (BKM) {
      b_off[j] = static_cast<uint32_t>(((16 * j + r16) * g.sb_n + kq) * 4);
      b_col_ok[j] = 16 * j + r16 < nv;
      b_krow[j] = kq;
    } else {
      // load j: k-rows j * 16 / J + l / (4 J), 4-float chunk l % (4 J)
      b_krow[j] = j * (16 / J) + lane / (4 * J);
      b_off[j] = static_cast<uint32_t>((b_krow[j] * g.sb_k + 4 * (lane % (4 * J))) * 4);
      b_col_ok[j] = 4 * (lane % (4 * J)) < nv;
    }
  }
  const uint32_t b_kstep = BKM ? 4u : static_cast<uint32_t>(g.sb_k * 4);  // bytes per k

  f32x4 acc[J][MB];
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[j][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int s0 = wave; s0 * 16 < g.K; s0 += NW * U) {
    f32x4 bq[U][J], aq[U][MB];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k0 = (s0 + NW * u) * 16;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const bool b_ok = b_col_ok[j] && k0 + b_krow[j] < g.K;
        bq[u][j] = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       rb, b_ok ? b_off[j] + static_cast<uint32_t>(k0) * b_kstep : kOOB, 0, 0));
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const bool a_ok = mb * 16 + r16 < g.M && k0 + kq < g.K;
        aq[u][mb] = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, a_ok ? a_off[mb] + k0 * 4u : kOOB, 0, 0));
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      f32x4 bf[J];
      if constexpr (BKM) {
#pragma unroll
        for (int j = 0; j < J; ++j) bf[j] = bq[u][j];
      } else {
        // row-major [16 k][NB] tile: load j's lanes write floats j * 256 + 4 l
#pragma unroll
        for (int j = 0; j < J; ++j) *reinterpret_cast<f32x4*>(&trs[wave][j * 256 + lane * 4]) = bq[u][j];
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) bf[j][e] = trs[wave][(kq + e) * NB + 16 * j + r16];
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
            acc[j][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(aq[u][mb][e], bf[j][e], acc[j][mb], 0, 0, 0);
    }
  }
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][j][mb][r][lane] = acc[j][mb][r];
  __syncthreads();
  float* D = static_cast<float*>(g.D) + bat * g.sd_b;
  const float* Cp = g.use_c ? static_cast<const float*>(g.C) + bat * g.sc_b : nullptr;
  for (int q = wave; q < J * MB; q += NW) {
    const int j = q / MB, mb = q - j * MB;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = mb * 16 + (lane >> 4) * 4 + r, n = n0 + 16 * j + r16;
      if (m < g.M && n < g.N) {
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) v += red[w][j][mb][r][lane];
        v *= g.alpha;
        if (Cp != nullptr) v += g.beta * Cp[m * g.sc_m + n * g.sc_n];
        D[static_cast<int64_t>(m) * g.sd_m + static_cast<int64_t>(n) * g.sd_n] = v;
      }
    }
  }
}

template <bool BKM, int MB>
int launch_skinny_f32_mb(const GemmArgs& g, hipStream_t st, int j) {
  const unsigned by = static_cast<unsigned>(g.batch);
  note_kernel("gemm_skinny_f32 m%d n%d %s", 16 * MB, 16 * j, BKM ? "B:K" : "B:N");
  if constexpr (kSkinnyMaxJ(MB) >= 4)
    if (j == 4) {
      hipLaunchKernelGGL((k_gemm_skinny_f32<BKM, MB, 4>), dim3((g.N + 63) / 64, by), dim3(256), 0, st, g);
      return check_launch("gemm");
    }
  if (j == 2)
    hipLaunchKernelGGL((k_gemm_skinny_f32<BKM, MB, 2>), dim3((g.N + 31) / 32, by), dim3(256), 0, st, g);
  else
    hipLaunchKernelGGL((k_gemm_skinny_f32<BKM, MB, 1>), dim3((g.N + 15) / 16, by), dim3(256), 0, st, g);
  return check_launch("gemm");
}

template <bool BKM>
int launch_skinny_f32(const GemmArgs& g, hipStream_t st) {
  const int mb = (g.M + 15) / 16;
  const int cus = cu_count_cached() > 0 ? cu_count_cached() : 256;
  int j = 1;
  for (int c : {4, 2}) {
    if (c <= kSkinnyMaxJ(mb) && static_cast<int64_t>((g.N + 16 * c - 1) / (16 * c)) * g.batch * 4 >= 3 * cus) {
      j = c;
      break;
    }
  }
  if (mb == 1) return launch_skinny_f32_mb<BKM, 1>(g, st, j);
  if (mb == 2) return launch_skinny_f32_mb<BKM, 2>(g, st, j);
  if (mb == 3) return launch_skinny_f32_mb<BKM, 3>(g, st, j);
  return launch_skinny_f32_mb<BKM, 4>(g, st, j);
}

// ---- fp32 tile kernel -------------------------------------------------------
// fp32 products on v_mfma_f32_16x16x4_f32 (IEEE fp32 products, fp32
// accumulation).  A block of WM x 2 waves (WM = 1 or 2) covers (64 WM) x 128 outputs, each
// wave a 64 x 64 tile (4 x 4 MFMA tiles).  K advances in 32-deep tiles of A
// and B shared through two LDS buffers: each thread loads its 16-byte chunks
// of the next tile into registers before the current tile's MFMAs and writes
// them to the other buffer after the first half of them.  Within a tile the
// fragments of the second 16-k step are read while the first step's MFMAs
// run, and those of the next tile's first step after the tile's one barrier,
// while the second step's run.  Lane l of a 16-k step holds 4 consecutive k,
// 4 (l >> 4) + e, of its row (A) or column (B), and element e feeds MFMA e:
// one 16-byte LDS read per fragment for K-major tiles.
// LDS layouts: a K-major tile is [row][32 k], 16-byte chunk c of row r at
// slot c ^ ((r >> 1) & 7), so the 16 rows a read covers hit all 64 banks;
// an N-major B tile is [32 k][128 + 4 n] (padded rows put the four k-rows a
// column read covers in different banks), read per element.
// Out-of-range rows, columns and k read as zero (buffer resources).
// SPLITK: block row blockIdx.y takes k in [blockIdx.y * kchunk, + kchunk)
// (kchunk a multiple of 32) and writes its raw fp32 partial tile to
// part + blockIdx.y * part_stride + batch * M * N (rows of N).
template <bool BKM, int WM, bool SPLITK = false>
__global__ __launch_bounds__(128 * WM) void k_gemm_f32_lds(GemmArgs g) {
  constexpr int T = 128 * WM, BM = 64 * WM, BN = 128, BK = 32;
  constexpr int kBRow = BN + 4;                         // floats per k-row of an N-major B tile
  constexpr int A_CH = BM * 8 / T, B_CH = BN * 8 / T;  // 16-byte chunks per thread per tile
  constexpr int A_FL = BM * BK, B_FL = BKM ? BN * BK : BK * kBRow;
  __shared__ __attribute__((aligned(16))) float lds[2][A_FL + B_FL];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tm_count = (g.M + BM - 1) / BM, tn_count = (g.N + BN - 1) / BN;
  int bat, tmi, tni;
  tile_of(blockIdx.x, gridDim.x, tm_count, tn_count, bat, tmi, tni);
  const int bm0 = tmi * BM, bn0 = tni * BN;
  const int mv = max(0, min(BM, g.M - bm0)), nv = max(0, min(BN, g.N - bn0));
  const float* A = static_cast<const float*>(g.A) + bat * g.sa_b;
  const float* B = static_cast<const float*>(g.B) + bat * g.sb_b;
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc_uniform(
      A + static_cast<int64_t>(bm0) * g.sa_m,
      mv > 0 ? static_cast<uint32_t>((static_cast<int64_t>(mv - 1) * g.sa_m + g.K) * 4) : 0u);
  const __amdgpu_buffer_rsrc_t rb =
      BKM ? buffer_rsrc_uniform(B + static_cast<int64_t>(bn0) * g.sb_n,
                                nv > 0 ? static_cast<uint32_t>((static_cast<int64_t>(nv - 1) * g.sb_n + g.K) * 4) : 0u)
          : buffer_rsrc_uniform(B + bn0,
                                nv > 0 ? static_cast<uint32_t>((static_cast<int64_t>(g.K - 1) * g.sb_k + nv) * 4) : 0u);
  // Loader slots.  K-major chunk q: row q / 8, k 4 (q % 8) .. + 3 of the tile;
  // N-major B chunk q: k-row q / 32, columns 4 (q % 32) .. + 3.
  uint32_t a_off[A_CH], a_lds[A_CH];
  int a_k[A_CH];
  bool a_ok[A_CH];
#pragma unroll
  for (int i = 0; i < A_CH; ++i) {
    const int q = tid + i * T, r = q >> 3, c = q & 7;
    a_off[i] = static_cast<uint32_t>((r * g.sa_m + 4 * c) * 4);
    a_ok[i] = r < mv;
    a_k[i] = 4 * c;
    a_lds[i] = r * BK + 4 * (c ^ ((r >> 1) & 7));
  }
  uint32_t b_off[B_CH], b_lds[B_CH];
  int b_k[B_CH];
  bool b_ok[B_CH];
#pragma unroll
  for (int i = 0; i < B_CH; ++i) {
    const int q = tid + i * T;
    if constexpr (BKM) {
      const int r = q >> 3, c = q & 7;
      b_off[i] = static_cast<uint32_t>((r * g.sb_n + 4 * c) * 4);
      b_ok[i] = r < nv;
      b_k[i] = 4 * c;
      b_lds[i] = A_FL + r * BK + 4 * (c ^ ((r >> 1) & 7));
    } else {
      const int kr = q >> 5, c = q & 31;
      b_off[i] = static_cast<uint32_t>((kr * g.sb_k + 4 * c) * 4);
      b_ok[i] = 4 * c < nv;
      b_k[i] = kr;
      b_lds[i] = A_FL + kr * kBRow + 4 * c;
    }
  }
  const uint32_t b_kstep = BKM ? 4u : static_cast<uint32_t>(g.sb_k * 4);  // bytes per k
  const int kbeg = SPLITK ? static_cast<int>(blockIdx.y) * g.kchunk : 0;
  const int kend = SPLITK ? min(g.K, kbeg + g.kchunk) : g.K;
  f32x4 qa[A_CH], qb[B_CH];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i)
      qa[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            ra, a_ok[i] && k0 + a_k[i] < kend ? a_off[i] + k0 * 4u : kOOB, 0, 0));
#pragma unroll
    for (int i = 0; i < B_CH; ++i)
      qb[i] = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     rb, b_ok[i] && k0 + b_k[i] < kend ? b_off[i] + static_cast<uint32_t>(k0) * b_kstep : kOOB, 0, 0));
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) *reinterpret_cast<f32x4*>(&lds[buf][a_lds[i]]) = qa[i];
#pragma unroll
    for (int i = 0; i < B_CH; ++i) *reinterpret_cast<f32x4*>(&lds[buf][b_lds[i]]) = qb[i];
  };
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int r16 = lane & 15, kg = lane >> 4;
  // fragments of 16-k step s (0 or 1) of the tile in `la`
  auto fread = [&](const float* la, int s, f32x4 (&a)[4], f32x4 (&b)[4]) {
    const int c = 4 * s + kg;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = wm + 16 * i + r16;
      a[i] = *reinterpret_cast<const f32x4*>(&la[r * BK + 4 * (c ^ ((r >> 1) & 7))]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (BKM) {
        const int r = wn + 16 * j + r16;
        b[j] = *reinterpret_cast<const f32x4*>(&la[A_FL + r * BK + 4 * (c ^ ((r >> 1) & 7))]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) b[j][e] = la[A_FL + (16 * s + 4 * kg + e) * kBRow + wn + 16 * j + r16];
      }
    }
  };
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto mma = [&](const f32x4 (&a)[4], const f32x4 (&b)[4]) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][e], b[j][e], acc[i][j], 0, 0, 0);
  };
  gload(kbeg);
  lstore(0);
  __syncthreads();
  f32x4 fa0[4], fb0[4], fa1[4], fb1[4];
  fread(lds[0], 0, fa0, fb0);
  int buf = 0;
  for (int k0 = kbeg; k0 < kend; k0 += BK) {
    const bool more = k0 + BK < kend;
    if (more) gload(k0 + BK);
    fread(lds[buf], 1, fa1, fb1);
    mma(fa0, fb0);
    // The other buffer's last reads (the previous tile's second step) were
    // made before the previous barrier: it is free to refill.
    if (more) lstore(buf ^ 1);
    __syncthreads();
    if (more) fread(lds[buf ^ 1], 0, fa0, fb0);
    mma(fa1, fb1);
    buf ^= 1;
  }
  float* D = static_cast<float*>(g.D) + bat * g.sd_b;
  const float* Cp = g.use_c ? static_cast<const float*>(g.C) + bat * g.sc_b : nullptr;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = bm0 + wm + 16 * i + kg * 4 + r, n = bn0 + wn + 16 * j + r16;
        if (m < g.M && n < g.N) {
          if constexpr (SPLITK) {
            g.part[blockIdx.y * g.part_stride + (static_cast<int64_t>(bat) * g.M + m) * g.N + n] = acc[i][j][r];
          } else {
            float v = g.alpha * acc[i][j][r];
            if (Cp != nullptr) v += g.beta * Cp[m * g.sc_m + n * g.sc_n];
            D[static_cast<int64_t>(m) * g.sd_m + static_cast<int64_t>(n) * g.sd_n] = v;
          }
        }
      }
}

// fp32 products with an N-major B, without shared LDS tiles: each wave owns
// a 64 x 64 output tile and loads its operands straight from L2 (A as one
// 16-byte load per lane and 16-row block holding k0 + 4 (l >> 4) + e, whose
// element e feeds MFMA e; B as 16-byte row pieces, 4 k-rows x 64 columns per
// instruction, staged in a per-wave LDS tile with padded rows and read back
// per column).  The next 16-k step's operands are loaded before the current
// step's MFMAs.  No barriers, four waves per SIMD; the k order is the LDS
// kernel's, so the two give identical results.  Blocks of 2 x 2 waves cover
// 128 x 128.
__global__ __launch_bounds__(256, 3) void k_gemm_f32_reg(GemmArgs g) {
  constexpr int TM = 4, TN = 4;
  constexpr int kTrRow = 68;  // floats per k-row of the staged B tile (64 + 4: conflict-free reads)
  __shared__ __attribute__((aligned(16))) float trs[4][16 * kTrRow];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tm_count = (g.M + 127) / 128, tn_count = (g.N + 127) / 128;
  int bat, tmi, tni;
  tile_of(blockIdx.x, gridDim.x, tm_count, tn_count, bat, tmi, tni);
  const int m0 = tmi * 128 + (wave >> 1) * 64, n0 = tni * 128 + (wave & 1) * 64;
  const int mv = max(0, min(64, g.M - m0)), nv = max(0, min(64, g.N - n0));
  const int r16 = lane & 15, kq = (lane >> 4) * 4;
  const float* A = static_cast<const float*>(g.A) + bat * g.sa_b;
  const float* B = static_cast<const float*>(g.B) + bat * g.sb_b;
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc_uniform(
      A + static_cast<int64_t>(m0) * g.sa_m,
      mv > 0 ? static_cast<uint32_t>((static_cast<int64_t>(mv - 1) * g.sa_m + g.K) * 4) : 0u);
  const __amdgpu_buffer_rsrc_t rb = buffer_rsrc_uniform(
      B + n0, nv > 0 ? static_cast<uint32_t>((static_cast<int64_t>(g.K - 1) * g.sb_k + nv) * 4) : 0u);
  uint32_t a_off[TM];
  bool a_ok[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    a_off[i] = static_cast<uint32_t>(((16 * i + r16) * g.sa_m + kq) * 4);
    a_ok[i] = 16 * i + r16 < mv;
  }
  // load j covers k-rows 4 j + (l >> 4), columns 4 (l & 15) .. + 3
  uint32_t b_off[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) b_off[j] = static_cast<uint32_t>(((4 * j + (lane >> 4)) * g.sb_k + 4 * r16) * 4);
  const bool b_ok = 4 * r16 < nv;
  const uint32_t b_kstep = static_cast<uint32_t>(g.sb_k * 4);  // bytes per k
  auto load = [&](int k, f32x4 (&aq)[TM], f32x4 (&bq)[TN]) {
    const bool k_ok = k + kq < g.K;
#pragma unroll
    for (int i = 0; i < TM; ++i)
      aq[i] = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, a_ok[i] && k_ok ? a_off[i] + k * 4u : kOOB, 0, 0));
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const bool ok = b_ok && k + 4 * j + (lane >> 4) < g.K;
      bq[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            rb, ok ? b_off[j] + static_cast<uint32_t>(k) * b_kstep : kOOB, 0, 0));
    }
  };
  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 aq[TM], bq[TN];
  load(0, aq, bq);
  for (int k0 = 0; k0 < g.K; k0 += 16) {
    f32x4 an[TM], bn[TN];
    load(k0 + 16, an, bn);  // past K every lane reads the out-of-range offset (zeros)
    // Stage the step's 16 x 64 B tile (row-major, padded rows) and read
    // column l & 15 of k-rows 4 (l >> 4) + e back for each 16-column group.
#pragma unroll
    for (int j = 0; j < TN; ++j)
      *reinterpret_cast<f32x4*>(&trs[wave][(4 * j + (lane >> 4)) * kTrRow + 4 * r16]) = bq[j];
    f32x4 bf[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) bf[j][e] = trs[wave][(kq + e) * kTrRow + 16 * j + r16];
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(aq[i][e], bf[j][e], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < TM; ++i) aq[i] = an[i];
#pragma unroll
    for (int j = 0; j < TN; ++j) bq[j] = bn[j];
  }
  float* D = static_cast<float*>(g.D) + bat * g.sd_b;
  const float* Cp = g.use_c ? static_cast<const float*>(g.C) + bat * g.sc_b : nullptr;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + 16 * i + (lane >> 4) * 4 + r, n = n0 + 16 * j + r16;
        if (m < g.M && n < g.N) {
          float v = g.alpha * acc[i][j][r];
          if (Cp != nullptr) v += g.beta * Cp[m * g.sc_m + n * g.sc_n];
          D[static_cast<int64_t>(m) * g.sd_m + static_cast<int64_t>(n) * g.sd_n] = v;
        }
      }
}

template <bool BKM, int WM>
int launch_f32_lds(const GemmArgs& g, hipStream_t st) {
  const int64_t tiles = static_cast<int64_t>((g.M + 64 * WM - 1) / (64 * WM)) * ((g.N + 127) / 128) * g.batch;
  if (tiles > 0x7fffffffLL) return set_error(NTOPS_ERR_UNSUPPORTED, "gemm: too many tiles");
  note_kernel("gemm_f32_lds m%d %s", 64 * WM, BKM ? "B:K" : "B:N");
  hipLaunchKernelGGL((k_gemm_f32_lds<BKM, WM>), dim3(static_cast<unsigned>(tiles)), dim3(128 * WM), 0, st, g);
  return check_launch("gemm");
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

// ---- split-K reduction -----------------------------------------------------
// out = alpha * (sum of the S fp32 partial tiles, in slice order) + beta * C,
// rounded once; a thread owns 4 consecutive columns of one row (the
// partials' 16-byte runs).  Fixed order, so the result does not depend on
// which slice finished first.
template <typename T, int CM>
__global__ __launch_bounds__(256) void k_gemm_splitk_reduce(GemmArgs g, int S) {
  const int n4 = g.N / 4;
  const int64_t per_batch = static_cast<int64_t>(g.M) * n4;
  int64_t id = block_id() * 256 + threadIdx.x;
  if (id >= per_batch * g.batch) return;
  const int bat = static_cast<int>(id / per_batch);
  id -= bat * per_batch;
  const int m = static_cast<int>(id / n4), n = static_cast<int>(id - static_cast<int64_t>(m) * n4) * 4;
  const float* P = g.part + (static_cast<int64_t>(bat) * g.M + m) * g.N + n;
  f32x4 sum = *reinterpret_cast<const f32x4*>(P);
  for (int z = 1; z < S; ++z) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(P + z * g.part_stride);
    sum.x += v.x;
    sum.y += v.y;
    sum.z += v.z;
    sum.w += v.w;
  }
  float c[4];
  c_values<T, CM>(g, static_cast<const T*>(g.C) + bat * g.sc_b, m, n, true, c);
  T o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float v = g.alpha * sum[e];
    if constexpr (CM != kCNone) v += c[e];
    o[e] = static_cast<T>(v);
  }
  T* D = static_cast<T*>(g.D) + bat * g.sd_b + static_cast<int64_t>(m) * g.sd_m;
  constexpr uintptr_t kAlign = 4 * sizeof(T) - 1;
  if (g.sd_n == 1 && (reinterpret_cast<uintptr_t>(D + n) & kAlign) == 0) {
    if constexpr (sizeof(T) == 2)
      *reinterpret_cast<u32x2*>(D + n) = __builtin_bit_cast(u32x2, o);
    else
      *reinterpret_cast<u32x4*>(D + n) = __builtin_bit_cast(u32x4, o);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) D[static_cast<int64_t>(n + e) * g.sd_n] = o[e];
  }
}

// ---- host dispatch ---------------------------------------------------------
template <typename T>
int launch_splitk_reduce(const GemmArgs& g, int S, hipStream_t st) {
  const dim3 grid = blocks_2d(ceil_div(static_cast<int64_t>(g.M) * (g.N / 4) * g.batch, 256));
  switch (g.use_c ? g.c_mode : kCNone) {
    case kCNone: hipLaunchKernelGGL((k_gemm_splitk_reduce<T, kCNone>), grid, dim3(256), 0, st, g, S); break;
    case kCVec4: hipLaunchKernelGGL((k_gemm_splitk_reduce<T, kCVec4>), grid, dim3(256), 0, st, g, S); break;
    case kCRow: hipLaunchKernelGGL((k_gemm_splitk_reduce<T, kCRow>), grid, dim3(256), 0, st, g, S); break;
    default: hipLaunchKernelGGL((k_gemm_splitk_reduce<T, kCStrided>), grid, dim3(256), 0, st, g, S); break;
  }
  return check_launch("gemm");
}

template <typename T, int BM, int BN, int WM, int WN, int BK, int STAGES, bool AK, bool BKM, bool EVEN,
          int CONV = 0>
int launch_mfma(const GemmArgs& g, hipStream_t st) {
  constexpr int NT = WM * WN * 64;
  constexpr int kLds = STAGES * (BM + BN) * BK * 2;
  auto kern = k_gemm_mfma<T, BM, BN, WM, WN, BK, STAGES, AK, BKM, EVEN, CONV>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLds) != hipSuccess)
      return set_error(NTOPS_ERR_HIP, "gemm: cannot reserve %d bytes of LDS", kLds);
    attr_set = true;
  }
  const int64_t tiles = static_cast<int64_t>((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN) * g.batch;
  if (tiles > 0x7fffffffLL) return set_error(NTOPS_ERR_UNSUPPORTED, "gemm: too many tiles");
  note_kernel("gemm_mfma %dx%d s%d %s %s %s%s", BM, BN, STAGES, AK ? "A:K" : "A:M", BKM ? "B:K" : "B:N",
              EVEN ? "even" : "ragged", CONV == 1 ? " conv" : CONV == 2 ? " conv_cl" : "");
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(tiles)), dim3(NT), kLds, st, g);
  return check_launch("gemm");
}

// Picks the epilogue's C access (see c_values) from C's strides and alignment.
void set_c_mode(GemmArgs& g) {
  if (!g.use_c)
    g.c_mode = kCNone;
  else if (g.sc_n == 0)
    g.c_mode = kCRow;
  else if (g.sc_n == 1 && g.sc_m % 4 == 0 && (g.batch == 1 || g.sc_b % 4 == 0) &&
           (reinterpret_cast<uintptr_t>(g.C) & 7u) == 0)
    g.c_mode = kCVec4;
  else
    g.c_mode = kCStrided;
}

// Number of CUs of the current device (queried once per device).
int cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cache[dev] = n;
  }
  return cache[dev];
}

template <typename T, bool AK, bool BKM>
int launch_panel(const GemmArgs& g, hipStream_t st) {
  constexpr int kLds = kPanelLds;
  auto kern = k_gemm_panel<T, AK, BKM>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLds) != hipSuccess)
      return set_error(NTOPS_ERR_HIP, "gemm: cannot reserve %d bytes of LDS", kLds);
    attr_set = true;
  }
  // Units of `seg` tiles down a tile column: the longest divisor of the
  // column's tile count that still leaves a unit for every block.
  const int cus = cu_count() > 0 ? cu_count() : 256;
  const int tm = g.M / 128;
  const int64_t cols = static_cast<int64_t>(g.N / 128) * g.batch;
  int seg = 1;
  for (int d = tm; d >= 1; --d) {
    if (tm % d == 0 && cols * (tm / d) >= cus * kPanelBlocksPerCu) {
      seg = d;
      break;
    }
  }
  const int64_t units = cols * (tm / seg);
  // Two blocks per CU; a multiple of 8 keeps each block on one XCD for the
  // whole walk.
  int64_t grid = (cus * kPanelBlocksPerCu / 8) * 8;
  if (grid <= 0) grid = 256;
  if (grid > units) grid = units;
  note_kernel("gemm_panel %s %s seg%d", AK ? "A:K" : "A:M", BKM ? "B:K" : "B:N", seg);
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(grid)), dim3(256), kLds, st, g, seg);
  return check_launch("gemm");
}

// 128 x 128 tiles of the product that leave a quarter of the CUs idle.
bool few_tiles128(int64_t M, int64_t N, int64_t batch) {
  const int64_t tiles = ((M + 127) / 128) * ((N + 127) / 128) * batch;
  return tiles * 4 <= static_cast<int64_t>(cu_count_cached()) * 3;
}

// Split-K for products whose 128 x 128 tiles do not fill the chip (few rows
// times few columns, long K: decode- and prefill-sized linear layers): the
// tiles times S slices of K make at most two blocks per CU (one round), each
// slice at least 512 deep.  1 = no split.
int splitk_slices(int64_t M, int64_t N, int64_t K, int* kchunk) {
  const int64_t tiles = ((M + 127) / 128) * ((N + 127) / 128);
  const int64_t cus = cu_count_cached();
  if (K < 1024 || !few_tiles128(M, N, 1)) return 1;
  int64_t S = 2 * cus / tiles;  // whole rounds of two blocks per CU
  S = std::min<int64_t>(std::min<int64_t>(S, K / 512), 16);
  if (S < 2) return 1;
  const int64_t chunk = ((K + S - 1) / S + 31) / 32 * 32;
  *kchunk = static_cast<int>(chunk);
  return static_cast<int>((K + chunk - 1) / chunk);
}

// fp32 split over K for products whose 128 x 128 tiles leave CUs idle:
// up to two blocks per CU, slices of at least 128 k (an fp32 k-step costs
// eight times a 16-bit one on the matrix cores, so shorter slices than the
// 16-bit path's 512 still pay for their partial tile); products with one to
// two tiles per CU (one wave per SIMD) and K >= 1024 split in two.
int splitk_slices_f32(int64_t M, int64_t N, int64_t K, int64_t batch, int* kchunk) {
  const int64_t tiles = ((M + 127) / 128) * ((N + 127) / 128) * batch;
  const int64_t cus = cu_count_cached() > 0 ? cu_count_cached() : 256;
  if (tiles >= 2 * cus || M <= kSkinnyMaxM || N % 4 != 0) return 1;
  int64_t S = tiles >= cus ? (K >= 1024 ? 2 : 1) : std::min<int64_t>(std::min<int64_t>(2 * cus / tiles, K / 128), 16);
  if (S < 2) return 1;
  const int64_t chunk = ((K + S - 1) / S + 31) / 32 * 32;
  *kchunk = static_cast<int>(chunk);
  return static_cast<int>((K + chunk - 1) / chunk);
}

template <bool BKM>
int launch_f32_splitk(GemmArgs g, int S, hipStream_t st) {
  const int64_t tiles = static_cast<int64_t>((g.M + 127) / 128) * ((g.N + 127) / 128) * g.batch;
  note_kernel("gemm_f32_lds m128 %s splitk%d", BKM ? "B:K" : "B:N", S);
  hipLaunchKernelGGL((k_gemm_f32_lds<BKM, 2, true>), dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(S)),
                     dim3(256), 0, st, g);
  const int rc = check_launch("gemm");
  if (rc != NTOPS_OK) return rc;
  if (g.c_mode == kCVec4) g.c_mode = kCStrided;  // (kCVec4 reads four 16-bit values)
  return launch_splitk_reduce<float>(g, S, st);
}

template <typename T, bool AK, bool BKM, bool EVEN>
int launch_splitk_part(const GemmArgs& g, int S, hipStream_t st) {
  constexpr int kLds = 4 * (128 + 128) * 32 * 2;
  auto kern = k_gemm_mfma<T, 128, 128, 2, 2, 32, 4, AK, BKM, EVEN, 0, true>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLds) != hipSuccess)
      return set_error(NTOPS_ERR_HIP, "gemm: cannot reserve %d bytes of LDS", kLds);
    attr_set = true;
  }
  const int64_t tiles = static_cast<int64_t>((g.M + 127) / 128) * ((g.N + 127) / 128);
  note_kernel("gemm_mfma 128x128 s4 %s %s %s splitk%d", AK ? "A:K" : "A:M", BKM ? "B:K" : "B:N",
              EVEN ? "even" : "ragged", S);
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(S)), dim3(256), kLds, st, g);
  return check_launch("gemm");
}

// The S partial products into the workspace, then their ordered sum (with
// alpha, beta * C and the one rounding) into out.
template <typename T, bool AK, bool BKM>
int launch_splitk(GemmArgs g, int S, hipStream_t st) {
  const bool even = g.M % 128 == 0 && g.N % 128 == 0 && g.K % 32 == 0;
  const int rc = even ? launch_splitk_part<T, AK, BKM, true>(g, S, st) : launch_splitk_part<T, AK, BKM, false>(g, S, st);
  if (rc != NTOPS_OK) return rc;
  return launch_splitk_reduce<T>(g, S, st);
}

template <typename T, bool AK, bool BKM>
int pick_tile(const GemmArgs& g, hipStream_t st) {
  if (g.K <= kPanelK && g.M % 128 == 0 && g.N % 128 == 0 && g.staged &&
      static_cast<int64_t>(g.M / 128) * (g.N / 128) * g.batch <= 0x7fffffffLL)
    return launch_panel<T, AK, BKM>(g, st);
  const int64_t big_tiles = static_cast<int64_t>((g.M + 255) / 256) * ((g.N + 255) / 256) * g.batch;
  constexpr int kBK = 32, kStages = 4;
  if (big_tiles >= 240 && g.K > 256) {
    const bool even = g.M % 256 == 0 && g.N % 256 == 0 && g.K % kBK == 0;
    if (even) return launch_mfma<T, 256, 256, 2, 4, kBK, kStages, AK, BKM, true>(g, st);
    // M or N not a multiple of 256: the bounds-checked kernel runs a third
    // slower than the even one over the whole product (bf16 8192 x 50264 x
    // 768: 839 against 625 us at N = 50176), so the even kernel takes the
    // 256-aligned interior and 128 x 128 ragged tiles the edge strips (right:
    // all rows; bottom: the interior's columns).
    const int m0 = g.M / 256 * 256, n0 = g.N / 256 * 256;
    if (g.K % kBK == 0 && static_cast<int64_t>(m0 / 256) * (n0 / 256) * g.batch >= 240) {
      const int64_t es = sizeof(T);
      GemmArgs in = g;
      in.M = m0;
      in.N = n0;
      int rc = launch_mfma<T, 256, 256, 2, 4, kBK, kStages, AK, BKM, true>(in, st);
      if (rc == NTOPS_OK && n0 < g.N) {
        GemmArgs r = g;
        r.N = g.N - n0;
        r.B = static_cast<const char*>(g.B) + n0 * g.sb_n * es;
        r.D = static_cast<char*>(g.D) + n0 * g.sd_n * es;
        if (g.use_c) r.C = static_cast<const char*>(g.C) + n0 * g.sc_n * es;
        rc = launch_mfma<T, 128, 128, 2, 2, kBK, kStages, AK, BKM, false>(r, st);
      }
      if (rc == NTOPS_OK && m0 < g.M) {
        GemmArgs b = g;
        b.M = g.M - m0;
        b.N = n0;
        b.A = static_cast<const char*>(g.A) + m0 * g.sa_m * es;
        b.D = static_cast<char*>(g.D) + m0 * g.sd_m * es;
        if (g.use_c) b.C = static_cast<const char*>(g.C) + m0 * g.sc_m * es;
        rc = launch_mfma<T, 128, 128, 2, 2, kBK, kStages, AK, BKM, false>(b, st);
      }
      if (rc == NTOPS_OK)
        note_kernel("gemm_mfma 256x256 s4 %s %s even+edges", AK ? "A:K" : "A:M", BKM ? "B:K" : "B:N");
      return rc;
    }
    return launch_mfma<T, 256, 256, 2, 4, kBK, kStages, AK, BKM, false>(g, st);
  }
  const bool even = g.M % 128 == 0 && g.N % 128 == 0 && g.K % kBK == 0;
  if (g.K <= 256) {
    // Short K: a tile's life is operand latency + a few MFMAs + its
    // epilogue; 2 stages (32 KiB of LDS) let 4-5 tiles share a CU and
    // overlap those phases.
    if (even) return launch_mfma<T, 128, 128, 2, 2, kBK, 2, AK, BKM, true>(g, st);
    return launch_mfma<T, 128, 128, 2, 2, kBK, 2, AK, BKM, false>(g, st);
  }
  if (even) return launch_mfma<T, 128, 128, 2, 2, kBK, kStages, AK, BKM, true>(g, st);
  return launch_mfma<T, 128, 128, 2, 2, kBK, kStages, AK, BKM, false>(g, st);
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
    // (any output layout: 4-column runs at 8-byte aligned addresses are
    // stored as such, anything else element by element -- g.ragged)
    const bool batch_ok = (g.batch == 1) || (g.sa_b % 8 == 0 && g.sb_b % 8 == 0);
    // Every operand byte offset inside a tile's buffer resource must stay
    // below 2 GiB (out-of-range chunks use offset 2^31).
    const int64_t lim = int64_t(1) << 31;
    const bool fits = (a_k ? (256 * g.sa_m + g.K) : (static_cast<int64_t>(g.K) * g.sa_k + 256)) * 2 < lim &&
                      (b_k ? (256 * g.sb_n + g.K) : (static_cast<int64_t>(g.K) * g.sb_k + 256)) * 2 < lim;
    // K == 0 goes to the generic kernel, which never touches A or B (they may
    // be null, and an empty M/N-major operand has no valid buffer extent).
    if (g.K > 0 && (a_k || a_m) && (b_k || b_n) && batch_ok && fits && al(g.A) && al(g.B)) {
      int kchunk = 0;
      // (up to kSplitKMinM rows a K-major A takes the skinny kernel)
      // (the reduce kernel sums 4-column groups: N % 4 == 0)
      const int S = (g.part != nullptr && g.batch == 1 && g.N % 4 == 0 && (g.M > kSplitKMinM || !a_k))
                        ? splitk_slices(g.M, g.N, g.K, &kchunk)
                        : 1;
      if (S > 1 && static_cast<int64_t>(S) * g.M * g.N * 4 <= g.part_bytes) {
        g.kchunk = kchunk;
        g.part_stride = static_cast<int64_t>(g.M) * g.N;
        if (a_k && b_n) return launch_splitk<T, true, false>(g, S, st);
        if (a_k && b_k) return launch_splitk<T, true, true>(g, S, st);
        if (a_m && b_n) return launch_splitk<T, false, false>(g, S, st);
        return launch_splitk<T, false, true>(g, S, st);
      }
      if (a_k && g.M <= kSkinnyMaxM && g.batch <= 65535 &&
          (g.M <= kSkinnyRouteM || few_tiles128(g.M, g.N, g.batch)))
        return b_k ? launch_skinny<T, true>(g, st) : launch_skinny<T, false>(g, st);
      if (a_k && b_n) return pick_tile<T, true, false>(g, st);
      if (a_k && b_k) return pick_tile<T, true, true>(g, st);
      if (a_m && b_n) return pick_tile<T, false, false>(g, st);
      return pick_tile<T, false, true>(g, st);
    }
  }
  if constexpr (std::is_same<T, float>::value) {
    // fp32 with few rows: the skinny MFMA kernel (K-major A, 16-byte rows).
    const bool a_k = g.sa_k == 1 && g.sa_m % 4 == 0 && g.K % 4 == 0;
    const bool b_k = g.sb_k == 1 && g.sb_n % 4 == 0;
    const bool b_n = g.sb_n == 1 && g.sb_k % 4 == 0 && g.N % 4 == 0 && !b_k;
    const bool batch_ok = g.batch <= 65535 && (g.batch == 1 || (g.sa_b % 4 == 0 && g.sb_b % 4 == 0));
    const int64_t lim = int64_t(1) << 31;
    const bool fits = (static_cast<int64_t>(kSkinnyMaxM) * g.sa_m + g.K) * 4 < lim &&
                      (b_k ? (16 * 64 * g.sb_n + g.K) : (static_cast<int64_t>(g.K) * g.sb_k + 64)) * 4 < lim;
    // (also for a batch of them: a convolution's 64-channel images of 3136
    // pixels measured 158 us here against 181 us in the tile kernel's 64-row
    // blocks; and 33-64 rows split over K in 64-row blocks measured slower,
    // 64 x 14336 x 4096 139 against 114 us, except at K = 14336)
    if (g.K > 0 && g.M <= kSkinnyMaxM && a_k && (b_k || b_n) && batch_ok && fits && aligned16(g.A) &&
        aligned16(g.B))
      return b_k ? launch_skinny_f32<true>(g, st) : launch_skinny_f32<false>(g, st);
    // Larger fp32 products.  When 128 x 128 tiles fill every CU (and M > 64),
    // the LDS-tiled kernel's 128-row blocks, except for an N-major B with
    // three or more tiles per CU: the LDS-free kernel, whose four waves per
    // SIMD then beat the LDS kernel's two by 4-8 % (with one tile per CU it
    // is 12-23 % slower, and 3-5 % slower for a K-major B at any count).
    // Fewer tiles: the LDS kernel's 64-row blocks (twice the blocks, none
    // half empty).
    const bool b_n4 = g.sb_n == 1 && g.sb_k % 4 == 0 && g.N % 4 == 0 && !b_k;
    const bool fits_t = (256 * g.sa_m + g.K) * 4 < lim &&
                        (b_k ? (128 * g.sb_n + g.K) : (static_cast<int64_t>(g.K) * g.sb_k + 128)) * 4 < lim;
    if (g.K > 0 && a_k && (b_k || b_n4) && fits_t && aligned16(g.A) && aligned16(g.B) &&
        (g.batch == 1 || (g.sa_b % 4 == 0 && g.sb_b % 4 == 0))) {
      int kchunk = 0;
      const int S = g.part != nullptr ? splitk_slices_f32(g.M, g.N, g.K, g.batch, &kchunk) : 1;
      if (S > 1 && static_cast<int64_t>(S) * g.batch * g.M * g.N * 4 <= g.part_bytes) {
        g.kchunk = kchunk;
        g.part_stride = static_cast<int64_t>(g.batch) * g.M * g.N;
        return b_k ? launch_f32_splitk<true>(g, S, st) : launch_f32_splitk<false>(g, S, st);
      }
      const int64_t cus = cu_count_cached() > 0 ? cu_count_cached() : 256;
      const int64_t tiles = static_cast<int64_t>((g.M + 127) / 128) * ((g.N + 127) / 128) * g.batch;
      if (g.M > 64 && tiles >= cus) {
        if (b_k || tiles < 3 * cus) return b_k ? launch_f32_lds<true, 2>(g, st) : launch_f32_lds<false, 2>(g, st);
        if (tiles > 0x7fffffffLL) return set_error(NTOPS_ERR_UNSUPPORTED, "gemm: too many tiles");
        note_kernel("gemm_f32_reg B:N");
        hipLaunchKernelGGL(k_gemm_f32_reg, dim3(static_cast<unsigned>(tiles)), dim3(256), 0, st, g);
        return check_launch("gemm");
      }
      return b_k ? launch_f32_lds<true, 1>(g, st) : launch_f32_lds<false, 1>(g, st);
    }
  }
  const int64_t tiles = static_cast<int64_t>((g.M + 63) / 64) * ((g.N + 63) / 64) * g.batch;
  if (tiles > 0x7fffffffLL) return set_error(NTOPS_ERR_UNSUPPORTED, "gemm: too many tiles");
  note_kernel("gemm_generic");
  hipLaunchKernelGGL((k_gemm_generic<T>), dim3(static_cast<unsigned>(tiles)), dim3(256), 0, st, g);
  return check_launch("gemm");
}

// CONV 1: shifted planes (B N-major); CONV 2: channels-last (B K-major).
template <typename T, int CONV>
int run_implicit_conv(const GemmArgs& g, hipStream_t st) {
  constexpr int kBK = 32, kStages = 4;
  constexpr bool BKM = CONV == 2;
  const int64_t big_tiles = static_cast<int64_t>((g.M + 255) / 256) * ((g.N + 255) / 256) * g.batch;
  if (big_tiles >= 240 && g.K > 256) {
    if (g.M % 256 == 0 && g.N % 256 == 0 && g.K % kBK == 0)
      return launch_mfma<T, 256, 256, 2, 4, kBK, kStages, true, BKM, true, CONV>(g, st);
    return launch_mfma<T, 256, 256, 2, 4, kBK, kStages, true, BKM, false, CONV>(g, st);
  }
  if (g.M % 128 == 0 && g.N % 128 == 0 && g.K % kBK == 0)
    return launch_mfma<T, 128, 128, 2, 2, kBK, kStages, true, BKM, true, CONV>(g, st);
  return launch_mfma<T, 128, 128, 2, 2, kBK, kStages, true, BKM, false, CONV>(g, st);
}

}  // namespace

int gemm_implicit_conv(int dtype, int batch, int M, int N, int K, const void* w, int64_t w_ld,
                       const void* b_base, int64_t b_batch, int R, int S, int64_t per_s, int64_t per_c,
                       int64_t per_r, const void* bias, int64_t bias_stride, void* out, int64_t out_batch,
                       int64_t out_ld, hipStream_t st) {
  if (batch <= 0 || M <= 0 || N <= 0 || K <= 0) return NTOPS_OK;
  if (!aligned16(w) || !aligned16(b_base) || w_ld % 8 || N % 8 || per_s % 8 || per_c % 8 || per_r % 8 ||
      b_batch % 8 || K % 8 || out_ld % 4 || out_batch % 4 || (reinterpret_cast<uintptr_t>(out) & 7u))
    return set_error(NTOPS_ERR_UNSUPPORTED, "conv2d: operand layout unsuited to the implicit GEMM");
  if (b_batch * 2 >= (int64_t(1) << 31) || (256 * w_ld + K) * 2 >= (int64_t(1) << 31))
    return set_error(NTOPS_ERR_UNSUPPORTED, "conv2d: operand exceeds the 2 GiB buffer range");
  GemmArgs g{};
  g.A = w;
  g.B = b_base;
  g.D = out;
  g.sa_b = 0;
  g.sa_m = w_ld;
  g.sa_k = 1;
  g.sb_b = b_batch;
  g.sb_k = 0;  // rows come from the convolution descriptor
  g.sb_n = 1;
  g.sd_b = out_batch;
  g.sd_m = out_ld;
  g.sd_n = 1;
  g.M = M;
  g.N = N;
  g.K = K;
  g.batch = batch;
  g.alpha = 1.f;
  g.beta = bias ? 1.f : 0.f;
  g.use_c = bias ? 1 : 0;
  g.C = bias;
  g.sc_b = 0;
  g.sc_m = bias ? bias_stride : 0;
  g.sc_n = 0;
  set_c_mode(g);
  g.staged = (out_ld % 8 == 0 && (batch == 1 || out_batch % 8 == 0) && N % 8 == 0 &&
              (reinterpret_cast<uintptr_t>(out) & 15u) == 0)
                 ? 1
                 : 0;
  constexpr int kBK = 32;  // k-rows per tile of the kernels run_implicit_conv launches
  g.cv_rs = R * S;
  g.cv_r = R;
  g.cv_s = S;
  g.cv_ds = kBK % S;
  g.cv_dr = (kBK / S) % R;
  g.cv_dc = kBK / (R * S);
  g.cv_per_s = per_s;
  g.cv_per_c = per_c;
  g.cv_per_r = per_r;
  switch (dtype) {
    case NTOPS_BF16: return run_implicit_conv<__bf16, 1>(g, st);
    case NTOPS_F16: return run_implicit_conv<_Float16, 1>(g, st);
    default: return set_error(NTOPS_ERR_UNSUPPORTED, "conv2d: the implicit GEMM needs BF16 or F16");
  }
}

int gemm_conv_channels_last(int dtype, int batch, int M, int N, int K, const void* w, const void* xt,
                            int64_t img_elems, int R, int S, int C, int Q, int sh, int sw, int wp, int dh,
                            int dw, const void* bias, int64_t bias_stride, void* out, int64_t out_batch,
                            int64_t out_ld, hipStream_t st) {
  if (batch <= 0 || M <= 0 || N <= 0 || K <= 0) return NTOPS_OK;
  if (!aligned16(w) || !aligned16(xt) || C % 32 || K != R * S * C || N % 4 || img_elems % 8 || out_ld % 4 ||
      out_batch % 4 || (reinterpret_cast<uintptr_t>(out) & 7u))
    return set_error(NTOPS_ERR_UNSUPPORTED, "conv2d: operand layout unsuited to the channels-last GEMM");
  if (img_elems * 2 >= (int64_t(1) << 31) || (257 * static_cast<int64_t>(K)) * 2 >= (int64_t(1) << 31))
    return set_error(NTOPS_ERR_UNSUPPORTED, "conv2d: operand exceeds the 2 GiB buffer range");
  GemmArgs g{};
  g.A = w;
  g.B = xt;
  g.D = out;
  g.sa_b = 0;
  g.sa_m = K;
  g.sa_k = 1;
  g.sb_b = img_elems;
  g.sb_k = 1;
  g.sb_n = 0;  // rows come from the convolution geometry
  g.sd_b = out_batch;
  g.sd_m = out_ld;
  g.sd_n = 1;
  g.M = M;
  g.N = N;
  g.K = K;
  g.batch = batch;
  g.alpha = 1.f;
  g.beta = bias ? 1.f : 0.f;
  g.use_c = bias ? 1 : 0;
  g.C = bias;
  g.sc_b = 0;
  g.sc_m = bias ? bias_stride : 0;
  g.sc_n = 0;
  set_c_mode(g);
  g.staged = (out_ld % 8 == 0 && (batch == 1 || out_batch % 8 == 0) && N % 8 == 0 &&
              (reinterpret_cast<uintptr_t>(out) & 15u) == 0)
                 ? 1
                 : 0;
  g.cv_r = R;
  g.cv_s = S;
  g.cl_q = Q;
  g.cl_sh = sh;
  g.cl_sw = sw;
  g.cl_wp = wp;
  g.cl_c = C;
  g.cl_dh = dh;
  g.cl_dw = dw;
  switch (dtype) {
    case NTOPS_BF16: return run_implicit_conv<__bf16, 2>(g, st);
    case NTOPS_F16: return run_implicit_conv<_Float16, 2>(g, st);
    default: return set_error(NTOPS_ERR_UNSUPPORTED, "conv2d: the channels-last GEMM needs BF16 or F16");
  }
}

namespace {
}  // namespace
}  // namespace ntops

using namespace ntops;

static int gemm_entry(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K, const void* A,
                      const int64_t* a_strides, const void* B, const int64_t* b_strides, const void* C,
                      const int64_t* c_strides, double alpha, double beta, void* out, const int64_t* out_strides,
                      void* workspace, int64_t workspace_bytes, void* stream) {
  if (batch < 0 || M < 0 || N < 0 || K < 0) return set_error(NTOPS_ERR_INVALID, "gemm: negative size");
  if (batch > 0x7fffffffLL || M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL)
    return set_error(NTOPS_ERR_UNSUPPORTED, "gemm: size exceeds int32");
  if (batch == 0 || M == 0 || N == 0) return NTOPS_OK;
  if (out == nullptr || out_strides == nullptr || a_strides == nullptr || b_strides == nullptr)
    return set_error(NTOPS_ERR_INVALID, "gemm: null pointer");
  if (K > 0 && (A == nullptr || B == nullptr)) return set_error(NTOPS_ERR_INVALID, "gemm: null operand");
  GemmArgs g{};
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
  g.ragged = (out_strides[2] == 1 && out_strides[1] % 4 == 0 && (batch == 1 || out_strides[0] % 4 == 0) &&
              (reinterpret_cast<uintptr_t>(out) & 7u) == 0)
                 ? 0
                 : 1;
  g.staged = (out_strides[2] == 1 && out_strides[1] % 8 == 0 && (batch == 1 || out_strides[0] % 8 == 0) &&
              N % 8 == 0 && (reinterpret_cast<uintptr_t>(out) & 15u) == 0)
                 ? 1
                 : 0;
  g.shifted = (!g.staged && out_strides[2] == 1 && (reinterpret_cast<uintptr_t>(out) & 1u) == 0) ? 1 : 0;
  g.C = C;
  if (g.use_c) {
    if (c_strides == nullptr) return set_error(NTOPS_ERR_INVALID, "gemm: null C strides");
    g.sc_b = c_strides[0];
    g.sc_m = c_strides[1];
    g.sc_n = c_strides[2];
  } else {
    g.sc_b = g.sc_m = g.sc_n = 0;
  }
  set_c_mode(g);
  // the workspace serves split-K only when 16-byte aligned
  if (workspace != nullptr && workspace_bytes > 0 && (reinterpret_cast<uintptr_t>(workspace) & 15u) == 0) {
    g.part = static_cast<float*>(workspace);
    g.part_bytes = workspace_bytes;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  return dispatch_float16_32(dtype, "gemm", [&](auto tag) {
    using T = decltype(tag);
    return run_gemm<T>(g, st);
  });
}

extern "C" int ntops_gemm(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K, const void* A,
                          const int64_t* a_strides, const void* B, const int64_t* b_strides, const void* C,
                          const int64_t* c_strides, double alpha, double beta, void* out,
                          const int64_t* out_strides, void* stream) {
  return gemm_entry(dtype, batch, M, N, K, A, a_strides, B, b_strides, C, c_strides, alpha, beta, out, out_strides,
                    nullptr, 0, stream);
}

extern "C" int ntops_gemm_ws(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K, const void* A,
                             const int64_t* a_strides, const void* B, const int64_t* b_strides, const void* C,
                             const int64_t* c_strides, double alpha, double beta, void* out,
                             const int64_t* out_strides, void* workspace, int64_t workspace_bytes, void* stream) {
  if (workspace_bytes < 0) return set_error(NTOPS_ERR_INVALID, "gemm: negative workspace size");
  return gemm_entry(dtype, batch, M, N, K, A, a_strides, B, b_strides, C, c_strides, alpha, beta, out, out_strides,
                    workspace, workspace_bytes, stream);
}

extern "C" int64_t ntops_gemm_workspace(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K) {
  if ((dtype != NTOPS_BF16 && dtype != NTOPS_F16 && dtype != NTOPS_F32) || batch < 1 || M <= 0 || N <= 0 ||
      K <= 0 || batch > 0x7fffffffLL || M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL)
    return 0;
  if (dtype == NTOPS_F32) {
    int kchunk = 0;
    const int S = splitk_slices_f32(M, N, K, batch, &kchunk);
    return S > 1 ? static_cast<int64_t>(S) * batch * M * N * 4 : 0;
  }
  if (batch != 1) return 0;
  // (a K-major A of up to kSplitKMinM rows takes the skinny kernel instead
  // and leaves the workspace unused)
  int kchunk = 0;
  const int S = splitk_slices(M, N, K, &kchunk);
  return S > 1 ? static_cast<int64_t>(S) * M * N * 4 : 0;
}
