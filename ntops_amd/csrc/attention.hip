// scaled_dot_product_attention forward:  O = softmax(Q K^T * scale + M) V.
//
// Reference: kernels/scaled_dot_product_attention.py:154-201 (an online
// softmax over key blocks in base 2: running max, exp2 of the shifted
// scores, rescaled accumulator; P cast to the value dtype for P @ V; the
// final O / l), torch/scaled_dot_product_attention.py:10-108 (GQA head
// mapping, bool masks as 0 / -inf, default scale 1 / sqrt(D), the two causal
// variants).  Rows whose every score is masked produce 0, as torch's CPU
// kernel does (the reference would produce NaN).
//
// MFMA path (bf16 / f16, unit stride along D, head dim a multiple of 8 up to
// 128: kernels for D = 64 and 128, the columns past a smaller head dim read
// as zero from Q, K and V -- their products add nothing to S, and their O
// columns are zero and never stored):
//  * one 4-wave workgroup per (batch, head, 128 query rows); wave w owns 32
//    rows and keeps their Q fragments in VGPRs for the whole kernel;
//  * key / value tiles of 64 rows are double-buffered in LDS (the next
//    tile's global loads are in flight while the current one is used; one
//    barrier per tile).  K is stored [kv][d] and read as the B operand of
//    S = Q K^T with ds_read_b128; V is stored [kv][d] and read as the B
//    operand of O += P V with ds_read_b64_tr_b16 (transposing reads); both
//    layouts are XOR-swizzled so every fragment read is bank-conflict free;
//  * S (32 x 64 per wave, fp32) is scaled into the base-2 domain
//    (scale * log2 e), masked, and folded into the running (max, sum) of each
//    row: lane l holds row (l & 31) and half of its columns, the other half is
//    in lane l ^ 32, so a row reduction is an in-lane reduction plus one
//    exchange.  exp2 is the hardware v_exp_f32;
//  * P goes from the S accumulators straight into MFMA A operands (rounded to
//    T): the accumulator layout gives lane l the key columns {0-3, 8-11} of
//    each 16-key slice (lane l ^ 32 the others), and V's fragments are read in
//    that same key order, so no cross-lane shuffle is needed;
//  * blocks are mapped XCD-aware (each XCD walks whole heads, so a head's K
//    and V stay in one L2) and, under a causal mask, the longest query blocks
//    of a head start first.
// Generic path (fp32, other head dims up to 256, any strides): one wave per
// query row, lanes split D, fp32 throughout.
#include "mfma.h"

namespace ntops {
namespace {

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* mask;
  void* o;
  int64_t qs[4], ks[4], vs[4], ms[4], os[4];
  int B, Hq, Hkv, Sq, Skv, D;
  int mask_dtype;    // -1: none; NTOPS_BOOL (true = attend), NTOPS_F32 / F16 / BF16 (additive)
  int causal;        // 0: none, 1: upper-left (kv <= q), 2: lower-right (kv <= q + Skv - Sq)
  float scale_log2;  // scale * log2(e)
};

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float neg_inf() { return -__builtin_huge_valf(); }

// Additive mask value at element offset `off`, in the base-2 domain.
__device__ __forceinline__ float mask_log2(const AttnArgs& a, int64_t off) {
  switch (a.mask_dtype) {
    case NTOPS_BOOL:
      return static_cast<const bool*>(a.mask)[off] ? 0.f : neg_inf();
    case NTOPS_F32:
      return static_cast<const float*>(a.mask)[off] * kLog2e;
    case NTOPS_F16:
      return static_cast<float>(static_cast<const _Float16*>(a.mask)[off]) * kLog2e;
    default:
      return static_cast<float>(static_cast<const __bf16*>(a.mask)[off]) * kLog2e;
  }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max(a, b, c) in one instruction, without the NaN-quieting moves the
// compiler puts in front of fmaxf in IEEE mode (a NaN operand may be
// dropped; a NaN score still reaches the output through its exponential).
__device__ __forceinline__ float max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Chunk slot of 16-byte chunk c of key row r in the V tile ([kv][d] with
// D / 8 chunks per row), conflict-free for the transposing fragment reads.
template <int D>
__device__ __forceinline__ int vslot(int r, int c) {
  if constexpr (D == 128)
    return mnslot(r, c);
  else
    return c ^ (((r >> 1) & 1) << 2);
}

// B fragment of S = Q K^T: key rows n0 .. n0 + 31 (lane l: row n0 + (l & 31)),
// d = 16 ks + 8 (l >> 5) .. + 7.
template <int D>
__device__ __forceinline__ u32x4 k_frag(const char* tile, int n0, int ks, int lane) {
  const int r = n0 + (lane & 31);
  const int c = ks * 2 + (lane >> 5);
  return *reinterpret_cast<const u32x4*>(tile + r * (D * 2) + kslot<D>(r, c) * 16);
}

// B fragment of O += P V for the 16-key slice sl and output columns
// n0 .. n0 + 31: lane l receives column n0 + (l & 31) at keys
// 16 sl + 4 (l >> 5) + 0..3 (elements 0..3) and 16 sl + 8 + 4 (l >> 5) + 0..3
// (elements 4..7) -- the key order in which the S accumulator holds P.
template <int D>
__device__ __forceinline__ u32x4 v_frag(const char* tile, int n0, int sl, int lane) {
  const int i = lane & 15;
  const int n = n0 + ((lane >> 4) & 1) * 16 + (i & 3) * 4;
  const int c = n >> 3, half = (n >> 2) & 1;
  s16x4 v[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int k = sl * 16 + h * 8 + (lane >> 5) * 4 + (i >> 2);
    const char* p = tile + k * (D * 2) + vslot<D>(k, c) * 16 + half * 8;
    v[h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p));
  }
  u32x4 r;
  r.x = static_cast<uint16_t>(v[0][0]) | (static_cast<uint32_t>(static_cast<uint16_t>(v[0][1])) << 16);
  r.y = static_cast<uint16_t>(v[0][2]) | (static_cast<uint32_t>(static_cast<uint16_t>(v[0][3])) << 16);
  r.z = static_cast<uint16_t>(v[1][0]) | (static_cast<uint32_t>(static_cast<uint16_t>(v[1][1])) << 16);
  r.w = static_cast<uint16_t>(v[1][2]) | (static_cast<uint32_t>(static_cast<uint16_t>(v[1][3])) << 16);
  return r;
}

// Maps a workgroup id to (batch * heads index, query block): XCD-aware
// (workgroups are dispatched round-robin over the 8 XCDs; each XCD gets a
// contiguous range of (batch, head, query block)), longest causal query
// blocks first within a head.
__device__ __forceinline__ void attn_block(int pid, int total, int nqb, int& bh, int& qb) {
  if ((total & 7) == 0) pid = (pid & 7) * (total >> 3) + (pid >> 3);
  bh = pid / nqb;
  qb = nqb - 1 - (pid - bh * nqb);
}

// DMA of one 64 x D K or V tile: D * 2 bytes per key row, 1 KiB per
// instruction, instructions spread evenly over the NW waves.
template <int D, bool IS_V, int NW>
struct KvDma {
  static constexpr int kRowsPerInst = 1024 / (D * 2);
  static constexpr int kInst = 64 / kRowsPerInst / NW;
  static_assert(kInst >= 1 && kInst * NW * kRowsPerInst == 64, "tile must split evenly over the waves");
  u32x4 rsrc;
  uint32_t voff[kInst];
  uint32_t tile_bytes;  // byte distance between consecutive 64-key tiles
  int lds_off;

  // base: element pointer of key row 0; ld: row stride in elements;
  // extent: readable bytes (rows at or past the end read as zero); dt: the
  // head dim of the data (a multiple of 8, at most D): the chunks of columns
  // dt .. D - 1 read as zero (their offset starts at kOOB, and a tile's
  // offset added to it stays below 2^32 and past every extent, since the
  // launch keeps (Skv + 256) * ld * 2 below 2^31).
  __device__ __forceinline__ void init(const void* base, int64_t ld, uint32_t extent, int wave, int lane, int dt) {
    const uint64_t addr = reinterpret_cast<uint64_t>(base);
    rsrc.x = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr));
    rsrc.y = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr >> 32) & 0xffffu);
    rsrc.z = __builtin_amdgcn_readfirstlane(extent);
    rsrc.w = 0x00020000u;
    lds_off = __builtin_amdgcn_readfirstlane(wave * kInst * 1024);
    constexpr int cpr = D / 8;
#pragma unroll
    for (int i = 0; i < kInst; ++i) {
      const int row = (wave * kInst + i) * kRowsPerInst + lane / cpr;
      const int slot = lane % cpr;
      const int c = IS_V ? vslot<D>(row, slot) : kslot<D>(row, slot);  // swizzles are involutions
      voff[i] = c * 8 < dt ? static_cast<uint32_t>(row * ld * 2 + c * 16) : kOOB;
    }
    tile_bytes = static_cast<uint32_t>(64 * ld * 2);
  }

  // Resource of the same operand for another (batch, head): same strides
  // and extent, so the per-lane offsets carry over.
  __device__ __forceinline__ u32x4 rsrc_at(const void* base) const {
    const uint64_t addr = reinterpret_cast<uint64_t>(base);
    u32x4 r = rsrc;
    r.x = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr));
    r.y = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr >> 32) & 0xffffu);
    return r;
  }

  // Loads tile t into LDS at the 32-bit LDS address `tile` through resource
  // r; a tile past the end loads nothing but still counts once per
  // instruction in vmcnt.  Kernels form the address from the LDS base once:
  // a generic -> LDS pointer cast per load instruction carries a null test,
  // 3-4 scalar instructions each.
  __device__ __forceinline__ void issue(u32x4 r, uint32_t tile, int t, bool valid) const {
    // t passes through an empty asm so that the offsets of tiles issued at
    // fixed points (an item's first and last tiles) are computed here, not
    // hoisted out of the item loop to sit in registers for the whole kernel
    asm volatile("" : "+s"(t));
#pragma unroll
    for (int i = 0; i < kInst; ++i) {
      const uint32_t off = valid ? voff[i] + static_cast<uint32_t>(t) * tile_bytes : kOOB;
      dma16(r, tile + static_cast<uint32_t>(lds_off + i * 1024), off);
    }
  }
};

// MM: explicit-mask mode -- 0 none, 1 runs of 4 keys per access (rows
// 4-element aligned), 2 element loads; ESZ: mask element bytes (1 bool, 2
// fp16 / bf16, 4 fp32).  Both are template parameters so that every mask
// load writes fixed registers.
template <typename T, int D, int MM, int ESZ>
__global__ __launch_bounds__(256, 2) void k_flash_fwd(AttnArgs a, int nqb, int total) {
  constexpr int BM = 128, BN = 64;
  constexpr int kFwdAhead = 4;  // fragments read ahead of the MFMA that uses them
  constexpr int KS = D / 16;   // k-steps of S = Q K^T
  constexpr int DT = D / 32;   // 32-column tiles of O
  constexpr int kTile = BN * D * 2;   // bytes of one K or V tile
  constexpr int L = 2 * KvDma<D, false, 4>::kInst;  // DMA instructions per lane per tile
  __shared__ __attribute__((aligned(1024))) char smem[2 * 2 * kTile];  // [stage][K, V]

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int bh, qb;
  if (block_id() >= total) return;  // the tail of a 2-D grid (the whole block)
  attn_block(static_cast<int>(block_id()), total, nqb, bh, qb);
  const int b = bh / a.Hq, h = bh - b * a.Hq;
  const int hk = h / (a.Hq / a.Hkv);
  const int q0 = qb * BM;
  const int qw = q0 + wave * 32;
  const int my_q = qw + (lane & 31);
  const int off = a.causal == 2 ? a.Skv - a.Sq : 0;
  const T* Q = static_cast<const T*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const T* K = static_cast<const T*>(a.k) + b * a.ks[0] + hk * a.ks[1];
  const T* V = static_cast<const T*>(a.v) + b * a.vs[0] + hk * a.vs[1];

  // Q fragments (A operand of S): row my_q, d = 16 ks + 8 (lane >> 5) .. + 7.
  u32x4 qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int d0 = ks * 16 + 8 * (lane >> 5);  // columns past the head dim read as zero
    if (my_q < a.Sq && d0 < a.D)
      qf[ks] = *reinterpret_cast<const u32x4*>(Q + my_q * a.qs[2] + d0);
    else
      qf[ks] = u32x4{0, 0, 0, 0};
  }

  int kv_end = a.Skv;
  if (a.causal) kv_end = max(0, min(a.Skv, q0 + BM + off));
  const int nkv = (kv_end + BN - 1) / BN;

  // Explicit mask (keys contiguous; other layouts take the generic kernel).
  // It enters S as the MFMA accumulator's initial value, mask / scale, so
  // S * scale carries it; its raw data for tile j + 1 is loaded while tile j
  // is softmaxed and multiplied by V (S's registers are free then), through
  // a buffer resource over this (batch, head)'s plane (a row past Sq or a key
  // past the plane reads 0; such keys are masked anyway).  mmode 1: every run
  // of 4 keys of a lane is one access (rows 4-element aligned); 2: element
  // loads.
  constexpr int esz = ESZ;
  constexpr int mmode = MM;
  const char* mp = mmode != 0 ? static_cast<const char*>(a.mask) + (b * a.ms[0] + h * a.ms[1]) * esz
                              : static_cast<const char*>(a.q);
  const int64_t mext =
      mmode != 0 ? (static_cast<int64_t>(a.Sq - 1) * a.ms[2] + static_cast<int64_t>(a.Skv - 1) + 1) * esz : 0;
  const __amdgpu_buffer_rsrc_t rm = buffer_rsrc(mp, static_cast<uint32_t>(mext));
  const int64_t mrow = static_cast<int64_t>(my_q) * a.ms[2];
  const float inv_scale = kLog2e / a.scale_log2;
  // raw mask data, run r (keys kv .. kv + 3 of mask_issue) in mraw[4 r ..]:
  // one word (bool runs), two (16-bit runs), four (fp32 runs or elementwise
  // loads) -- the same slots in every mode, so that the compiler, which
  // merges the branches' stores, never sees a variable index
  uint32_t mraw[32];
  auto mask_issue = [&](int j) {
    const bool row_ok = my_q < a.Sq;
#pragma unroll
    for (int r = 0; r < 8; ++r) {  // run r: keys kv .. kv + 3
      const int kv = j * BN + 32 * (r >> 2) + 8 * (r & 3) + 4 * (lane >> 5);
      const uint32_t o = row_ok && kv < a.Skv ? static_cast<uint32_t>((mrow + kv) * esz) : kOOB;
      if constexpr (mmode == 1) {
        if constexpr (esz == 1) {
          mraw[4 * r] = __builtin_amdgcn_raw_buffer_load_b32(rm, o, 0, 0);
        } else if constexpr (esz == 2) {
          const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rm, o, 0, 0));
          mraw[4 * r] = w.x;
          mraw[4 * r + 1] = w.y;
        } else {
          const u32x4 w = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rm, o, 0, 0));
#pragma unroll
          for (int e = 0; e < 4; ++e) mraw[4 * r + e] = w[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (esz == 1)
            mraw[4 * r + e] = __builtin_amdgcn_raw_buffer_load_b8(rm, o, e, 0);
          else if constexpr (esz == 2)
            mraw[4 * r + e] = __builtin_amdgcn_raw_buffer_load_b16(rm, o, 2 * e, 0);
          else
            mraw[4 * r + e] = __builtin_amdgcn_raw_buffer_load_b32(rm, o, 4 * e, 0);
        }
      }
    }
  };
  // S's initial value: mask / scale (bool: 0 or -inf) for element 4 q + e of half t
  auto mask_init = [&](f32x16 (&sv)[2]) {
#pragma unroll
    for (int r = 0; r < 8; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t w;
        if constexpr (mmode == 1)
          w = esz == 1 ? (mraw[4 * r] >> (8 * e)) : esz == 2 ? (mraw[4 * r + (e >> 1)] >> (16 * (e & 1))) : mraw[4 * r + e];
        else
          w = mraw[4 * r + e];
        float m;
        if constexpr (esz == 1)
          m = (w & 0xffu) ? 0.f : neg_inf();
        else if constexpr (esz == 4)
          m = __builtin_bit_cast(float, w) * inv_scale;
        else if (a.mask_dtype == NTOPS_F16)
          m = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w))) * inv_scale;
        else
          m = static_cast<float>(__builtin_bit_cast(__bf16, static_cast<uint16_t>(w))) * inv_scale;
        sv[r >> 2][4 * (r & 3) + e] = m;
      }
  };

  // K and V tiles go global -> LDS by direct DMA into two stages (keys past
  // the end read as zero, keeping 0 * V finite)
  KvDma<D, false, 4> kd;
  KvDma<D, true, 4> vd;
  kd.init(K, a.ks[2], static_cast<uint32_t>(static_cast<int64_t>(a.Skv) * a.ks[2] * 2), wave, lane, a.D);
  vd.init(V, a.vs[2], static_cast<uint32_t>(static_cast<int64_t>(a.Skv) * a.vs[2] * 2), wave, lane, a.D);
  const uint32_t smem_addr = lds_addr(smem);
  auto dma = [&](int t) {
    const uint32_t st = smem_addr + static_cast<uint32_t>((t & 1) * 2 * kTile);
    kd.issue(kd.rsrc, st, t, true);
    vd.issue(vd.rsrc, st + kTile, t, true);
  };

  f32x16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[t][e] = 0.f;
  float m_i = neg_inf(), l_i = 0.f;  // running max (base 2) and sum of row my_q

  if (nkv > 0) {
    dma(0);
    if constexpr (mmode != 0) mask_issue(0);
  }
  wait_vmcnt<0>();
  __syncthreads();

  for (int j = 0; j < nkv; ++j) {
    const int cur = j & 1;
    const char* sk = smem + cur * 2 * kTile;
    const char* sv = sk + kTile;

    // S = Q K^T (+ mask / scale) for this wave's 32 rows x 64 keys (two
    // 32x32 tiles)
    f32x16 s[2];
    if constexpr (mmode != 0) {
      mask_init(s);
    } else {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) s[t][e] = 0.f;
    }
    // the other stage was last read in the previous iteration, before the
    // barrier that ended it
    if (j + 1 < nkv) dma(j + 1);
    {
      // fragment i + kFwdAhead is read while MFMA i runs (hand-pipelined, one
      // scheduling fence per step)
      constexpr int nm = 2 * KS;  // MFMA i: d slice i / 2, key half i % 2
      u32x4 f[kFwdAhead];
#pragma unroll
      for (int i = 0; i < kFwdAhead; ++i) f[i] = k_frag<D>(sk, (i % 2) * 32, i / 2, lane);
#pragma unroll
      for (int i = 0; i < nm; ++i) {
        __builtin_amdgcn_sched_barrier(0);
        s[i % 2] = mfma32<T>(f[i % kFwdAhead], qf[i / 2], s[i % 2]);
        if (i + kFwdAhead < nm) f[i % kFwdAhead] = k_frag<D>(sk, ((i + kFwdAhead) % 2) * 32, (i + kFwdAhead) / 2, lane);
      }
      __builtin_amdgcn_sched_barrier(0);
    }

    // base-2 scores with masking; element 4q + e of tile t is key
    // kv0 + 32 t + 8 q + 4 (lane >> 5) + e
    const int kv0 = j * BN;
    const bool full = kv0 + BN <= a.Skv && a.mask_dtype < 0 &&
                      (a.causal == 0 || kv0 + BN - 1 <= qw + off);
    float x[2][16];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) x[t][e] = s[t][e] * a.scale_log2;
    if constexpr (mmode != 0)
      if (j + 1 < nkv) mask_issue(j + 1);
    if (!full) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int kv = kv0 + 32 * t + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
          bool ok = kv < a.Skv && my_q < a.Sq;
          if (a.causal) ok = ok && kv <= my_q + off;
          x[t][e] = ok ? x[t][e] : neg_inf();
        }
    }

    // online softmax of row my_q (lanes l and l ^ 32 hold its two halves)
    float mx = neg_inf();
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, x[t][e]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_i, mx);
    const float m_use = m_new == neg_inf() ? 0.f : m_new;  // fully masked so far: keep P = 0
    const float alpha = fast_exp2(m_i - m_use);
    float rs = 0.f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        x[t][e] = fast_exp2(x[t][e] - m_use);
        rs += x[t][e];
      }
    rs += __shfl_xor(rs, 32, 64);
    l_i = l_i * alpha + rs;
    m_i = m_new;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[t][e] *= alpha;

    // O += P V over the four 16-key slices, hand-pipelined as S above
    {
      u32x4 pf[4];
#pragma unroll
      for (int sl = 0; sl < 4; ++sl) pf[sl] = pack8<T>(&x[sl >> 1][8 * (sl & 1)]);
      constexpr int nm = 4 * DT;  // MFMA i: key slice i / DT, d tile i % DT
      u32x4 f[kFwdAhead];
#pragma unroll
      for (int i = 0; i < kFwdAhead; ++i) f[i] = v_frag<D>(sv, (i % DT) * 32, i / DT, lane);
#pragma unroll
      for (int i = 0; i < nm; ++i) {
        __builtin_amdgcn_sched_barrier(0);
        o[i % DT] = mfma32<T>(f[i % kFwdAhead], pf[i / DT], o[i % DT]);
        if (i + kFwdAhead < nm)
          f[i % kFwdAhead] = v_frag<D>(sv, ((i + kFwdAhead) % DT) * 32, (i + kFwdAhead) / DT, lane);
      }
      __builtin_amdgcn_sched_barrier(0);
    }

    // tile j + 1 landed (the next tile's mask loads, issued after it, may
    // still be in flight)
    if (j + 1 < nkv) {
      if constexpr (mmode == 1)
        wait_vmcnt<8>();
      else if constexpr (mmode == 2)
        wait_vmcnt<32>();
      else
        wait_vmcnt<0>();
    }
    __syncthreads();
  }

  if (my_q >= a.Sq) return;
  const float inv = l_i > 0.f ? 1.f / l_i : 0.f;
  T* O = static_cast<T*>(a.o) + b * a.os[0] + h * a.os[1] + static_cast<int64_t>(my_q) * a.os[2];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      T v4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v4[e] = static_cast<T>(o[t][4 * qq + e] * inv);
      const int col = t * 32 + 8 * qq + 4 * (lane >> 5);
      if (col < a.D)  // a.D % 8 == 0: the 4 columns are all in or all out
        *reinterpret_cast<u32x2*>(O + col) = __builtin_bit_cast(u32x2, v4);
    }
}

// ---- flash forward without an explicit mask (none or causal) ---------------
//
// Persistent 8-wave workgroups (one per CU) over work items of (batch, head,
// 256 query rows); wave w owns rows 32w .. 32w + 31 of the item with their
// Q fragments in VGPRs.
// K and V tiles of 64 keys go global -> LDS by direct DMA (no VGPR staging)
// into a ring of kFaStages stages, with the swizzles of k_frag / v_frag
// applied on the global side (a lane's LDS destination is fixed, so it
// fetches the chunk that belongs there).  The two waves sharing a SIMD run
// half a tile apart: while one runs a matrix phase (O += P_j V_j, then
// S_{j+1} = Q K_{j+1}^T) the other runs a vector phase (mask, max, exp2,
// sum, pack P), two barriers per tile (see the loops in k_flash_attn).
// Lazy rescaling: exponentials use a running reference max m that is raised
// only when a row's max exceeds it by more than 2^8 (then O and l are scaled
// by exp2(m_old - m_new) once); P <= 256 keeps fp32 sums and the T-rounded P
// exact in relative terms, and O / l is unchanged by the choice of m.
// Causal: the block walks keys up to its last row's limit; a wave skips the
// tiles beyond its own rows' limit (it still issues its share of the DMA and
// joins the barriers).
constexpr int kFaRows = 256;
constexpr int kFaWaves = 8;
constexpr int kFaStages = 4;
constexpr int kPrefetch = 4;  // fragments read ahead of the MFMA that uses them

// Work item of this workgroup in round r (false: no more items).
// Workgroups are dispatched round-robin over the 8 XCDs, so workgroup g runs
// on XCD g % 8; with a grid that is a multiple of 8, XCD x owns the heads
// bh = x, x + 8, ...  Its workgroups process those heads in groups of HG
// heads whose HG * nqb query blocks roughly fill them (so a head's K / V is
// read into the XCD's L2 once per group); within a group, items go longest
// query block first (more keys under a causal mask), and the slot order is
// reversed every other round so that long and short items pair up.
__device__ __forceinline__ bool fa_item(int r, int nbh, int nqb, int& bh, int& qb) {
  const int grid = static_cast<int>(gridDim.x);
  const int nx = (grid % 8 == 0) ? 8 : 1;
  const int x = static_cast<int>(blockIdx.x) % nx;
  const int gl = grid / nx;                      // workgroups on this XCD
  const int lb = static_cast<int>(blockIdx.x) / nx;
  const int hx = nbh > x ? (nbh - x + nx - 1) / nx : 0;  // heads of this XCD
  const int li = r * gl + ((r & 1) ? gl - 1 - lb : lb);
  if (li >= hx * nqb) return false;
  const int hg = max(1, gl / nqb);              // heads per group
  const int g = li / (hg * nqb);
  const int hg_g = min(hg, hx - g * hg);         // the last group may be smaller
  const int pos = li - g * hg * nqb;
  const int rank = pos / hg_g;
  const int hl = g * hg + (pos - rank * hg_g);
  bh = hl * nx + x;
  qb = nqb - 1 - rank;
  return true;
}

// TAIL: the head dim a.D is below D (columns a.D .. D - 1 masked); compiled
// apart so the D-wide kernels carry no column tests.
template <typename T, int D, bool CAUSAL, bool TAIL>
__global__ __launch_bounds__(512, 1) void k_flash_attn(AttnArgs a, int nqb) {
  constexpr int BN = 64;
  constexpr int NS = kFaStages;
  constexpr int NW = kFaWaves;
  constexpr int KS = D / 16;
  constexpr int DT = D / 32;
  constexpr int kTile = BN * D * 2;
  constexpr int kStage = 2 * kTile;                  // K tile, then V tile
  constexpr int L = 2 * KvDma<D, false, NW>::kInst;  // DMA instructions per lane per tile
  static_assert(NS == 4, "the phase schedule refills the stage of tile k - 2 with tile k + 2");
  extern __shared__ __attribute__((aligned(1024))) char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2;  // 0: leads, 1: one phase behind (one wave of each per SIMD)
  // Consecutive items of a workgroup are chained: the LDS ring keeps
  // rotating (item i's tile t lives in stage (base_i + t) mod 4, base_{i+1} =
  // base_i + nkv_i), the K / V loads of the next item's first two tiles take
  // the slots of item i's last two periods (the slots a lone item fills with
  // empty loads), and its Q fragments are loaded at the start of item i's
  // last period, when every wave has computed its last S.  So an item
  // starts with its first tiles and Q on chip instead of paying two memory
  // round trips.  Between those tiles and the item's first period the
  // wave's vector-memory queue then also holds the Q loads and the previous
  // item's O stores (kHandoff of them), which the first two waits allow for.
  constexpr int kHandoff = KS + 4 * DT;
  u32x4 qf[KS];             // Q fragments (A operand of S): row my_q, d = 16 ks + 8 (lane >> 5) .. + 7
  int base = 0;             // stage of the current item's tile 0
  const int off = (CAUSAL && a.causal == 2) ? a.Skv - a.Sq : 0;
  // key tiles of query block qb
  auto tiles_of = [&](int qb) {
    int kv_end = a.Skv;
    if (CAUSAL) kv_end = max(0, min(a.Skv, qb * kFaRows + kFaRows + off));
    return (kv_end + BN - 1) / BN;
  };
  // Q rows of item (bh, qb) into qf (buffer loads: rows past Sq read as zero)
  auto load_q = [&](int bh, int qb) {
    const int b = bh / a.Hq, h = bh - b * a.Hq;
    const T* Q = static_cast<const T*>(a.q) + b * a.qs[0] + h * a.qs[1];
    const __amdgpu_buffer_rsrc_t rq =
        buffer_rsrc(Q, static_cast<uint32_t>(static_cast<int64_t>(a.Sq) * a.qs[2] * 2));
    const uint32_t row = static_cast<uint32_t>((qb * kFaRows + wave * 32 + (lane & 31)) * a.qs[2] * 2);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d0 = ks * 16 + 8 * (lane >> 5);  // columns past the head dim read as zero
      qf[ks] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             rq, !TAIL || d0 < a.D ? row + d0 * 2 : kOOB, 0, 0));
    }
  };
  // K / V of (batch * head) bh
  auto k_base = [&](int bh) {
    const int b = bh / a.Hq, h = bh - b * a.Hq;
    return static_cast<const T*>(a.k) + b * a.ks[0] + (h / (a.Hq / a.Hkv)) * a.ks[1];
  };
  auto v_base = [&](int bh) {
    const int b = bh / a.Hq, h = bh - b * a.Hq;
    return static_cast<const T*>(a.v) + b * a.vs[0] + (h / (a.Hq / a.Hkv)) * a.vs[1];
  };
  KvDma<D, false, NW> kd;
  KvDma<D, true, NW> vd;
  kd.init(k_base(0), a.ks[2], static_cast<uint32_t>(static_cast<int64_t>(a.Skv) * a.ks[2] * 2), wave, lane, a.D);
  vd.init(v_base(0), a.vs[2], static_cast<uint32_t>(static_cast<int64_t>(a.Skv) * a.vs[2] * 2), wave, lane, a.D);
  // Work item (batch * head, query block) of a persistent workgroup (one
  // per CU) walking the items fa_item picks, so that a head's query blocks
  // run together on one XCD (its K and V stay in that L2) and per-workgroup
  // work evens out under a causal mask.  nbh < 0: no next item.  CHAINED (a std::bool_constant): the item's
  // first tiles and Q were issued by the previous item.
  auto item = [&](auto chained_tag, int bh, int qb, int nbh, int nqbi) {
  constexpr bool chained = decltype(chained_tag)::value;
  const int b = bh / a.Hq, h = bh - b * a.Hq;
  const int q0 = qb * kFaRows;
  const int qw = q0 + wave * 32;
  const int my_q = qw + (lane & 31);
  const float c = a.scale_log2;  // > 0 on this path
  const int nkv = tiles_of(qb);
  const bool has_next = nbh >= 0;
  const int nkv_next = has_next ? tiles_of(nqbi) : 0;
  // last tile this wave needs (-1: none)
  int jl = nkv - 1;
  if (CAUSAL) {
    const int last = qw + 31 + off;
    jl = min(jl, last >= 0 ? last / BN : -1);
  }
  if (qw >= a.Sq) jl = -1;
  // last key of row my_q, relative to a tile's first key and this lane's
  // column group: element (u, e) of a tile is key 32 u + 8 (e >> 2) + (e & 3)
  // past that origin
  int lim = a.Skv - 1;
  if (CAUSAL) lim = min(lim, my_q + off);
  lim -= 4 * (lane >> 5);

  const u32x4 rk = kd.rsrc_at(k_base(bh)), rv = vd.rsrc_at(v_base(bh));
  const u32x4 rkn = kd.rsrc_at(k_base(has_next ? nbh : bh)), rvn = vd.rsrc_at(v_base(has_next ? nbh : bh));
  // Slot g of the load stream: this item's tile g, then the next item's
  // tiles 0 and 1 (empty loads when there is no next item, so that every
  // period issues L instructions until the last one), then nothing.
  const uint32_t smem_addr = lds_addr(smem);
  auto dma = [&](int g) {
    const uint32_t st = smem_addr + static_cast<uint32_t>(((base + g) & 3) * kStage);
    if (g < nkv) {
      kd.issue(rk, st, g, true);
      vd.issue(rv, st + kTile, g, true);
    } else if (!has_next) {
      kd.issue(rk, st, 0, false);
      vd.issue(rv, st + kTile, 0, false);
    } else if (g - nkv < 2) {
      kd.issue(rkn, st, g - nkv, g - nkv < nkv_next);
      vd.issue(rvn, st + kTile, g - nkv, g - nkv < nkv_next);
    }
  };
  if constexpr (!chained) {
    load_q(bh, qb);
    dma(0);
    dma(1);
  }
  // The S products read qf: settle its loads here, once per item, rather
  // than let the compiler wait for them (and so for every memory operation
  // in flight) inside the tile loop.  First items are compiled apart from
  // chained ones so that for the latter the compiler sees what the wave's
  // queue holds -- Q loads older than the previous item's O stores only --
  // and waits for Q alone.
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) asm volatile("" ::"v"(qf[ks]));

  f32x16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[t][e] = 0.f;
  float m_run = neg_inf();  // reference max (base 2) of row my_q
  float l_half = 0.f;       // this lane's half of the row's sum of exponentials
  f32x16 s[2];              // S of the tile being softmaxed
  u32x4 pf[4];              // P of that tile, as MFMA A operands per 16-key slice

  // matrix phase of tile j: O += P_j V_j (if j >= 0) and S = Q K_{j+1}^T
  // (if j + 1 <= jl).  Software-pipelined by hand: fragment i + kPrefetch is
  // read while MFMA i runs, and a scheduling fence per step pins that order
  // (left to the scheduler, the phase was compiled with one fragment register
  // set and an LDS round trip before every MFMA).
  auto pv_part = [&](int j) {
    {
      const char* sv = smem + ((base + j) & 3) * kStage + kTile;
      constexpr int nm = 4 * DT;  // MFMA i: key slice i / DT, d tile i % DT
      u32x4 f[kPrefetch];
#pragma unroll
      for (int i = 0; i < kPrefetch; ++i) f[i] = v_frag<D>(sv, (i % DT) * 32, i / DT, lane);
#pragma unroll
      for (int i = 0; i < nm; ++i) {
        __builtin_amdgcn_sched_barrier(0);
        o[i % DT] = mfma32<T>(f[i % kPrefetch], pf[i / DT], o[i % DT]);
        if (i + kPrefetch < nm)
          f[i % kPrefetch] = v_frag<D>(sv, ((i + kPrefetch) % DT) * 32, (i + kPrefetch) / DT, lane);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto qk_part = [&](int j) {
    {
      const char* sk = smem + ((base + j + 1) & 3) * kStage;
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int e = 0; e < 16; ++e) s[u][e] = 0.f;
      constexpr int nm = 2 * KS;  // MFMA i: d slice i / 2, key half i % 2
      u32x4 f[kPrefetch];
#pragma unroll
      for (int i = 0; i < kPrefetch; ++i) f[i] = k_frag<D>(sk, (i % 2) * 32, i / 2, lane);
#pragma unroll
      for (int i = 0; i < nm; ++i) {
        __builtin_amdgcn_sched_barrier(0);
        s[i % 2] = mfma32<T>(f[i % kPrefetch], qf[i / 2], s[i % 2]);
        if (i + kPrefetch < nm) f[i % kPrefetch] = k_frag<D>(sk, ((i + kPrefetch) % 2) * 32, (i + kPrefetch) / 2, lane);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // The matrix phase runs at raised wave priority, so the SIMD's arbiter
  // issues it ahead of the partner wave's vector phase (+2 % causal).
  auto matrix_phase = [&](int j) {
    __builtin_amdgcn_s_setprio(1);
    if (j >= 0) pv_part(j);
    if (j + 1 <= jl) qk_part(j);
    __builtin_amdgcn_s_setprio(0);
  };
  // vector phase of tile t: mask (on tiles that reach the end of the keys or
  // cross the wave's diagonal); a raise of the reference max of the rows
  // whose tile max exceeds it by more than 2^8 (rescaling O and l) -- each
  // lane tests its own half of the row, so the exchange with the other half
  // (lane l ^ 32) happens only when some row needs the raise; then
  // P = exp2(S c - m) rounded to T (masked: 0; nothing unmasked yet: m = 0).
  // Reductions are trees so the phase is not one long dependency chain.
  auto vector_phase = [&](int t) {
    const int kv0 = t * BN;
    bool edge = kv0 + BN > a.Skv;
    if (CAUSAL) edge = edge || kv0 + BN - 1 > qw + off;
    if (edge) {
      const int rel = lim - kv0;
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int e = 0; e < 16; ++e) s[u][e] = 32 * u + 8 * (e >> 2) + (e & 3) <= rel ? s[u][e] : neg_inf();
    }
    // max of this lane's half of the row: 16 three-way maxima in a tree
    float mh;
    {
      float v[32];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int e = 0; e < 16; ++e) v[16 * u + e] = s[u][e];
      float m1[11];
#pragma unroll
      for (int i = 0; i < 10; ++i) m1[i] = max3(v[3 * i], v[3 * i + 1], v[3 * i + 2]);
      m1[10] = max3(v[30], v[31], v[31]);
      const float m2a = max3(m1[0], m1[1], m1[2]), m2b = max3(m1[3], m1[4], m1[5]);
      const float m2c = max3(m1[6], m1[7], m1[8]), m2d = max3(m1[9], m1[10], m1[10]);
      mh = max3(m2a, m2b, max3(m2c, m2d, m2d));
    }
    const float th = mh * c;  // max of this lane's half of the row (base 2)
    if (__any(th > m_run + 8.f)) {
      const float tmax = fmaxf(th, __shfl_xor(th, 32, 64));
      const bool up = tmax > m_run + 8.f;
      const float alpha = up ? fast_exp2(m_run - tmax) : 1.f;
      m_run = up ? tmax : m_run;
      l_half *= alpha;
#pragma unroll
      for (int t2 = 0; t2 < DT; ++t2)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[t2][e] *= alpha;
    }
    const float mb = m_run == neg_inf() ? 0.f : m_run;
    float x[2][16];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int e = 0; e < 16; ++e) x[u][e] = fast_exp2(fmaf(s[u][e], c, -mb));
    float r[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) r[e] = x[0][e] + x[1][e];
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
      for (int e = 0; e < w; ++e) r[e] += r[e + w];
    l_half += r[0];
#pragma unroll
    for (int sl = 0; sl < 4; ++sl) pf[sl] = pack8<T>(&x[sl >> 1][8 * (sl & 1)]);
  };

  // Each tile period k has two phases separated by barriers.  Group 0 runs
  // the matrix phase of tile k - 1 then the vector phase of tile k; group 1
  // runs the vector phase of tile k - 1 then the matrix phase of tile k - 1,
  // so the two waves sharing a SIMD are always in opposite kinds of phase.
  // Tile k is read from the first phase of period k to the second phase of
  // period k + 1; at the start of period k it must have landed, and the
  // stage of tile k - 2 is free for tile k + 2.  Each group has a loop of its
  // own so that S and P are never both live across an iteration.
  auto period_start = [&](int k) {
    // this wave's DMA of tile k landed (tile k + 1 may be in flight, and in a
    // chained item's first two periods the Q loads and previous O stores)
    if (chained && k < 2)
      wait_vmcnt<L + kHandoff>();
    else
      wait_vmcnt<L>();
    block_barrier();
    dma(k + 2);
  };
  if (grp == 0) {
    for (int k = 0; k < nkv; ++k) {
      period_start(k);
      if (k - 1 <= jl) matrix_phase(k - 1);
      block_barrier();
      if (k <= jl) vector_phase(k);
    }
  } else {
    for (int k = 0; k < nkv; ++k) {
      period_start(k);
      if (k >= 1 && k - 1 <= jl) vector_phase(k - 1);
      block_barrier();
      if (k - 1 <= jl) matrix_phase(k - 1);
    }
  }
  // last period (k = nkv): only P V of the last tile is left, so Q is dead
  // and the next item's Q loads go out first (peeled out of the loops so the
  // compiler never sees them pending at an S product inside a loop)
  period_start(nkv);
  if (has_next) load_q(nbh, nqbi);
  const bool last_pv = nkv - 1 <= jl && nkv >= 1;
  if (grp == 0) {
    if (last_pv) pv_part(nkv - 1);
    block_barrier();
  } else {
    if (last_pv) vector_phase(nkv - 1);
    block_barrier();
    if (last_pv) pv_part(nkv - 1);
  }
  const float l = l_half + __shfl_xor(l_half, 32, 64);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  // O rows via buffer stores: rows past Sq are dropped, and every lane
  // issues exactly 4 DT stores (the count the next item's waits rely on)
  T* O = static_cast<T*>(a.o) + b * a.os[0] + h * a.os[1];
  const __amdgpu_buffer_rsrc_t ro = buffer_rsrc(O, static_cast<uint32_t>(static_cast<int64_t>(a.Sq) * a.os[2] * 2));
  const uint32_t orow = static_cast<uint32_t>(my_q * a.os[2] * 2);
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      T v4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v4[e] = static_cast<T>(o[t][4 * qq + e] * inv);
      const int col = t * 32 + 8 * qq + 4 * (lane >> 5);  // columns past the head dim: dropped
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v4), ro,
                                            !TAIL || col < a.D ? orow + col * 2 : kOOB, 0, 0);
    }
  base = (base + nkv) & 3;
  };  // item
  int bh, qb, nbh, nqbi;
  if (fa_item(0, a.B * a.Hq, nqb, bh, qb)) {
    bool more = fa_item(1, a.B * a.Hq, nqb, nbh, nqbi);
    item(std::false_type{}, bh, qb, more ? nbh : -1, more ? nqbi : 0);
    for (int round = 1; more; ++round) {
      bh = nbh;
      qb = nqbi;
      more = fa_item(round + 1, a.B * a.Hq, nqb, nbh, nqbi);
      item(std::true_type{}, bh, qb, more ? nbh : -1, more ? nqbi : 0);
    }
  }
  wait_vmcnt<0>();  // no DMA may land after the workgroup ends
}

// Generic path: one wave per (batch, head, query row); lane owns d = lane +
// 64 u.  fp32 arithmetic throughout (accurate exp2).
template <typename T>
__global__ __launch_bounds__(64) void k_attn_generic(AttnArgs a) {
  const int lane = threadIdx.x;
  const int64_t row = block_id();  // (b, h, q) linear; blocks_2d grid
  if (row >= static_cast<int64_t>(a.B) * a.Hq * a.Sq) return;  // the tail of the grid (the whole block)
  const int q = static_cast<int>(row % a.Sq);
  const int64_t bh = row / a.Sq;
  const int h = static_cast<int>(bh % a.Hq);
  const int b = static_cast<int>(bh / a.Hq);
  const int hk = h / (a.Hq / a.Hkv);
  const T* Q = static_cast<const T*>(a.q) + b * a.qs[0] + h * a.qs[1] + q * a.qs[2];
  const T* K = static_cast<const T*>(a.k) + b * a.ks[0] + hk * a.ks[1];
  const T* V = static_cast<const T*>(a.v) + b * a.vs[0] + hk * a.vs[1];
  float qv[4], acc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int d = lane + 64 * u;
    qv[u] = d < a.D ? static_cast<float>(Q[d * a.qs[3]]) * a.scale_log2 : 0.f;
    acc[u] = 0.f;
  }
  const int off = a.causal == 2 ? a.Skv - a.Sq : 0;
  int kv_end = a.Skv;
  if (a.causal) kv_end = max(0, min(a.Skv, q + off + 1));
  const int64_t mrow = b * a.ms[0] + h * a.ms[1] + static_cast<int64_t>(q) * a.ms[2];
  float m = neg_inf(), l = 0.f;
  for (int kv = 0; kv < kv_end; ++kv) {
    float s = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int d = lane + 64 * u;
      if (d < a.D) s += qv[u] * static_cast<float>(K[kv * a.ks[2] + d * a.ks[3]]);
    }
    s = wave_sum(s);
    if (a.mask_dtype >= 0) s += mask_log2(a, mrow + kv * a.ms[3]);
    if (s == neg_inf()) continue;  // wave-uniform
    const float m_new = fmaxf(m, s);
    const float alpha = exp2f(m - m_new);
    const float p = exp2f(s - m_new);
    l = l * alpha + p;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int d = lane + 64 * u;
      const float vv = d < a.D ? static_cast<float>(V[kv * a.vs[2] + d * a.vs[3]]) : 0.f;
      acc[u] = acc[u] * alpha + p * vv;
    }
    m = m_new;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  T* O = static_cast<T*>(a.o) + b * a.os[0] + h * a.os[1] + q * a.os[2];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int d = lane + 64 * u;
    if (d < a.D) O[d * a.os[3]] = static_cast<T>(acc[u] * inv);
  }
}

// ---- fp32 attention on the matrix cores --------------------------------------
// IEEE fp32 products (v_mfma_f32_16x16x4_f32) with fp32 accumulation and the
// online-softmax recurrence in fp32.  Work item: (batch, head, 128 query
// rows), 8 waves of 16 rows.  The scores are computed transposed,
// S^T = K Q^T (keys x queries): lane l's accumulator r holds key
// 4 (l >> 4) + r of a 16-key block for query l & 15.  That is the B operand
// of O^T += V^T P^T for MFMA step r when the keys of step r are taken as
// 4 (l >> 4) + r (a sum over keys does not depend on their order), so P
// never leaves the registers; and every accumulator of a lane belongs to
// one query, so the rescale of O is per lane while the row max and sum
// combine the four lanes l & 15 + 16 g.  The head dim is walked as
// d = 16 t + 4 g + e (g = l >> 4, e = MFMA step of a 4-step group) in both
// products, so a lane reads 4 consecutive floats per 4 MFMAs.  K (32 keys x
// DP) and V^T (DP x 32 keys) tiles are double-buffered in LDS, each tile's
// global loads issued into registers before the previous tile's products
// and stored after them (one barrier per tile).  Keys past Skv, past the
// causal bound, and head-dim columns past D read as zero / are masked.
constexpr int kF32K = 32;  // keys per tile

template <int DP>
constexpr int f32_attn_lds_bytes() {
  return 2 * (kF32K * (DP + 4) + DP * (kF32K + 4)) * 4;
}

// NW waves, each with RG blocks of 16 query rows (the K and V fragments read
// from LDS serve all RG of them).
template <int DP, int NW, int RG>
__global__ __launch_bounds__(64 * NW) void k_flash_f32(AttnArgs a, int nqb) {
  constexpr int QB = 16 * NW * RG;  // query rows per block
  constexpr int KP = DP + 4;        // floats per K row in LDS
  constexpr int VP = kF32K + 4;     // floats per V^T row in LDS
  constexpr int kKTile = kF32K * KP, kBuf = kKTile + DP * VP;
  constexpr int kThreads = 64 * NW;
  constexpr int kF4 = kF32K * DP / 4;                   // float4 per operand and tile
  constexpr int kLd = (kF4 + kThreads - 1) / kThreads;  // per thread
  static_assert(kF4 % kThreads == 0 || kThreads % kF4 == 0, "tile must split evenly over the block");
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int64_t item = block_id();  // (batch, head, query block); blocks_2d grid
  const int64_t nbh = static_cast<int64_t>(a.B) * a.Hq;
  if (item >= nbh * nqb) return;  // the tail of the grid (the whole block)
  // causal: longest query blocks first over the whole grid (the blocks run
  // 4 .. S / 32 key tiles; dealing them longest first keeps the last
  // round from being one long block); otherwise the query blocks of a head
  // run together
  int qb;
  int64_t bh;
  if (a.causal) {
    qb = nqb - 1 - static_cast<int>(item / nbh);
    bh = item % nbh;
  } else {
    qb = static_cast<int>(item % nqb);
    bh = item / nqb;
  }
  const int h = static_cast<int>(bh % a.Hq);
  const int b = static_cast<int>(bh / a.Hq);
  const int hk = h / (a.Hq / a.Hkv);
  const float* Q = static_cast<const float*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const float* K = static_cast<const float*>(a.k) + b * a.ks[0] + hk * a.ks[1];
  const float* V = static_cast<const float*>(a.v) + b * a.vs[0] + hk * a.vs[1];
  const int q_wave = qb * QB + wave * 16 * RG;  // this wave's first query
  const int dt = a.D;
  int qrow[RG];
  f32x4 qf[RG][DP / 16];
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) {
    qrow[rg] = q_wave + 16 * rg + r16;
#pragma unroll
    for (int t = 0; t < DP / 16; ++t) {
      const int d = 16 * t + 4 * g;
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (qrow[rg] < a.Sq && d < dt) v = *reinterpret_cast<const f32x4*>(Q + qrow[rg] * a.qs[2] + d);
      qf[rg][t] = v * a.scale_log2;
    }
  }
  const int off = a.causal == 2 ? a.Skv - a.Sq : 0;
  int kv_end = a.Skv;
  if (a.causal) kv_end = max(0, min(a.Skv, qb * QB + QB - 1 + off + 1));
  const int ntiles = (kv_end + kF32K - 1) / kF32K;
  f32x4 kst[kLd], vst[kLd];
  auto load_tile = [&](int t) {
#pragma unroll
    for (int j = 0; j < kLd; ++j) {
      const int f = threadIdx.x + kThreads * j;
      const int key = t * kF32K + f / (DP / 4), d = 4 * (f % (DP / 4));
      const bool ok = f < kF4 && key < kv_end && d < dt;
      f32x4 kz = {0.f, 0.f, 0.f, 0.f}, vz = {0.f, 0.f, 0.f, 0.f};
      if (ok) {
        kz = *reinterpret_cast<const f32x4*>(K + key * a.ks[2] + d);
        vz = *reinterpret_cast<const f32x4*>(V + key * a.vs[2] + d);
      }
      kst[j] = kz;
      vst[j] = vz;
    }
  };
  auto store_tile = [&](int buf) {
    float* kt = sm + buf * kBuf;
    float* vt = kt + kKTile;
#pragma unroll
    for (int j = 0; j < kLd; ++j) {
      const int f = threadIdx.x + kThreads * j;
      if (f >= kF4) break;
      const int kl = f / (DP / 4), d = 4 * (f % (DP / 4));
      *reinterpret_cast<f32x4*>(kt + kl * KP + d) = kst[j];
#pragma unroll
      for (int e = 0; e < 4; ++e) vt[(d + e) * VP + kl] = vst[j][e];
    }
  };
  int64_t mrow[RG];
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) mrow[rg] = b * a.ms[0] + h * a.ms[1] + static_cast<int64_t>(qrow[rg]) * a.ms[2];
  f32x4 o[RG][DP / 16];
  float m[RG], l[RG];
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) {
    m[rg] = neg_inf();
    l[rg] = 0.f;
#pragma unroll
    for (int i = 0; i < DP / 16; ++i) o[rg][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  if (ntiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();
  // the last key this wave's rows attend to (causal): tiles past it are
  // loaded and stored for the block but not computed
  const int wave_end = a.causal ? min(kv_end, q_wave + 16 * RG - 1 + off + 1) : kv_end;
  for (int t = 0; t < ntiles; ++t) {
    if (t + 1 < ntiles) load_tile(t + 1);
    const float* kt = sm + (t & 1) * kBuf;
    const float* vt = kt + kKTile;
    if (t * kF32K < wave_end) {  // wave-uniform
      f32x4 sc[RG][2];
#pragma unroll
      for (int rg = 0; rg < RG; ++rg)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) sc[rg][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int tt = 0; tt < DP / 16; ++tt)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const f32x4 kf = *reinterpret_cast<const f32x4*>(kt + (kb * 16 + r16) * KP + 16 * tt + 4 * g);
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int rg = 0; rg < RG; ++rg)
              sc[rg][kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[e], qf[rg][tt][e], sc[rg][kb], 0, 0, 0);
        }
      // mask, then the online softmax of each of this lane's queries
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) {
        float mx = neg_inf();
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = t * kF32K + kb * 16 + 4 * g + r;
            float v = sc[rg][kb][r];
            if (a.mask_dtype >= 0 && key < a.Skv && qrow[rg] < a.Sq) v += mask_log2(a, mrow[rg] + key * a.ms[3]);
            if (key >= a.Skv || (a.causal && key > qrow[rg] + off)) v = neg_inf();
            sc[rg][kb][r] = v;
            mx = fmaxf(mx, v);
          }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m[rg], mx);
        const float m_use = m_new == neg_inf() ? 0.f : m_new;
        const float alpha = fast_exp2(m[rg] - m_use);
        float ps = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float p = fast_exp2(sc[rg][kb][r] - m_use);
            sc[rg][kb][r] = p;
            ps += p;
          }
        ps += __shfl_xor(ps, 16, 64);
        ps += __shfl_xor(ps, 32, 64);
        l[rg] = l[rg] * alpha + ps;
        m[rg] = m_new;
#pragma unroll
        for (int i = 0; i < DP / 16; ++i) o[rg][i] *= alpha;
      }
#pragma unroll
      for (int i = 0; i < DP / 16; ++i)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const f32x4 vf = *reinterpret_cast<const f32x4*>(vt + (16 * i + r16) * VP + kb * 16 + 4 * g);
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int rg = 0; rg < RG; ++rg)
              o[rg][i] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[e], sc[rg][kb][e], o[rg][i], 0, 0, 0);
        }
    }
    if (t + 1 < ntiles) store_tile((t + 1) & 1);  // read last in tile t - 1, before the barrier that ended it
    __syncthreads();
  }
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) {
    if (qrow[rg] >= a.Sq) continue;
    const float inv = l[rg] > 0.f ? 1.f / l[rg] : 0.f;  // fully masked rows give 0
    float* O = static_cast<float*>(a.o) + b * a.os[0] + h * a.os[1] + static_cast<int64_t>(qrow[rg]) * a.os[2];
#pragma unroll
    for (int i = 0; i < DP / 16; ++i) {
      const int d = 16 * i + 4 * g;
      if (d < dt) *reinterpret_cast<f32x4*>(O + d) = o[rg][i] * inv;
    }
  }
}

template <int DP, int NW, int RG>
int launch_flash_f32(const AttnArgs& a, hipStream_t st) {
  constexpr int kLds = f32_attn_lds_bytes<DP>();
  auto kern = k_flash_f32<DP, NW, RG>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, kLds) !=
        hipSuccess)
      return set_error(NTOPS_ERR_HIP, "sdpa: cannot reserve %d bytes of LDS", kLds);
    attr_set = true;
  }
  constexpr int QB = 16 * NW * RG;
  const int nqb = (a.Sq + QB - 1) / QB;
  const int64_t total = static_cast<int64_t>(nqb) * a.Hq * a.B;
  if (total > 0x7fffffffLL) return set_error(NTOPS_ERR_UNSUPPORTED, "sdpa: too many blocks");
  note_kernel("sdpa_f32 d%d", DP);
  hipLaunchKernelGGL(kern, blocks_2d(total), dim3(64 * NW), kLds, st, a, nqb);
  return check_launch("sdpa");
}

template <typename T, int D, bool CAUSAL, bool TAIL>
int launch_flash_attn(const AttnArgs& a, hipStream_t st) {
  constexpr int kLds = kFaStages * 2 * 64 * D * 2;
  auto kern = k_flash_attn<T, D, CAUSAL, TAIL>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            kLds) != hipSuccess)
      return set_error(NTOPS_ERR_HIP, "sdpa: cannot reserve %d bytes of LDS", kLds);
    attr_set = true;
  }
  const int nqb = (a.Sq + kFaRows - 1) / kFaRows;
  const int64_t total = static_cast<int64_t>(nqb) * a.Hq * a.B;
  if (total > 0x3fffffffLL) return set_error(NTOPS_ERR_UNSUPPORTED, "sdpa: too many work items");
  // persistent: one workgroup per CU (each takes 128 KiB of LDS), chained
  // items of equal or unequal length (same-box A/B, non-causal
  // (4, 32, 2048, 128): 903 against 865 TFLOP/s for one workgroup per item)
  const int64_t grid = std::min<int64_t>(total, cu_count_cached());
  note_kernel("sdpa_flash d%d %s items%lld grid%lld", D, CAUSAL ? (a.causal == 2 ? "causal_lr" : "causal_ul") : "full",
              static_cast<long long>(total), static_cast<long long>(grid));
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(grid)), dim3(kFaWaves * 64), kLds, st, a, nqb);
  return check_launch("sdpa");
}

template <typename T, int D>
int launch_flash_attn(const AttnArgs& a, hipStream_t st) {
  if (a.D < D)
    return a.causal ? launch_flash_attn<T, D, true, true>(a, st) : launch_flash_attn<T, D, false, true>(a, st);
  return a.causal ? launch_flash_attn<T, D, true, false>(a, st) : launch_flash_attn<T, D, false, false>(a, st);
}

template <typename T>
int run_attention(const AttnArgs& a, hipStream_t st) {
  const auto unit_d = [&](const int64_t* s) { return s[3] == 1 && s[2] % 8 == 0 && s[1] % 8 == 0 && s[0] % 8 == 0; };
  // head dims up to 128 in multiples of 8 run on the D = 64 / 128 kernels,
  // the columns past the head dim zero in Q, K and V and dropped from O
  const bool mfma = !std::is_same<T, float>::value && a.D % 8 == 0 && a.D <= 128 && unit_d(a.qs) &&
                    unit_d(a.ks) && unit_d(a.vs) && a.os[3] == 1 && a.os[2] % 4 == 0 &&
                    a.os[1] % 4 == 0 && a.os[0] % 4 == 0 && aligned16(a.q) && aligned16(a.k) &&
                    aligned16(a.v) && (reinterpret_cast<uintptr_t>(a.o) & 7u) == 0;
  if constexpr (!std::is_same<T, float>::value) {
    // DMA path: no explicit mask, a positive scale (the max of the scaled
    // scores is the scaled max), rows that do not overlap, and every key,
    // query and output row's byte offset (up to one block past the end)
    // within 2^31
    const int64_t ld = std::max(a.ks[2], a.vs[2]);
    const int64_t qo = std::max(a.qs[2], a.os[2]);
    const bool dma = mfma && a.mask_dtype < 0 && a.scale_log2 > 0.f && a.Sq > 128 && a.Skv > 0 &&
                     a.ks[2] >= a.D && a.vs[2] >= a.D && (static_cast<int64_t>(a.Skv) + 256) * ld * 2 < 0x7fffffffLL &&
                     (static_cast<int64_t>(a.Sq) + kFaRows) * qo * 2 < 0x7fffffffLL;
    if (dma) return a.D > 64 ? launch_flash_attn<T, 128>(a, st) : launch_flash_attn<T, 64>(a, st);
    // the masked MFMA kernel takes the mask with contiguous keys through a
    // per-(batch, head) buffer resource (its plane spanning less than 2^31
    // bytes) and folds it into S as mask / scale (scale != 0)
    const int esz = a.mask_dtype == NTOPS_BOOL ? 1 : a.mask_dtype == NTOPS_F32 ? 4 : 2;
    const bool mask_fits = a.mask_dtype < 0 ||
                           (a.ms[3] == 1 && a.scale_log2 != 0.f &&
                            (static_cast<int64_t>(a.Sq) * a.ms[2] + a.Skv + 68) * esz < 0x7fffffffLL);
    if (mfma && mask_fits) {
      const int nqb = (a.Sq + 127) / 128;
      const int64_t total = static_cast<int64_t>(nqb) * a.Hq * a.B;
      if (total > 0x7fffffffLL) return set_error(NTOPS_ERR_UNSUPPORTED, "sdpa: too many blocks");
      const uintptr_t mp = reinterpret_cast<uintptr_t>(a.mask);
      const int mm = a.mask_dtype < 0 ? 0
                     : (a.ms[2] % 4 == 0 && a.ms[1] % 4 == 0 && a.ms[0] % 4 == 0 && mp % (4 * esz) == 0) ? 1 : 2;
      const dim3 grid = blocks_2d(total), block(256);
      note_kernel("sdpa_fwd d%d mask%d es%d", a.D > 64 ? 128 : 64, mm, esz);
#define NTOPS_FWD(DD, MM, ES) hipLaunchKernelGGL((k_flash_fwd<T, DD, MM, ES>), grid, block, 0, st, a, nqb, static_cast<int>(total))
#define NTOPS_FWD_D(DD)                         \
  if (mm == 0) NTOPS_FWD(DD, 0, 1);             \
  else if (mm == 1 && esz == 1) NTOPS_FWD(DD, 1, 1); \
  else if (mm == 1 && esz == 2) NTOPS_FWD(DD, 1, 2); \
  else if (mm == 1) NTOPS_FWD(DD, 1, 4);        \
  else if (esz == 1) NTOPS_FWD(DD, 2, 1);       \
  else if (esz == 2) NTOPS_FWD(DD, 2, 2);       \
  else NTOPS_FWD(DD, 2, 4);
      if (a.D > 64) {
        NTOPS_FWD_D(128)
      } else {
        NTOPS_FWD_D(64)
      }
#undef NTOPS_FWD_D
#undef NTOPS_FWD
      return check_launch("sdpa");
    }
  }
  if constexpr (std::is_same<T, float>::value) {
    // fp32 on the matrix cores: head dims up to 128 in multiples of 4,
    // unit-stride head dims with 16-byte aligned rows
    const auto unit4 = [&](const int64_t* s) { return s[3] == 1 && s[2] % 4 == 0 && s[1] % 4 == 0 && s[0] % 4 == 0; };
    if (a.D % 4 == 0 && a.D <= 128 && unit4(a.qs) && unit4(a.ks) && unit4(a.vs) && unit4(a.os) && aligned16(a.q) &&
        aligned16(a.k) && aligned16(a.v) && aligned16(a.o)) {
      // 8 waves of one 16-row block each measured fastest: two blocks per
      // wave (4 or 8 waves) need 190-400 registers and ran 2-45 % slower
      if (a.D <= 32) return launch_flash_f32<32, 8, 1>(a, st);
      if (a.D <= 64) return launch_flash_f32<64, 8, 1>(a, st);
      return launch_flash_f32<128, 8, 1>(a, st);
    }
  }
  const int64_t rows = static_cast<int64_t>(a.B) * a.Hq * a.Sq;
  if (rows > 0x7fffffffLL) return set_error(NTOPS_ERR_UNSUPPORTED, "sdpa: too many rows");
  note_kernel("sdpa_generic");
  hipLaunchKernelGGL((k_attn_generic<T>), blocks_2d(rows), dim3(64), 0, st, a);
  return check_launch("sdpa");
}

}  // namespace
}  // namespace ntops

using namespace ntops;

extern "C" int ntops_sdpa(int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Skv,
                          int64_t D, const void* q, const int64_t* q_strides, const void* k,
                          const int64_t* k_strides, const void* v, const int64_t* v_strides,
                          const void* mask, int mask_dtype, const int64_t* mask_strides, int causal,
                          double scale, void* out, const int64_t* out_strides, void* stream) {
  if (B < 0 || Hq < 0 || Hkv < 0 || Sq < 0 || Skv < 0 || D < 0)
    return set_error(NTOPS_ERR_INVALID, "sdpa: negative size");
  if (B > 0x7fffffffLL || Hq > 0x7fffffffLL || Sq > 0x7fffffffLL || Skv > 0x7fffffffLL)
    return set_error(NTOPS_ERR_UNSUPPORTED, "sdpa: size exceeds int32");
  if (D > 256) return set_error(NTOPS_ERR_UNSUPPORTED, "sdpa: head dim %lld > 256", (long long)D);
  if (causal < 0 || causal > 2) return set_error(NTOPS_ERR_INVALID, "sdpa: bad causal mode %d", causal);
  if (causal && mask) return set_error(NTOPS_ERR_INVALID, "sdpa: a mask and a causal mode together");
  if (mask && mask_dtype != NTOPS_BOOL && mask_dtype != NTOPS_F32 && mask_dtype != NTOPS_F16 &&
      mask_dtype != NTOPS_BF16)
    return set_error(NTOPS_ERR_UNSUPPORTED, "sdpa: mask dtype %d", mask_dtype);
  if (B == 0 || Hq == 0 || Sq == 0 || D == 0) return NTOPS_OK;
  if (Hkv == 0 || Hq % Hkv != 0)
    return set_error(NTOPS_ERR_INVALID, "sdpa: query heads %lld not a multiple of key heads %lld",
                     (long long)Hq, (long long)Hkv);
  if (!q || !out || !q_strides || !k_strides || !v_strides || !out_strides || (Skv > 0 && (!k || !v)) ||
      (mask && !mask_strides))
    return set_error(NTOPS_ERR_INVALID, "sdpa: null pointer");
  AttnArgs a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.mask = mask;
  a.o = out;
  for (int i = 0; i < 4; ++i) {
    a.qs[i] = q_strides[i];
    a.ks[i] = k_strides[i];
    a.vs[i] = v_strides[i];
    a.ms[i] = mask ? mask_strides[i] : 0;
    a.os[i] = out_strides[i];
  }
  a.B = static_cast<int>(B);
  a.Hq = static_cast<int>(Hq);
  a.Hkv = static_cast<int>(Hkv);
  a.Sq = static_cast<int>(Sq);
  a.Skv = static_cast<int>(Skv);
  a.D = static_cast<int>(D);
  a.mask_dtype = mask ? mask_dtype : -1;
  a.causal = causal;
  a.scale_log2 = static_cast<float>(scale * 1.4426950408889634);
  hipStream_t st = static_cast<hipStream_t>(stream);
  return dispatch_float16_32(dtype, "sdpa", [&](auto tag) {
    using T = decltype(tag);
    return run_attention<T>(a, st);
  });
}
