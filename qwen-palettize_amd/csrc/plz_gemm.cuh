// MFMA GEMM core for gfx950: C[I,J] = sum_r A(i,r) * B(j,r), bf16 operands, fp32 accumulate.
//
// One workgroup = 256 threads = 4 wave64s arranged (BI/WI) x (BJ/WJ); each wave owns a
// WI x WJ sub-tile built from 16x16 accumulator blocks of v_mfma_f32_16x16x32_bf16.
// The reduction runs in stages of BK=64, double-buffered in LDS through registers:
// the next stage's global loads are in flight while the current stage's MFMAs issue.
// LDS tiles are stored [row][r] as 16-byte chunks (8 bf16 of consecutive r) with an
// XOR swizzle chunk ^ (row & 7), so a fragment read (16 rows x one chunk) is
// bank-conflict free.
//
// Operand loaders (one per source format) fill a ROWS x BK tile:
//   LoadRC    dense bf16, element (row, r) at p[row*ld + r]            (r contiguous)
//   LoadMNC   dense bf16, element (row, r) at p[r*ld + row]            (rows contiguous;
//             8x8 blocks are transposed in registers before the LDS write)
//   LoadLutRC palettized W[n,k] with the reduction over k (forward: y = x W^T)
//   LoadLutNN palettized W[n,k] with the reduction over n (grad_x = grad_y W)
#pragma once
#include "plz_common.h"

namespace plz {

constexpr int BK = 64;       // reduction depth of one stage
constexpr int CH = BK / 8;   // 16-byte chunks per tile row

__device__ __forceinline__ int swz(int row, int ch) { return row * CH + (ch ^ (row & 7)); }

struct GemmArgs {
  // main segment operands
  const uint16_t* a;
  int64_t lda;
  const uint16_t* b;
  int64_t ldb;
  const int32_t* packed;  // palettized operand: [Nw, Kw/16]
  const float* pal;       // [Nw, Kw/256, 4]
  int64_t Nw, Kw;         // shape of the palettized weight
  int64_t I, J, R;        // C is I x J, reduction length R
  int64_t r_split;        // reduction length handled by one blockIdx.z
  // optional second segment (rank-r LoRA term), reduction length R2 <= BK
  const uint16_t* a2;
  int64_t lda2;
  const uint16_t* b2;
  int64_t ldb2;
  int R2;
  // epilogue
  void* c;
  int64_t ldc;
  const uint16_t* bias;  // [J] bf16 or null
  float alpha;
  float* partial;        // split / palette partial sums
  // soft epilogue
  const uint16_t* logits;  // [I=N, J=K, 4] bf16 or fp16 bits
  const float* noise;      // [N, K, 4]
  float inv_tau;
  float glog_scale;        // 1 (reference semantics) or inv_tau
  uint16_t* grad_logits;   // [N, K, 4], same dtype as logits
  int logits_f16;
  int tiles_i, tiles_j;
};

// ---------------------------------------------------------------------------------
// Loaders. Each has: static constexpr int kRegs; load(args, row0, r0, regs) issues the
// global loads for one stage; store(lds, regs) writes them (dequantised/transposed).
// ---------------------------------------------------------------------------------

// Dense, r contiguous. SRC selects the operand pointer (0: a, 1: b, 2: a2, 3: b2).
template <int ROWS, int SRC>
struct LoadRC {
  static constexpr int kItems = ROWS * CH;
  static constexpr int kRegs = (kItems + 255) / 256;
  __device__ static void ptrs(const GemmArgs& g, const uint16_t*& p, int64_t& ld, int64_t& nrows,
                              int64_t& R) {
    if (SRC == 0) { p = g.a; ld = g.lda; nrows = g.I; R = g.R; }
    if (SRC == 1) { p = g.b; ld = g.ldb; nrows = g.J; R = g.R; }
    if (SRC == 2) { p = g.a2; ld = g.lda2; nrows = g.I; R = g.R2; }
    if (SRC == 3) { p = g.b2; ld = g.ldb2; nrows = g.J; R = g.R2; }
  }
  __device__ static void load(const GemmArgs& g, int64_t row0, int64_t r0, uint4* regs) {
    const uint16_t* p; int64_t ld, nrows, R;
    ptrs(g, p, ld, nrows, R);
#pragma unroll
    for (int i = 0; i < kRegs; ++i) {
      int c = threadIdx.x + 256 * i;
      int row = c / CH, ch = c % CH;
      int64_t gr = row0 + row, gk = r0 + ch * 8;
      uint4 v = make_uint4(0, 0, 0, 0);
      if ((kItems % 256 == 0 || c < kItems) && gr < nrows && gk < R)
        v = *reinterpret_cast<const uint4*>(p + gr * ld + gk);
      regs[i] = v;
    }
  }
  __device__ static void store(uint4* lds, const uint4* regs) {
#pragma unroll
    for (int i = 0; i < kRegs; ++i) {
      int c = threadIdx.x + 256 * i;
      if (kItems % 256 == 0 || c < kItems) lds[swz(c / CH, c % CH)] = regs[i];
    }
  }
};

// Dense, rows contiguous: element (row, r) at p[r*ld + row]. Works on 8x8 blocks.
template <int ROWS, int SRC>
struct LoadMNC {
  static constexpr int kBlocks = (ROWS / 8) * (BK / 8);
  static constexpr int kIters = (kBlocks + 255) / 256;
  static constexpr int kRegs = 8 * kIters;
  __device__ static void ptrs(const GemmArgs& g, const uint16_t*& p, int64_t& ld, int64_t& nrows,
                              int64_t& R) {
    if (SRC == 0) { p = g.a; ld = g.lda; nrows = g.I; R = g.R; }
    if (SRC == 1) { p = g.b; ld = g.ldb; nrows = g.J; R = g.R; }
    if (SRC == 2) { p = g.a2; ld = g.lda2; nrows = g.I; R = g.R2; }
    if (SRC == 3) { p = g.b2; ld = g.ldb2; nrows = g.J; R = g.R2; }
  }
  __device__ static void load(const GemmArgs& g, int64_t row0, int64_t r0, uint4* regs) {
    const uint16_t* p; int64_t ld, nrows, R;
    ptrs(g, p, ld, nrows, R);
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      int blk = threadIdx.x + 256 * it;
      int rb = blk % (ROWS / 8), kb = blk / (ROWS / 8);
      int64_t gr = row0 + rb * 8;
      bool ok = (kBlocks % 256 == 0 || blk < kBlocks) && gr < nrows;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        int64_t gk = r0 + kb * 8 + j;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (ok && gk < R) v = *reinterpret_cast<const uint4*>(p + gk * ld + gr);
        regs[8 * it + j] = v;
      }
    }
  }
  __device__ static void store(uint4* lds, const uint4* regs) {
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      int blk = threadIdx.x + 256 * it;
      if (!(kBlocks % 256 == 0 || blk < kBlocks)) continue;
      int rb = blk % (ROWS / 8), kb = blk / (ROWS / 8);
      const uint4* in = regs + 8 * it;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;
        uint32_t d[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint4 lo4 = in[2 * j], hi4 = in[2 * j + 1];
          uint32_t lo = (i >> 1) == 0 ? lo4.x : (i >> 1) == 1 ? lo4.y : (i >> 1) == 2 ? lo4.z : lo4.w;
          uint32_t hi = (i >> 1) == 0 ? hi4.x : (i >> 1) == 1 ? hi4.y : (i >> 1) == 2 ? hi4.z : hi4.w;
          d[j] = perm(hi, lo, sel);
        }
        lds[swz(rb * 8 + i, kb)] = make_uint4(d[0], d[1], d[2], d[3]);
      }
    }
  }
};

// Palettized W[n,k] (n = tile row), reduction over k. Item = (row, 32 consecutive k).
template <int ROWS>
struct LoadLutRC {
  static constexpr int kItems = ROWS * (BK / 32);
  static constexpr int kIters = (kItems + 255) / 256;
  static constexpr int kRegs = 2 * kIters;  // {q0, q1, -, -} + palette
  __device__ static void load(const GemmArgs& g, int64_t row0, int64_t r0, uint4* regs) {
    const int64_t wpr = g.Kw / kIdxPerWord, gpr = g.Kw / kPalGroup;
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      int item = threadIdx.x + 256 * it;
      int row = item / 2, h = item % 2;
      int64_t n = row0 + row;
      uint4 q = make_uint4(0, 0, 0, 0), p = make_uint4(0, 0, 0, 0);
      if ((kItems % 256 == 0 || item < kItems) && n < g.Nw) {
        int64_t k = r0 + 32 * h;
        const u32x2 w = *reinterpret_cast<const u32x2*>(g.packed + n * wpr + k / kIdxPerWord);
        q.x = w.x; q.y = w.y;
        p = *reinterpret_cast<const uint4*>(g.pal + (n * gpr + k / kPalGroup) * 4);
      }
      regs[2 * it] = q;
      regs[2 * it + 1] = p;
    }
  }
  __device__ static void store(uint4* lds, const uint4* regs) {
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      int item = threadIdx.x + 256 * it;
      if (!(kItems % 256 == 0 || item < kItems)) continue;
      int row = item / 2, h = item % 2;
      const uint4 p = regs[2 * it + 1];
      PalLut t = make_lut(__builtin_bit_cast(float, p.x), __builtin_bit_cast(float, p.y),
                          __builtin_bit_cast(float, p.z), __builtin_bit_cast(float, p.w));
      uint32_t o[8];
      dequant16(regs[2 * it].x, t, o);
      lds[swz(row, 4 * h + 0)] = make_uint4(o[0], o[1], o[2], o[3]);
      lds[swz(row, 4 * h + 1)] = make_uint4(o[4], o[5], o[6], o[7]);
      dequant16(regs[2 * it].y, t, o);
      lds[swz(row, 4 * h + 2)] = make_uint4(o[0], o[1], o[2], o[3]);
      lds[swz(row, 4 * h + 3)] = make_uint4(o[4], o[5], o[6], o[7]);
    }
  }
};

// Palettized W[n,k] seen as B(k, n): tile rows are k, the reduction runs over n.
// Item = (2 consecutive n, 16 consecutive k); the tile's k range must sit inside one
// 256-wide palette group (ROWS divides 256 and row0 is a multiple of ROWS).
template <int ROWS>
struct LoadLutNN {
  static constexpr int kKW = ROWS / 16;                 // packed words per tile row-span
  static constexpr int kItems = kKW * (BK / 2);
  static constexpr int kIters = (kItems + 255) / 256;
  static constexpr int kRegs = 3 * kIters;              // {qa, qb}, pal a, pal b
  __device__ static void load(const GemmArgs& g, int64_t row0, int64_t r0, uint4* regs) {
    const int64_t wpr = g.Kw / kIdxPerWord, gpr = g.Kw / kPalGroup;
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      int item = threadIdx.x + 256 * it;
      int kw = item % kKW, np = item / kKW;
      int64_t n = r0 + 2 * np, k = row0 + 16 * kw;
      uint4 q = make_uint4(0, 0, 0, 0), pa = make_uint4(0, 0, 0, 0), pb = pa;
      if ((kItems % 256 == 0 || item < kItems) && k < g.Kw) {
        if (n < g.Nw) {
          q.x = (uint32_t)g.packed[n * wpr + k / kIdxPerWord];
          pa = *reinterpret_cast<const uint4*>(g.pal + (n * gpr + k / kPalGroup) * 4);
        }
        if (n + 1 < g.Nw) {
          q.y = (uint32_t)g.packed[(n + 1) * wpr + k / kIdxPerWord];
          pb = *reinterpret_cast<const uint4*>(g.pal + ((n + 1) * gpr + k / kPalGroup) * 4);
        }
      }
      regs[3 * it] = q;
      regs[3 * it + 1] = pa;
      regs[3 * it + 2] = pb;
    }
  }
  __device__ static void store(uint4* lds, const uint4* regs) {
    uint32_t* lds32 = reinterpret_cast<uint32_t*>(lds);
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      int item = threadIdx.x + 256 * it;
      if (!(kItems % 256 == 0 || item < kItems)) continue;
      int kw = item % kKW, np = item / kKW;
      const uint4 pa = regs[3 * it + 1], pb = regs[3 * it + 2];
      PalLut ta = make_lut(__builtin_bit_cast(float, pa.x), __builtin_bit_cast(float, pa.y),
                           __builtin_bit_cast(float, pa.z), __builtin_bit_cast(float, pa.w));
      PalLut tb = make_lut(__builtin_bit_cast(float, pb.x), __builtin_bit_cast(float, pb.y),
                           __builtin_bit_cast(float, pb.z), __builtin_bit_cast(float, pb.w));
      uint32_t o[16];
      dequant16_pair(regs[3 * it].x, ta, regs[3 * it].y, tb, o);
      const int rpos = 2 * np;  // reduction position of row n inside the tile
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) {
        int row = 16 * kw + kk;
        lds32[swz(row, rpos / 8) * 4 + (rpos % 8) / 2] = o[kk];
      }
    }
  }
};

// ---------------------------------------------------------------------------------
// Accumulator geometry shared by the epilogues.
// acc[ti][tj] holds C rows wi*WI + 16*ti + 4*(lane/16) + e (e = 0..3) and
// column wj*WJ + 16*tj + lane%16.
// ---------------------------------------------------------------------------------
template <int BI, int BJ, int WI, int WJ>
struct Geo {
  static constexpr int TI = WI / 16, TJ = WJ / 16;
  static constexpr int WAVES_J = BJ / WJ;
  static_assert((BI / WI) * (BJ / WJ) == 4, "4 waves per workgroup");
};

}  // namespace plz
