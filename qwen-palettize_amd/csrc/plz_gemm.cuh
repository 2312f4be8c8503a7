// Skinny MFMA GEMM core for gfx950 (rank-r LoRA products): C[I,J] = sum_r A(i,r) * B(j,r), bf16 operands, fp32 accumulate.
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
