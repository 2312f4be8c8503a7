// The large GEMMs of the LUT-linear path on the 256x256 MFMA core (plz_gemm2.cuh):
//
//   plz_lut_linear_fwd          y = x W^T (+ bias) (+ t B^T)     fused_lut_kernel.cu:309-518
//   plz_lut_linear_bwd_x        grad_x = grad_y W (+ gt A)       fused_lut_kernel.cu:551-720
//   plz_lut_linear_bwd_palette  class-reduced dW = grad_y^T x    fused_lut_kernel.cu:902-1123
//   plz_soft_bwd                soft grad_logits / grad_palette in the dW epilogue
//                               (fused_lut_kernel.cu:1877-1924, triton_soft_backward.py:227-325)
//   plz_linear_fwd_dense / plz_linear_bwd_x_dense   the same on a materialised bf16 W
//                               (fused_lut_linear_cuda.py:912, 944)
#include <mutex>
#include <type_traits>

#include "plz_gemm2.cuh"
#include "palettize_hip.h"

namespace plz {
namespace g2 {

enum { OP_ROW = 0, OP_COL = 1, OP_LUT_ROW = 2, OP_LUT_COL = 3, OP_LUT_REG = 4 };
enum { EPI_BF16 = 0, EPI_PAL = 1, EPI_SOFT = 2, EPI_F32 = 3, EPI_SWIGLU = 4 };

// Masked register-path copies for a partial reduction stage (r >= rend reads as zero) and for
// the rank-r second segment.
__device__ __forceinline__ void copy_row_tile_masked(uint4* lds, const uint16_t* p, int64_t ld,
                                                     int64_t row0, int64_t nrows, int64_t r0,
                                                     int64_t rend, int64_t half = 0) {
#pragma unroll
  for (int it = 0; it < COPY_INSTS; ++it) {
    const int ch = it * NTHR + threadIdx.x;
    const int row = ch >> 3, c = ch & 7;
    const int64_t gr = row0 + row, gk = r0 + 8 * c;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (gr < nrows && gk < rend)
      v = *reinterpret_cast<const uint4*>(p + half_row(gr, half) * ld + gk);
    lds[row_chunk(row, c)] = v;
  }
}
__device__ __forceinline__ void copy_col_tile_masked(uint4* lds, const uint16_t* p, int64_t ld,
                                                     int64_t row0, int64_t nrows, int64_t r0,
                                                     int64_t rend) {
#pragma unroll
  for (int it = 0; it < COPY_INSTS; ++it) {
    const int ch = it * NTHR + threadIdx.x;
    const int kr = ch >> 5, c = ch & 31;
    const int64_t gr = row0 + 8 * c, gk = r0 + kr;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (gr < nrows && gk < rend) v = *reinterpret_cast<const uint4*>(p + gk * ld + gr);
    lds[col_chunk(kr, c)] = v;
  }
}

// 128 x 256 fp32 staging tile: 16-byte group g = col / 4 of a row at g ^ key, a bijection per
// row (key changes bits 4-5 of g only through row). The key makes each access pattern of the dW
// epilogues conflict-free on the 64 banks:
//   staging writes (a half-wave per row, rows r and r + 4 side by side): bit 3 follows row bit 2;
//   class sums (16 lanes = 4 rows x 4 groups 16 apart, 16-byte reads): bits 2-3 follow g bits 4-5;
//   soft / F32 items and the LoRA grad_B reads: one group per lane pair or per row.
__device__ __forceinline__ int ptile(int row, int col) {
  const int g = col >> 2;
  const int key = (row & 63) ^ (((row >> 2) & 1) << 3) ^ (((g >> 4) & 3) << 2);
  return row * 256 + ((g ^ key) << 2) + (col & 3);
}

// ---- LoRA weight gradients from a dW tile (EPI_PAL / EPI_SOFT / EPI_F32 with g.wg_r > 0) ---
// With t = s x A^T and gt = s grad_y B (A = lora_a [r, K], B = lora_b [N, r]):
//   grad_B = grad_y^T t = s dW A^T,   grad_A = gt^T x = s B^T dW,   dW = grad_y^T x.
// Every dW tile (256 n x 256 k of one M split) adds its share: grad_A's from the accumulator
// registers (they are directly the dW^T operand of an MFMA: lane = k, registers = n), grad_B's
// from the fp32 staging the palette and soft epilogues already write (rows n as MFMA A
// fragments).
// Partials: [split][tiles_i][r][K] (the two wave rows summed in LDS) and
// [split][tiles_j][r][N], summed in a fixed order by pal_wg_reduce_kernel, which also
// applies s.
// 32x32x16 MFMAs with the rank padded to 32 columns (lanes j >= r feed zeros).
constexpr int WG_BT_OFF = 128 * 1024;  // B^T of the tile's rows in LDS: [32][256] bf16,
                                       // column n of row j at n ^ bt_swz(j)
__device__ __forceinline__ int bt_swz(int j) { return (j & 15) << 2; }  // keeps 4-n groups
constexpr int WG_AT_OFF = 144 * 1024;  // A's slice of the tile's k: [32][256] bf16, 16-byte
                                       // chunk c of row j at chunk c ^ (j & 31)
typedef __attribute__((address_space(3))) uint16_t lds_u16;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
typedef __attribute__((address_space(3))) u32x4 lds_w4;

// The tile's slices of both LoRA operands into LDS (all threads; every global load is issued
// before any is used): B^T[j][n - i0] for its 256 rows (zero past N) and A[j][k - j0].
__device__ __forceinline__ void stage_lora_operands(const Args& g, lds_u8* lbase, int64_t i0,
                                                    int64_t j0) {
  lds_u16* bt = reinterpret_cast<lds_u16*>(lbase + WG_BT_OFF);
  lds_w4* at = reinterpret_cast<lds_w4*>(lbase + WG_AT_OFF);
  const int r = g.wg_r, cpr = r / 8;  // 16-byte chunks per row of B
  const int64_t K = g.J;
  constexpr int MAXIT = TILE * 4 / NTHR;  // rank 32: 2 chunks of B and 2 of A per thread
  uint4 vb[MAXIT], va[MAXIT];
#pragma unroll
  for (int it = 0; it < MAXIT; ++it) {
    const int idx = threadIdx.x + it * NTHR;
    vb[it] = va[it] = make_uint4(0, 0, 0, 0);
    if (idx < TILE * cpr) {
      const int nl = idx / cpr, c = idx - nl * cpr;
      if (i0 + nl < g.I) vb[it] = *reinterpret_cast<const uint4*>(g.wg_b + (i0 + nl) * r + 8 * c);
    }
    if (idx < r * (TILE / 8)) {
      const int j = idx >> 5, c = idx & 31;
      if (j0 + 8 * c < K) va[it] = *reinterpret_cast<const uint4*>(g.wg_a + j * K + j0 + 8 * c);
    }
  }
#pragma unroll
  for (int it = 0; it < MAXIT; ++it) {
    const int idx = threadIdx.x + it * NTHR;
    if (idx < TILE * cpr) {
      const int nl = idx / cpr, c = idx - nl * cpr;
      const uint32_t w[4] = {vb[it].x, vb[it].y, vb[it].z, vb[it].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j0r = 8 * c + 2 * e, j1r = j0r + 1;
        bt[j0r * TILE + (nl ^ bt_swz(j0r))] = (uint16_t)(w[e] & 0xffffu);
        bt[j1r * TILE + (nl ^ bt_swz(j1r))] = (uint16_t)(w[e] >> 16);
      }
    }
    if (idx < r * (TILE / 8)) {
      const int j = idx >> 5, c = idx & 31;
      at[j * 32 + (c ^ (j & 31))] = u32x4{va[it].x, va[it].y, va[it].z, va[it].w};
    }
  }
}

// grad_A share of this wave's 128 x 64 of dW: C^T[k][j] = sum_n dW[n][k] B[n][j]. MFMA slot
// s = 8h + i (h = lane / 32) of block (ti, eh) is n = 32 ti + 16 eh + 8 (i / 4) + 4 h + i % 4:
// the accumulator registers 8 eh .. 8 eh + 7 of lane (k, h) hold exactly those n.
__device__ __forceinline__ void lora_grad_a(const Args& g, const f32x16 (&acc)[WT_I][WT_J],
                                            const lds_u8* lbase, int wi, int lane,
                                            f32x16 (&ca)[WT_J]) {
  const lds_u16* bt = reinterpret_cast<const lds_u16*>(lbase + WG_BT_OFF);
  const int j = lane & 31, h = lane >> 5;
  const bool jv = j < g.wg_r;
#pragma unroll
  for (int tj = 0; tj < WT_J; ++tj) ca[tj] = f32x16{};
#pragma unroll
  for (int ti = 0; ti < WT_I; ++ti)
#pragma unroll
    for (int eh = 0; eh < 2; ++eh) {
      const int nl = wi * 128 + 32 * ti + 16 * eh + 4 * h;
      u32x2 lo = {0u, 0u}, hi = {0u, 0u};
      if (jv) {
        lo = *reinterpret_cast<const lds_u32x2*>(bt + j * TILE + (nl ^ bt_swz(j)));
        hi = *reinterpret_cast<const lds_u32x2*>(bt + j * TILE + ((nl + 8) ^ bt_swz(j)));
      }
      const bf16x8 bf = __builtin_bit_cast(bf16x8, u32x4{lo.x, lo.y, hi.x, hi.y});
#pragma unroll
      for (int tj = 0; tj < WT_J; ++tj) {
        const f32x16& a = acc[ti][tj];
        const bf16x8 af = __builtin_bit_cast(
            bf16x8, u32x4{f2bf2(a[8 * eh], a[8 * eh + 1]), f2bf2(a[8 * eh + 2], a[8 * eh + 3]),
                          f2bf2(a[8 * eh + 4], a[8 * eh + 5]), f2bf2(a[8 * eh + 6], a[8 * eh + 7])});
        ca[tj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bf, ca[tj], 0, 0, 0);
      }
    }
}

// grad_B share of one 32-row block of the staged half (staging rows 32 q .. 32 q + 31) over the
// tile's 256 k: C[n][j] = sum_k dW[n][k] A[j][k].
__device__ __forceinline__ void lora_grad_b(const Args& g, const float* sC, const lds_u8* lbase,
                                            int64_t i0, int half, int zsl, int tile_j, int q,
                                            int lane) {
  const lds_w4* at = reinterpret_cast<const lds_w4*>(lbase + WG_AT_OFF);
  const int j = lane & 31, h = lane >> 5;
  const bool jv = j < g.wg_r;
  const int sr = 32 * q + (lane & 31);
  f32x16 cb = f32x16{};
#pragma unroll 4
  for (int ks = 0; ks < TILE / 16; ++ks) {
    const int col = 16 * ks + 8 * h;
    const float4 v0 = *reinterpret_cast<const float4*>(&sC[ptile(sr, col)]);
    const float4 v1 = *reinterpret_cast<const float4*>(&sC[ptile(sr, col + 4)]);
    const bf16x8 af = __builtin_bit_cast(
        bf16x8, u32x4{f2bf2(v0.x, v0.y), f2bf2(v0.z, v0.w), f2bf2(v1.x, v1.y), f2bf2(v1.z, v1.w)});
    u32x4 bv = {0u, 0u, 0u, 0u};
    if (jv) bv = at[j * 32 + ((2 * ks + h) ^ (j & 31))];
    cb = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, __builtin_bit_cast(bf16x8, bv), cb, 0, 0, 0);
  }
  if (!jv) return;
  // j-major partial [split][tiles_j][r][N]: registers 4 e4 .. 4 e4 + 3 are 4 consecutive rows
  float* dst = g.wg_part_b + (((int64_t)zsl * g.tiles_j + tile_j) * g.wg_r + j) * g.I;
#pragma unroll
  for (int e4 = 0; e4 < 4; ++e4) {
    const int srr = 32 * q + 8 * e4 + 4 * h;
    const int64_t n = i0 + (srr >> 6) * 128 + 64 * half + (srr & 63);
    if (n < g.I)
      *reinterpret_cast<float4*>(dst + n) =
          make_float4(cb[4 * e4], cb[4 * e4 + 1], cb[4 * e4 + 2], cb[4 * e4 + 3]);
  }
}

// One reduction stage of MFMAs on LDS tiles: 4 k-steps of 16, 4x4 blocks of 32x32 per wave.
// Fragments are double-buffered in registers: the LDS reads of k-step ks+1 are issued before
// the 16 MFMAs of k-step ks, so one wave per SIMD keeps the matrix core busy. The scheduling
// barriers pin that order (left alone, the compiler sinks each A read next to its first
// MFMA and exposes the LDS latency every 4 MFMAs). fill(part), part = 0..1, runs between
// the MFMA groups: VALU work for the next stage (the palette dequantisation) that then
// overlaps with the matrix core.
template <bool A_COL, bool B_COL>
__device__ __forceinline__ void load_frags(const lds_u8* a_s, const lds_u8* b_s, int ks, int wi,
                                           int wj, int lane, bf16x8 (&a)[WT_I], bf16x8 (&b)[WT_J]) {
#pragma unroll
  for (int i = 0; i < WT_I; ++i)
    a[i] = A_COL ? frag_col(a_s, wi * (32 * WT_I) + 32 * i, ks, lane)
                 : frag_row((const uint4*)a_s, wi * (32 * WT_I) + 32 * i, ks, lane);
#pragma unroll
  for (int j = 0; j < WT_J; ++j)
    b[j] = B_COL ? frag_col(b_s, wj * (32 * WT_J) + 32 * j, ks, lane)
                 : frag_row((const uint4*)b_s, wj * (32 * WT_J) + 32 * j, ks, lane);
}
constexpr int MFMA_PER_KSTEP = WT_I * WT_J;  // 8
__device__ __forceinline__ void mma_kstep(f32x16 (&acc)[WT_I][WT_J], const bf16x8 (&a)[WT_I],
                                          const bf16x8 (&b)[WT_J]) {
#pragma unroll
  for (int i = 0; i < WT_I; ++i)
#pragma unroll
    for (int j = 0; j < WT_J; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
}
// Instruction interleave of one k-step (MFMA_PER_KSTEP MFMAs): the LDS reads of the next
// k-step, the next stage's global->LDS copies (first k-step only) and the palette
// dequantisation (VALU and LDS stores) are spread between the MFMAs, so that no burst of one
// kind stalls the issue of MFMAs (sched_group_barrier masks: 0x008 MFMA, 0x100 LDS read,
// 0x200 LDS write, 0x020 VMEM, 0x002 VALU).
template <int NREAD, int NVMEM, int NVALU, int NWRITE>
__device__ __forceinline__ void interleave_kstep() {
  constexpr int M = MFMA_PER_KSTEP;
  constexpr int R = (NREAD + M - 1) / M, V = (NVMEM + M - 1) / M;
  constexpr int A = (NVALU + M - 1) / M, W = (NWRITE + M - 1) / M;
#pragma unroll
  for (int i = 0; i < M; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if (R > 0 && i * R < NREAD) __builtin_amdgcn_sched_group_barrier(0x100, R, 0);
    if (V > 0 && i * V < NVMEM) __builtin_amdgcn_sched_group_barrier(0x020, V, 0);
    if (A > 0) __builtin_amdgcn_sched_group_barrier(0x002, A, 0);
    if (W > 0 && i * W < NWRITE) __builtin_amdgcn_sched_group_barrier(0x200, W, 0);
  }
}

// A whole stage without overlap (the partial and LoRA stages). Only the first nks k-steps
// hold data (the rest of the stage is zero fill), so only those run.
template <bool A_COL, bool B_COL>
__device__ __forceinline__ void mma_stage_sync(const lds_u8* a_s, const lds_u8* b_s,
                                               f32x16 (&acc)[WT_I][WT_J], int wi, int wj,
                                               int lane, int nks) {
#pragma unroll
  for (int ks = 0; ks < BK / 16; ++ks) {
    if (ks >= nks) break;
    bf16x8 a[WT_I], b[WT_J];
    load_frags<A_COL, B_COL>(a_s, b_s, ks, wi, wj, lane, a, b);
    mma_kstep(acc, a, b);
  }
}

// a_s, b_s: this stage's tiles; na_s, nb_s: the LDS slots that dma(na_s, nb_s) and
// fill(part, nb_s) write for a later stage. All four are distinct slots, and saying so
// (__restrict__) lets the compiler see that the fragment reads cannot alias the copies in
// flight: without it, it waits for every outstanding copy before the first LDS read that
// follows them, one k-step after issuing the next stage's copies.
template <bool A_COL, bool B_COL, bool FILL, typename Dma, typename Fill>
__device__ __forceinline__ void mma_stage(const lds_u8* __restrict__ a_s,
                                          const lds_u8* __restrict__ b_s,
                                          lds_u8* __restrict__ na_s, lds_u8* __restrict__ nb_s,
                                          f32x16 (&acc)[WT_I][WT_J], int wi, int wj, int lane,
                                          Dma&& dma, Fill&& fill) {
  // LDS read instructions per k-step: a row fragment is one ds_read_b128, a col fragment two
  // ds_read_b64_tr_b16
  constexpr int NREAD = WT_I * (A_COL ? 2 : 1) + WT_J * (B_COL ? 2 : 1);
  // palette dequantisation of one word: ~31 VALU and two 16-byte LDS stores (k-steps 0, 1)
  constexpr int NV = FILL ? 32 : 0;
  constexpr int NW = FILL ? 2 : 0;
  // global->LDS copies of the next stage issued by dma(): COPY_INSTS per dense operand
  constexpr int NDMA = COPY_INSTS * (FILL ? 1 : 2);
  ColBases<WT_I> ca;
  ColBases<WT_J> cb;
  if constexpr (A_COL) col_bases(a_s, wi * (32 * WT_I), lane, ca);
  if constexpr (A_COL && B_COL) col_bases(b_s, wj * (32 * WT_J), lane, cb);
  auto frags = [&](int ks, bf16x8 (&a)[WT_I], bf16x8 (&b)[WT_J]) {
    if constexpr (!A_COL) {  // one Col operand at most: the compiler's own addressing is as good
      load_frags<false, B_COL>(a_s, b_s, ks, wi, wj, lane, a, b);
      return;
    }
#pragma unroll
    for (int i = 0; i < WT_I; ++i)
      a[i] = A_COL ? frag_col_at(ca.p1[i], ca.p2[i], ks)
                   : frag_row((const uint4*)a_s, wi * (32 * WT_I) + 32 * i, ks, lane);
#pragma unroll
    for (int j = 0; j < WT_J; ++j)
      b[j] = B_COL ? frag_col_at(cb.p1[j], cb.p2[j], ks)
                   : frag_row((const uint4*)b_s, wj * (32 * WT_J) + 32 * j, ks, lane);
  };
  bf16x8 a0[WT_I], b0[WT_J], a1[WT_I], b1[WT_J];
  frags(0, a0, b0);
  __builtin_amdgcn_sched_barrier(0);
  frags(1, a1, b1);
  dma(na_s, nb_s);
  mma_kstep(acc, a0, b0);
  fill(0, nb_s);
  interleave_kstep<NREAD, NDMA, NV, NW>();
  __builtin_amdgcn_sched_barrier(0);
  frags(2, a0, b0);
  mma_kstep(acc, a1, b1);
  fill(1, nb_s);
  interleave_kstep<NREAD, 0, NV, NW>();
  __builtin_amdgcn_sched_barrier(0);
  frags(3, a1, b1);
  mma_kstep(acc, a0, b0);
  interleave_kstep<NREAD, 0, 0, 0>();
  __builtin_amdgcn_sched_barrier(0);
  mma_kstep(acc, a1, b1);
  interleave_kstep<0, 0, 0, 0>();
  __builtin_amdgcn_sched_barrier(0);
}

// One stage of the dense kernels' two-slot ring whose last k-step overlaps the boundary with
// the next stage. A barrier between stages stalls every SIMD: the workgroup's waves reach it
// together, and behind it each wave must read the next stage's first fragments before its
// next MFMA. Here the barrier runs before the last k-step instead: k-steps 0..2 issue their
// MFMAs and the fragment reads of the following k-step; bar() waits for this wave's copies of
// the next stage and its own fragment reads and passes the barrier, after which no wave reads
// this stage's slot any more and the next stage's tiles are complete; dma() then copies the
// stage after next into this stage's slot (d_a, d_b: the same LDS as a_s, b_s, written only
// after the barrier), and the last k-step's MFMAs cover the reads of the next stage's first
// fragments into a0/b0.
template <bool A_COL, bool B_COL, typename Bar, typename Dma>
__device__ __forceinline__ void mma_stage_pipe(const lds_u8* __restrict__ a_s,
                                               const lds_u8* __restrict__ b_s,
                                               const lds_u8* __restrict__ na_s,
                                               const lds_u8* __restrict__ nb_s,
                                               lds_u8* __restrict__ d_a, lds_u8* __restrict__ d_b,
                                               f32x16 (&acc)[WT_I][WT_J], int wi, int wj,
                                               int lane, bf16x8 (&a0)[WT_I], bf16x8 (&b0)[WT_J],
                                               Bar&& bar, Dma&& dma) {
  constexpr int NREAD = WT_I * (A_COL ? 2 : 1) + WT_J * (B_COL ? 2 : 1);
  bf16x8 a1[WT_I], b1[WT_J];
  load_frags<A_COL, B_COL>(a_s, b_s, 1, wi, wj, lane, a1, b1);
  mma_kstep(acc, a0, b0);
  interleave_kstep<NREAD, 0, 0, 0>();
  __builtin_amdgcn_sched_barrier(0);
  load_frags<A_COL, B_COL>(a_s, b_s, 2, wi, wj, lane, a0, b0);
  mma_kstep(acc, a1, b1);
  interleave_kstep<NREAD, 0, 0, 0>();
  __builtin_amdgcn_sched_barrier(0);
  load_frags<A_COL, B_COL>(a_s, b_s, 3, wi, wj, lane, a1, b1);
  mma_kstep(acc, a0, b0);
  interleave_kstep<NREAD, 0, 0, 0>();
  __builtin_amdgcn_sched_barrier(0);
  bar();
  __builtin_amdgcn_sched_barrier(0);
  dma(d_a, d_b);
  load_frags<A_COL, B_COL>(na_s, nb_s, 0, wi, wj, lane, a0, b0);
  mma_kstep(acc, a1, b1);
  interleave_kstep<NREAD, 2 * COPY_INSTS, 0, 0>();
  __builtin_amdgcn_sched_barrier(0);
}

// mma_stage_pipe for two Col tiles (the dW kernels' ring): fragment reads through per-stage
// opaque addresses (ColBases, see col_bases), those of the next stage formed after the barrier
// from its slots na_s / nb_s and carried into the next call through ca / cb.
template <typename Bar, typename Dma>
__device__ __forceinline__ void mma_stage_pipe_col(ColBases<WT_I>& ca, ColBases<WT_J>& cb,
                                                   const lds_u8* __restrict__ na_s,
                                                   const lds_u8* __restrict__ nb_s,
                                                   lds_u8* __restrict__ d1, lds_u8* __restrict__ d2,
                                                   f32x16 (&acc)[WT_I][WT_J], int wi, int wj,
                                                   int lane, bf16x8 (&a0)[WT_I],
                                                   bf16x8 (&b0)[WT_J], Bar&& bar, Dma&& dma) {
  constexpr int NREAD = 2 * (WT_I + WT_J);
  auto frags = [&](int ks, bf16x8 (&a)[WT_I], bf16x8 (&b)[WT_J]) {
#pragma unroll
    for (int i = 0; i < WT_I; ++i) a[i] = frag_col_at(ca.p1[i], ca.p2[i], ks);
#pragma unroll
    for (int j = 0; j < WT_J; ++j) b[j] = frag_col_at(cb.p1[j], cb.p2[j], ks);
  };
  bf16x8 a1[WT_I], b1[WT_J];
  frags(1, a1, b1);
  mma_kstep(acc, a0, b0);
  interleave_kstep<NREAD, 0, 0, 0>();
  __builtin_amdgcn_sched_barrier(0);
  frags(2, a0, b0);
  mma_kstep(acc, a1, b1);
  interleave_kstep<NREAD, 0, 0, 0>();
  __builtin_amdgcn_sched_barrier(0);
  frags(3, a1, b1);
  mma_kstep(acc, a0, b0);
  interleave_kstep<NREAD, 0, 0, 0>();
  __builtin_amdgcn_sched_barrier(0);
  bar();
  __builtin_amdgcn_sched_barrier(0);
  dma(d1, d2);
  col_bases(na_s, wi * (32 * WT_I), lane, ca);
  col_bases(nb_s, wj * (32 * WT_J), lane, cb);
  frags(0, a0, b0);
  mma_kstep(acc, a1, b1);
  interleave_kstep<NREAD, 2 * COPY_INSTS, 0, 0>();
  __builtin_amdgcn_sched_barrier(0);
}

// One stage of the forward with the palettized operand dequantised in registers (B slot
// holds the raw words and palettes, copy_lut_raw). MFMA k-slots are assigned so that no
// dequantised weight is wasted: for the k-step pair p (32 k = two packed words per row),
// lanes 0..31 feed word 2p and lanes 32..63 word 2p+1 -- the first MFMA of the pair takes
// weights 0..7 of each lane's word, the second weights 8..15. The A fragments read the
// matching 16-byte chunks (chunk 4p + 2*(lane/32) + s), so the products are unchanged.
//
// The instruction order is fixed by hand (sched_barrier(0) between groups): each MFMA is
// followed by a slice of the dequantisation of a word needed by a later MFMA, the LDS reads
// of the next A fragments and the next stage's copies, so that the ~31 VALU per word issue
// while the matrix core is busy. Only the first word of the stage is dequantised up front.
struct DqPart {
  uint32_t a[4], b[4];
};
// lookups of index group g (indices g, g+4, g+8, g+12 of the word)
__device__ __forceinline__ void dq_part(uint32_t q, PalLut t, DqPart& d, int g) {
  const uint32_t u = g == 0 ? (q & 0x03030303u) : ((q >> (2 * g)) & 0x03030303u);
  const uint32_t l = perm(0, t.lo, u), h = perm(0, t.hi, u);
  d.a[g] = perm(h, l, 0x05010400u);  // {w_g, w_g+4}
  d.b[g] = perm(h, l, 0x07030602u);  // {w_g+8, w_g+12}
}
// the word's 8 dwords of bf16 pairs in natural k order (as dequant16)
__device__ __forceinline__ void dq_final(const DqPart& d, uint32_t (&out)[8]) {
  out[0] = perm(d.a[1], d.a[0], 0x05040100u);
  out[1] = perm(d.a[3], d.a[2], 0x05040100u);
  out[2] = perm(d.a[1], d.a[0], 0x07060302u);
  out[3] = perm(d.a[3], d.a[2], 0x07060302u);
  out[4] = perm(d.b[1], d.b[0], 0x05040100u);
  out[5] = perm(d.b[3], d.b[2], 0x05040100u);
  out[6] = perm(d.b[1], d.b[0], 0x07060302u);
  out[7] = perm(d.b[3], d.b[2], 0x07060302u);
}
template <typename Dma>
__device__ __forceinline__ void mma_stage_lutreg(const lds_u8* __restrict__ a_s,
                                                 const lds_u8* __restrict__ b_s,
                                                 lds_u8* __restrict__ na_s,
                                                 lds_u8* __restrict__ nb_s,
                                                 f32x16 (&acc)[WT_I][WT_J], int wi, int wj,
                                                 int lane, Dma&& dma) {
  typedef __attribute__((address_space(3))) const u32x4 lds_u32x4;
  typedef __attribute__((address_space(3))) const f32x4 lds_f32x4;
  const int h = lane >> 5, nn = lane & 31;
  u32x4 qv[WT_J];
  PalLut t[WT_J];
#pragma unroll
  for (int j = 0; j < WT_J; ++j) {
    const int row = wj * (32 * WT_J) + 32 * j + nn;
    qv[j] = *reinterpret_cast<lds_u32x4*>(b_s + 16 * row);
    const f32x4 p = *reinterpret_cast<lds_f32x4*>(b_s + LUT_RAW_PAL + 16 * row);
    t[j] = make_lut(p[0], p[1], p[2], p[3]);
  }
  // word of pair p for block j: lanes 0..31 word 2p, lanes 32..63 word 2p+1
  auto word = [&](int p, int j) -> uint32_t {
    return p == 0 ? (h ? qv[j][1] : qv[j][0]) : (h ? qv[j][3] : qv[j][2]);
  };
  auto afrag = [&](int p, int s2, int i) {
    return frag_row_chunk((const uint4*)a_s, wi * (32 * WT_I) + 32 * i, 4 * p + 2 * h + s2, lane);
  };
  auto mfma = [&](int i, int j, bf16x8 a, const uint32_t (&w)[8], int s2) {
    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        a, __builtin_bit_cast(bf16x8, u32x4{w[4 * s2], w[4 * s2 + 1], w[4 * s2 + 2], w[4 * s2 + 3]}),
        acc[i][j], 0, 0, 0);
  };
  uint32_t w[2][WT_J][8];  // dequantised words, [pair][block]
  DqPart d;
  bf16x8 a0[WT_I], a1[WT_I];
  // up front: A fragments of (p0, s0) and the word of (p0, j0)
#pragma unroll
  for (int i = 0; i < WT_I; ++i) a0[i] = afrag(0, 0, i);
#pragma unroll
  for (int g = 0; g < 4; ++g) dq_part(word(0, 0), t[0], d, g);
  dq_final(d, w[0][0]);
  __builtin_amdgcn_sched_barrier(0);
  // (p0, s0, j0) x 4 with word (p0, j1) and the A fragments of (p0, s1)
#pragma unroll
  for (int i = 0; i < WT_I; ++i) {
    mfma(i, 0, a0[i], w[0][0], 0);
    dq_part(word(0, 1), t[1], d, i);
    if (i == WT_I - 1) dq_final(d, w[0][1]);
    a1[i] = afrag(0, 1, i);
    __builtin_amdgcn_sched_barrier(0);
  }
  // (p0, s0, j1) x 4 with word (p1, j0) and the next stage's copies
#pragma unroll
  for (int i = 0; i < WT_I; ++i) {
    mfma(i, 1, a0[i], w[0][1], 0);
    dq_part(word(1, 0), t[0], d, i);
    if (i == WT_I - 1) dq_final(d, w[1][0]);
    if (i == 0) dma(na_s, nb_s);
    __builtin_amdgcn_sched_barrier(0);
  }
  // (p0, s1, j0..1) x 8 with word (p1, j1) and the A fragments of (p1, s0)
#pragma unroll
  for (int i = 0; i < WT_I; ++i) {
#pragma unroll
    for (int j = 0; j < WT_J; ++j) {
      mfma(i, j, a1[i], w[0][j], 1);
      if (j == 0) dq_part(word(1, 1), t[1], d, i);
      if (j == 1) a0[i] = afrag(1, 0, i);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  dq_final(d, w[1][1]);
  __builtin_amdgcn_sched_barrier(0);
  // (p1, s0) x 8 with the A fragments of (p1, s1)
#pragma unroll
  for (int i = 0; i < WT_I; ++i) {
#pragma unroll
    for (int j = 0; j < WT_J; ++j) {
      mfma(i, j, a0[i], w[1][j], 0);
      if (j == 1) a1[i] = afrag(1, 1, i);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // (p1, s1) x 8
#pragma unroll
  for (int i = 0; i < WT_I; ++i)
#pragma unroll
    for (int j = 0; j < WT_J; ++j) mfma(i, j, a1[i], w[1][j], 1);
  __builtin_amdgcn_sched_barrier(0);
}

// Soft backward of one (row n, 128-k segment) item, one wave; lane holds dW at k = kseg + 2*lane,
// +1. Recomputes P = softmax((logits + noise) / tau) per weight (fp32), writes
//   grad_logits[n, k, c] = glog_scale * dW * P_c * (palette_c - W_soft)   (W_soft = sum_c P_c palette_c)
// and the segment's P-weighted class sums of dW to partial[n][kseg/128][4] (the palette
// gradient before the sum over the group's two segments): fused_lut_kernel.cu:1877-1924.
// The item's operands (palette row, logits, tensor noise) are loaded by soft_load, separately
// from the math, so a loop over items can issue the next item's loads before this one's math.
struct SoftIn {
  float4 pal;
  uint4 lg;
  float4 z0, z1;  // tensor noise of the lane's two weights (unused with Philox noise)
};
__device__ __forceinline__ SoftIn soft_load(const Args& g, int64_t n, int64_t kseg, int lane) {
  const int64_t k = kseg + 2 * lane, e0 = (n * g.J + k) * 4;
  SoftIn in;
  in.pal = *reinterpret_cast<const float4*>(g.pal + (n * (g.J / 256) + k / 256) * 4);
  if (g.pin) {  // the forward's P of the lane's two weights
    in.lg = *reinterpret_cast<const uint4*>(g.pin + e0);
    return in;
  }
  in.lg = *reinterpret_cast<const uint4*>(g.logits + e0);
  if (g.noise) {
    in.z0 = *reinterpret_cast<const float4*>(g.noise + e0);
    in.z1 = *reinterpret_cast<const float4*>(g.noise + e0 + 4);
  }
  return in;
}

// Sum of four per-lane values over the wave, one class per 16-lane row: on return lane l holds
// the total of class l / 16. Each step halves the values a lane carries: lanes 0-31 keep classes
// 0, 1 and take lanes 32-63's (v_permlane32_swap: lane l <-> l + 32 in one VALU instruction),
// then each 16-lane half keeps one class (v_permlane16_swap), then a row sums its 16 lanes by
// DPP rotations (8, 4, 2, 1). No LDS traffic, 10 VALU instructions against 24 lane shuffles.
__device__ __forceinline__ float swap32_sum(float lo, float hi) {
  // lanes 0-31: lo[l] + lo[l + 32];  lanes 32-63: hi[l - 32] + hi[l]
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(lo), __float_as_uint(hi), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float swap16_sum(float lo, float hi) {
  // within each 32-lane half: lanes 0-15 lo[l] + lo[l + 16];  lanes 16-31 hi[l - 16] + hi[l]
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF,
                                                        false));
}
// the sum of v over the 64 lanes, in every lane
__device__ __forceinline__ float wave_sum1(float v) {
  const float w = swap32_sum(v, v);  // lanes l, l ^ 32
  float q = swap16_sum(w, w);          // and l ^ 16, l ^ 48
  q = dpp_add<0x128>(q);
  q = dpp_add<0x124>(q);
  q = dpp_add<0x122>(q);
  return dpp_add<0x121>(q);
}
__device__ __forceinline__ float wave_sum4(const float (&sp)[4]) {
  const float a = swap32_sum(sp[0], sp[2]);  // class 0 (lanes 0-31) / class 2 (lanes 32-63)
  const float b = swap32_sum(sp[1], sp[3]);  // class 1 / class 3
  float q = swap16_sum(a, b);                // class l / 16, over lanes l % 16 + 16 j
  q = dpp_add<0x128>(q);                     // row_ror:8
  q = dpp_add<0x124>(q);                     // row_ror:4
  q = dpp_add<0x122>(q);                     // row_ror:2
  return dpp_add<0x121>(q);                  // row_ror:1
}

__device__ __forceinline__ void soft_math(const Args& g, int64_t n, int64_t kseg, int lane,
                                          float2 gw, const SoftIn& in) {
  const int64_t k = kseg + 2 * lane;
  const float pc[4] = {in.pal.x, in.pal.y, in.pal.z, in.pal.w};
  const int64_t e0 = (n * g.J + k) * 4;
  const uint32_t lw[4] = {in.lg.x, in.lg.y, in.lg.z, in.lg.w};
  // P of the lane's two weights and dm_c = pal_c - W_soft, W_soft = sum_c P_c pal_c
  float P[2][4], dm[2][4];
  if (g.pin) {  // the forward's P (fp16), as the reference's backward reads its P_aos
#pragma unroll
    for (int el = 0; el < 2; ++el) {
#pragma unroll
      for (int c = 0; c < 4; ++c) P[el][c] = h2f((lw[2 * el + c / 2] >> (16 * (c & 1))) & 0xffffu);
      // pal_c - W_soft as sum_c' P_c' (pal_c - pal_c'), which holds when sum_c P_c = 1: with
      // P rounded to fp16 and one class near 1, pal_c - W_soft for that class would be the
      // difference of two nearly equal numbers whose rounding errors do not cancel
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float d = 0.f;
#pragma unroll
        for (int c2 = 0; c2 < 4; ++c2)
          if (c2 != c) d += P[el][c2] * (pc[c] - pc[c2]);
        dm[el][c] = d;
      }
    }
  } else {
    float ws[2] = {0.f, 0.f};
    float nz[8];
    if (g.noise) {
      nz[0] = in.z0.x; nz[1] = in.z0.y; nz[2] = in.z0.z; nz[3] = in.z0.w;
      nz[4] = in.z1.x; nz[5] = in.z1.y; nz[6] = in.z1.z; nz[7] = in.z1.w;
    } else {  // the noise the forward drew: Philox at noise_offset + n*K + k
      float z[4];
      philox_gumbel4(g.noise_seed, g.noise_offset + (uint64_t)(n * g.J + k), z);
      nz[0] = z[0]; nz[1] = z[1]; nz[2] = z[2]; nz[3] = z[3];
      philox_gumbel4(g.noise_seed, g.noise_offset + (uint64_t)(n * g.J + k + 1), z);
      nz[4] = z[0]; nz[5] = z[1]; nz[6] = z[2]; nz[7] = z[3];
    }
#pragma unroll
    for (int el = 0; el < 2; ++el) {
      float a[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t bits = (lw[2 * el + c / 2] >> (16 * (c & 1))) & 0xffffu;
        a[c] = ((g.logits_f16 ? h2f(bits) : bf2f(bits)) + nz[4 * el + c]) * g.inv_tau;
      }
      const float m = fmaxf(fmaxf(a[0], a[1]), fmaxf(a[2], a[3]));
      float ex[4], s = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        ex[c] = __expf(a[c] - m);
        s += ex[c];
      }
      const float rs = 1.f / s;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        P[el][c] = ex[c] * rs;
        ws[el] += P[el][c] * pc[c];
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) dm[el][c] = pc[c] - ws[el];
    }
  }
  float sp[4] = {0.f, 0.f, 0.f, 0.f};
  uint32_t out[4];
#pragma unroll
  for (int el = 0; el < 2; ++el) {
    const float gv = el == 0 ? gw.x : gw.y;
    uint32_t o16[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float gp = gv * P[el][c];
      sp[c] += gp;
      const float gl = g.glog_scale * gp * dm[el][c];
      o16[c] = g.logits_f16 ? f2h(gl) : f2bf(gl);
    }
    out[2 * el] = o16[0] | (o16[1] << 16);
    out[2 * el + 1] = o16[2] | (o16[3] << 16);
  }
  *reinterpret_cast<uint4*>(g.grad_logits + e0) = make_uint4(out[0], out[1], out[2], out[3]);
  const float tot = wave_sum4(sp);
  if ((lane & 15) == 0) g.partial[(n * (g.J / 128) + kseg / 128) * 4 + (lane >> 4)] = tot;
  if (g.gsq) {  // the squares of the stored values, which a gradient-norm clip sums
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = g.logits_f16 ? h2f(out[i] & 0xffffu) : bf2f(out[i] & 0xffffu);
      const float hi = g.logits_f16 ? h2f(out[i] >> 16) : bf2f(out[i] >> 16);
      q += lo * lo;
      q += hi * hi;
    }
    q = wave_sum1(q);
    if (lane == 0) g.gsq[n * (g.J / 128) + kseg / 128] = q;
  }
}

__device__ __forceinline__ void tile_of(const Args& g, int bid, int& tile_i, int& tile_j) {
  tile_coords(g.group, g.tiles_i, g.tiles_j, bid, tile_i, tile_j);
}

// bf16 epilogue: C = alpha * acc (+ bias). The tile is staged in LDS (rows padded to 528 B so
// the two 64-byte row segments a wave writes per instruction fall in different banks), then
// written out with 16-byte coalesced stores: 16 per thread instead of 128 scattered 2-byte
// stores. acc[ti][tj][e]: row wi*128 + 32*ti + 8*(e/4) + 4*(lane/32) + e%4,
// col wj*64 + 32*tj + lane%32.
constexpr int EPI_RS = 528;  // staging row stride in bytes
// The whole 256x256 tile as bf16 (alpha * acc + bias) in LDS, rows EPI_RS bytes apart.
__device__ __forceinline__ void stage_tile_bf16(const Args& g, const f32x16 (&acc)[WT_I][WT_J],
                                                lds_u8* st, int64_t j0, int wi, int wj,
                                                int lane) {
  float bj[WT_J];
#pragma unroll
  for (int tj = 0; tj < WT_J; ++tj) {
    const int64_t j = j0 + wj * (32 * WT_J) + 32 * tj + (lane & 31);
    bj[tj] = (g.bias && j < g.J) ? bf2f(g.bias[j]) : 0.f;
  }
#pragma unroll
  for (int ti = 0; ti < WT_I; ++ti)
#pragma unroll
    for (int tj = 0; tj < WT_J; ++tj)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = wi * (32 * WT_I) + 32 * ti + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const int col = wj * (32 * WT_J) + 32 * tj + (lane & 31);
        *reinterpret_cast<__attribute__((address_space(3))) uint16_t*>(st + row * EPI_RS + col * 2) =
            (uint16_t)f2bf(g.alpha * acc[ti][tj][e] + bj[tj]);
      }
  __syncthreads();
}
// 8 stored bf16 values plus 8 bf16 residual values, each sum rounded to bf16: what a bf16 tensor
// add of the residual to the GEMM's bf16 output computes
__device__ __forceinline__ u32x4 add_residual8(u32x4 v, const uint16_t* r) {
  const uint4 q = *reinterpret_cast<const uint4*>(r);
  const uint32_t rs[4] = {q.x, q.y, q.z, q.w};
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = f2bf2(bf2f(v[e] & 0xffffu) + bf2f(rs[e] & 0xffffu), bf2f(v[e] >> 16) + bf2f(rs[e] >> 16));
  return o;
}

// 8 stored bf16 values of grad_h at (i, j) through the SwiGLU backward (g.sw_pre set): its gate
// and up gradients go to columns j and J + j of the [I, 2J] output
__device__ __forceinline__ void store_swiglu_bwd8(const Args& g, u32x4 v, uint16_t* C, int64_t i,
                                                  int64_t j) {
  const uint16_t* pre = g.sw_pre + i * g.ld_sw + j;
  uint4 gg, gu;
  swiglu_bwd8(*reinterpret_cast<const uint4*>(pre), *reinterpret_cast<const uint4*>(pre + g.J),
              make_uint4(v[0], v[1], v[2], v[3]), gg, gu);
  const u32x4 a = {gg.x, gg.y, gg.z, gg.w}, b = {gu.x, gu.y, gu.z, gu.w};
  __builtin_nontemporal_store(a, reinterpret_cast<u32x4*>(C + i * g.ldc + j));
  __builtin_nontemporal_store(b, reinterpret_cast<u32x4*>(C + i * g.ldc + g.J + j));
}

__device__ __forceinline__ void store_tile_bf16(const Args& g, const f32x16 (&acc)[WT_I][WT_J],
                                                lds_u8* st, int64_t i0, int64_t j0, int wi,
                                                int wj, int lane) {
  stage_tile_bf16(g, acc, st, j0, wi, wj, lane);
  uint16_t* C = reinterpret_cast<uint16_t*>(g.c);
#pragma unroll 4
  for (int it = 0; it < TILE * TILE / 8 / NTHR; ++it) {
    const int ch = it * NTHR + threadIdx.x;  // 32 chunks of 8 columns per row
    const int row = ch >> 5, c8 = (ch & 31) * 8;
    const int64_t i = i0 + row, j = j0 + c8;
    if (i < g.I && j < g.J) {
      u32x4 v = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(st + row * EPI_RS + c8 * 2);
      if (g.res) v = add_residual8(v, g.res + i * g.ldres + j);
      // streaming store: the output is not read again by this launch, so it should not take
      // cache lines from the operands the other workgroups are still reading
      if (g.sw_pre)
        store_swiglu_bwd8(g, v, C, i, j);
      else
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(C + i * g.ldc + j));
    }
  }
}

// EPI_SWIGLU: the tile's columns are 128 gate columns followed by the 128 matching up columns
// (the weight's rows interleaved in 128-row blocks, or a [gate | up] weight read through
// half_row); writes h = swiglu(gate, up) to the 128 columns j0/2 .. j0/2+127 of the [I, J/2]
// output, from the staged bf16 values, exactly as a bf16 gate/up GEMM followed by the
// elementwise SwiGLU, and with c2 set also the staged gate/up values themselves.
__device__ __forceinline__ void store_tile_swiglu(const Args& g, const f32x16 (&acc)[WT_I][WT_J],
                                                  lds_u8* st, int64_t i0, int64_t j0, int wi,
                                                  int wj, int lane) {
  stage_tile_bf16(g, acc, st, j0, wi, wj, lane);
  uint16_t* C = reinterpret_cast<uint16_t*>(g.c);
  const int64_t h0 = j0 / 2;
  if (g.c2) {
#pragma unroll 4
    for (int it = 0; it < TILE * TILE / 8 / NTHR; ++it) {
      const int ch = it * NTHR + threadIdx.x;  // 32 chunks of 8 columns per row
      const int row = ch >> 5, c8 = (ch & 31) * 8;
      const int64_t i = i0 + row;
      if (i < g.I) {
        const u32x4 v = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(st + row * EPI_RS + c8 * 2);
        // 8 consecutive columns never straddle the two halves (c8 % 8 == 0)
        __builtin_nontemporal_store(
            v, reinterpret_cast<u32x4*>(g.c2 + i * g.ldc2 + half_row(j0 + c8, g.b_half)));
      }
    }
  }
#pragma unroll 2
  for (int it = 0; it < TILE * (TILE / 2) / 8 / NTHR; ++it) {
    const int ch = it * NTHR + threadIdx.x;  // 16 chunks of 8 output columns per row
    const int row = ch >> 4, c8 = (ch & 15) * 8;
    const int64_t i = i0 + row;
    if (i < g.I) {
      const lds_u8* r = st + row * EPI_RS;
      const u32x4 gv = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(r + c8 * 2);
      const u32x4 uv = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(r + (TILE / 2 + c8) * 2);
      u32x4 hv;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float lo = swiglu_elem(bf2f(gv[w] & 0xffffu), bf2f(uv[w] & 0xffffu));
        const float hi = swiglu_elem(bf2f(gv[w] >> 16), bf2f(uv[w] >> 16));
        hv[w] = f2bf2(lo, hi);
      }
      __builtin_nontemporal_store(hv, reinterpret_cast<u32x4*>(C + i * g.ldc + h0 + c8));
    }
  }
}

template <int KA, int KB, int EPI>
__global__ __launch_bounds__(NTHR) void gemm2_kernel(const Args g) {
  extern __shared__ uint4 smem[];
  lds_u8* lbase = (lds_u8*)smem;
  constexpr bool A_COL = KA == OP_COL;
  constexpr bool B_COL = KB == OP_COL || KB == OP_LUT_COL;

  // (split, tile) items in XCD-contiguous ranges; in a tail-split launch the workgroups after
  // the tail_first whole tiles each run one reduction part of a tail tile (map_item)
  const int T = g.tiles_i * g.tiles_j;
  const Item itm = map_item(T, EPI == EPI_BF16 && g.tail_split > 1, g.tail_first, g.tail_split,
                            (int)blockIdx.x, (int)blockIdx.z, (int)gridDim.z);
  const bool tail_part = itm.tail_part;
  const int zsl = itm.zsl, bid = itm.bid, part = itm.part;
  int tile_i, tile_j;
  tile_of(g, bid, tile_i, tile_j);
  const int64_t i0 = (int64_t)tile_i * TILE, j0 = (int64_t)tile_j * TILE;
  const int64_t rbeg = tail_part ? (int64_t)part * g.tail_len : (int64_t)zsl * g.r_split;
  const int64_t rend = min(g.R, rbeg + (tail_part ? g.tail_len : g.r_split));
  const int64_t rlen = rend > rbeg ? rend - rbeg : 0;
  const int nfull = (int)(rlen / BK);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wi = wave / WAVES_J, wj = wave % WAVES_J;
  // copy rings: dW kernels (both operands transposed) -> 5 operand slots; grad_x (B written by
  // this workgroup's VALU) -> 3 A slots + 2 B slots; the forward -> 3 stage slots; the others
  // -> two stage pairs (the dense kernels measured slower with the 5-slot ring)
  constexpr bool RING5 = KA == OP_COL && KB == OP_COL;
  constexpr bool RING3A = KB == OP_LUT_COL;
  constexpr bool RING3 = KB == OP_LUT_REG;

  f32x16 acc[WT_I][WT_J];
#pragma unroll
  for (int i = 0; i < WT_I; ++i)
#pragma unroll
    for (int j = 0; j < WT_J; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Stage list: nfull full stages (asynchronous global->LDS copies), then optionally one
  // partial stage (zero-filled register copy) and one rank-r LoRA stage. The LoRA operands
  // have the same LDS layouts as the main ones (A row-major; B row tile in the forward,
  // col tile in grad_x), so every stage runs the same MFMA body.
  const bool tail = (rlen % BK) != 0;
  const bool lora = (EPI == EPI_BF16 || EPI == EPI_SWIGLU) && g.R2 > 0 && zsl == 0 && part == 0;
  const int nst = nfull + (tail ? 1 : 0) + (lora ? 1 : 0);

  // The palette operand's registers are loaded one stage ahead of the copies: during stage
  // kt, lr_cur holds the LUT words of stage kt+1 (loaded during stage kt-1), which are
  // dequantised between this stage's MFMAs, and lr_next receives those of stage kt+2. So no
  // wave waits on a fresh global load.
  LutRegs lr_cur, lr_next;
  auto lut_load = [&](int kt, LutRegs& r) {
    const int64_t r0 = rbeg + (int64_t)kt * BK;
    if (KB == OP_LUT_ROW) lut_row_load(g, j0, r0, r);
    if (KB == OP_LUT_COL) lut_col_load(g, j0, r0, r);
  };
  // this tile's copy plans (per-lane offsets; stages add uniform offsets)
  TileDma dA, dB;
  LutDma dL;
  if (KA == OP_ROW) dA = row_tile_dma(g.a, g.lda, i0, g.I);
  else dA = col_tile_dma(g.a, g.lda, i0, g.I, g.R);
  // B rows of a [gate | up] weight (EPI_SWIGLU only: the other kernels' copies are unchanged)
  const int64_t bhalf = EPI == EPI_SWIGLU ? g.b_half : 0;
  if (KB == OP_ROW) dB = row_tile_dma(g.b, g.ldb, j0, g.J, bhalf);
  if (KB == OP_COL) dB = col_tile_dma(g.b, g.ldb, j0, g.J, g.R);
  if (KB == OP_LUT_REG) dL = lut_raw_dma(g, j0);
  auto copy_stage = [&](lds_u8* As, lds_u8* Bs, int64_t r0) {
    tile_copy(As, dA, (uint32_t)(KA == OP_ROW ? r0 * 2 : r0 * g.lda * 2));
    if (KB == OP_ROW) tile_copy(Bs, dB, (uint32_t)(r0 * 2));
    else if (KB == OP_COL) tile_copy(Bs, dB, (uint32_t)(r0 * g.ldb * 2));
    else if (KB == OP_LUT_REG) copy_lut_raw(Bs, dL, r0);
  };
  auto issue = [&](int s, int kt) {
    lds_u8* As = lbase + s * 2 * TILE_BYTES;
    lds_u8* Bs = As + TILE_BYTES;
    if (kt < nfull) {
      copy_stage(As, Bs, rbeg + (int64_t)kt * BK);
    } else if (tail && kt == nfull) {
      const int64_t r0 = rbeg + (int64_t)nfull * BK;
      if (KA == OP_ROW) copy_row_tile_masked((uint4*)As, g.a, g.lda, i0, g.I, r0, rend);
      else copy_col_tile_masked((uint4*)As, g.a, g.lda, i0, g.I, r0, rend);
      if (KB == OP_ROW) copy_row_tile_masked((uint4*)Bs, g.b, g.ldb, j0, g.J, r0, rend, bhalf);
      else if (KB == OP_COL) copy_col_tile_masked((uint4*)Bs, g.b, g.ldb, j0, g.J, r0, rend);
      else {
        LutRegs t;
        // (OP_LUT_REG: a partial stage is a dequantised row tile, multiplied by the dense body)
        if (KB == OP_LUT_ROW || KB == OP_LUT_REG) { lut_row_load(g, j0, r0, t); lut_row_store((uint4*)Bs, t); }
        else { lut_col_load(g, j0, r0, t); lut_col_store((uint4*)Bs, t); }
      }
    } else {
      copy_row_tile_masked((uint4*)As, g.a2, g.R2, i0, g.I, 0, g.R2);
      if (B_COL) copy_col_tile_masked((uint4*)Bs, g.b2, g.J, j0, g.J, 0, g.R2);
      else copy_row_tile_masked((uint4*)Bs, g.b2, g.R2, j0, g.J, 0, g.R2, bhalf);
    }
  };
  constexpr bool LUT = KB == OP_LUT_ROW || KB == OP_LUT_COL;
  // Full stages run through the pipelined loop (one MFMA body per kernel kind); the
  // partial stage and the LoRA stage follow, synchronously, through buffer 0.
  if constexpr (RING5) {
    // Both operands are copied (32 KB each per stage) into a ring of 5 operand slots. The
    // operand that changes between consecutive tiles of the walk (B when consecutive tiles
    // share their tile-row, else A) misses L2 more often and is copied two stages ahead, the
    // other one stage ahead. Copy c of the sequence lead_0, other_0, lead_1, other_1, ... goes
    // to slot c % 5. Stages run as mma_stage_pipe_col: the barrier before stage s's last k-step
    // frees the slots of lead_s and other_s, and the two copies issued right after it,
    // other_s+2 then lead_s+3, go to exactly those slots (c = 2s+5 and 2s+6); the slots of
    // lead_s+1, other_s+1 and lead_s+2 stay live. Past the last stage the copies repeat stage
    // nfull-1 into the free slots, so every stage issues the same instructions.
    auto ring = [&](auto lead_tag) {
      constexpr bool A_LEADS = decltype(lead_tag)::value;
      auto slot = [&](bool is_a, int kt) -> lds_u8* {
        return lbase + ((2 * kt + (is_a == A_LEADS ? 0 : 1)) % RING_SLOTS) * TILE_BYTES;
      };
      // copy of operand a (else b) of stage kt (past the last stage: of stage nfull-1) to dst
      auto copy = [&](bool a, int kt, lds_u8* dst) {
        const int ks = kt < nfull ? kt : nfull - 1;
        const int64_t r0 = rbeg + (int64_t)ks * BK;
        if (a) tile_copy(dst, dA, (uint32_t)(KA == OP_ROW ? r0 * 2 : r0 * g.lda * 2));
        else tile_copy(dst, dB, (uint32_t)(KB == OP_ROW ? r0 * 2 : r0 * g.ldb * 2));
      };
      ColBases<WT_I> ca;
      ColBases<WT_J> cb;
      bf16x8 a0[WT_I], b0[WT_J];
      if (nfull > 0) {
        copy(A_LEADS, 0, slot(A_LEADS, 0));
        copy(!A_LEADS, 0, slot(!A_LEADS, 0));
        __builtin_amdgcn_sched_barrier(0);
        copy(A_LEADS, 1, slot(A_LEADS, 1));
        copy(!A_LEADS, 1, slot(!A_LEADS, 1));
        copy(A_LEADS, 2, slot(A_LEADS, 2));
        wait_vmcnt<3 * COPY_INSTS>();  // stage 0 has landed; lead_1, other_1, lead_2 may not
        stage_barrier();
        col_bases(slot(true, 0), wi * (32 * WT_I), lane, ca);
        col_bases(slot(false, 0), wj * (32 * WT_J), lane, cb);
#pragma unroll
        for (int i = 0; i < WT_I; ++i) a0[i] = frag_col_at(ca.p1[i], ca.p2[i], 0);
#pragma unroll
        for (int j = 0; j < WT_J; ++j) b0[j] = frag_col_at(cb.p1[j], cb.p2[j], 0);
      }
      for (int kt = 0; kt < nfull; ++kt) {
        mma_stage_pipe_col(
            ca, cb, slot(true, kt + 1), slot(false, kt + 1), slot(A_LEADS, kt),
            slot(!A_LEADS, kt), acc, wi, wj, lane, a0, b0,
            [&] {
              wait_vmcnt<COPY_INSTS>();  // stage kt+1 has landed; lead_kt+2 may not
              stage_barrier();
            },
            [&](lds_u8* other_next2, lds_u8* lead_next3) {
              copy(!A_LEADS, kt + 2, other_next2);
              __builtin_amdgcn_sched_barrier(0);  // other_kt+2 is issued before lead_kt+3
              copy(A_LEADS, kt + 3, lead_next3);
            });
      }
    };
    if (g.group != 1) ring(std::true_type{});
    else ring(std::false_type{});
    __builtin_amdgcn_s_waitcnt(0);  // the repeated copies past the last stage
    __syncthreads();
  } else if constexpr (RING3A) {
    // grad_x: the A tiles (grad_y) are copied two stages ahead through 3 slots; the B tiles
    // (dequantised W^T) are written by the workgroup's VALU one stage ahead into 2 slots, from
    // palette words loaded into registers two stages ahead. Past the last stage the A copies
    // repeat stage nfull-1 into the free slot.
    lds_u8* const bbase = lbase + 3 * TILE_BYTES;
    auto aslot = [&](int kt) { return lbase + (kt % 3) * TILE_BYTES; };
    auto bslot = [&](int kt) { return bbase + (kt & 1) * TILE_BYTES; };
    auto copy_a = [&](int kt, lds_u8* dst) {
      const int ks = kt < nfull ? kt : nfull - 1;
      tile_copy(dst, dA, (uint32_t)((rbeg + (int64_t)ks * BK) * 2));
    };
    if (nfull > 0) {
      lut_load(0, lr_cur);
      if (nfull > 1) lut_load(1, lr_next);
      __builtin_amdgcn_sched_barrier(0);  // the palette words are issued before the copies
      copy_a(0, aslot(0));
      copy_a(1, aslot(1));
      lut_col_store((uint4*)bslot(0), lr_cur);
      wait_vmcnt<COPY_INSTS>();  // A_0 has landed; A_1 may be in flight
      stage_barrier();
    }
    for (int kt = 0; kt < nfull; ++kt) {
      const bool more = kt + 1 < nfull;
      lr_cur = lr_next;  // stage kt+1's words, loaded a stage ago
      if (kt + 2 < nfull) lut_load(kt + 2, lr_next);
      __builtin_amdgcn_sched_barrier(0);  // the palette words are issued before the copies
      mma_stage<A_COL, B_COL, true>(
          aslot(kt), bslot(kt), aslot(kt + 2), bslot(kt + 1), acc, wi, wj, lane,
          [&](lds_u8* na, lds_u8*) { copy_a(kt + 2, na); },
          [&](int part, lds_u8* nb) {
            if (more) lut_col_store_part((uint4*)nb, lr_cur, part);
          });
      wait_vmcnt<COPY_INSTS>();  // A_kt+1 (and the words of stage kt+2) landed; A_kt+2 may not
      stage_barrier();           // also orders the B tile of stage kt+1 before its reads
    }
    __builtin_amdgcn_s_waitcnt(0);  // the repeated copies past the last stage
    __syncthreads();
  } else if constexpr (RING3) {
    // forward: a stage is the x tile (32 KB) and the raw words and palettes (8 KB); both are
    // copied two stages ahead through 3 stage slots (120 KB). Past the last stage the copies
    // repeat stage nfull-1 into the free slot.
    constexpr int SLOT = TILE_BYTES + 8192, PER_STAGE = COPY_INSTS + 1;
    auto sa = [&](int kt) { return lbase + (kt % 3) * SLOT; };
    auto copy = [&](int kt, lds_u8* a, lds_u8* b) {
      const int ks = kt < nfull ? kt : nfull - 1;
      copy_stage(a, b, rbeg + (int64_t)ks * BK);
    };
    if (nfull > 0) {
      copy(0, sa(0), sa(0) + TILE_BYTES);
      copy(1, sa(1), sa(1) + TILE_BYTES);
      wait_vmcnt<PER_STAGE>();  // stage 0 has landed; stage 1 may be in flight
      stage_barrier();
    }
    for (int kt = 0; kt < nfull; ++kt) {
      mma_stage_lutreg(sa(kt), sa(kt) + TILE_BYTES, sa(kt + 2), sa(kt + 2) + TILE_BYTES, acc,
                       wi, wj, lane, [&](lds_u8* na, lds_u8* nb) { copy(kt + 2, na, nb); });
      wait_vmcnt<PER_STAGE>();  // stage kt+1 has landed; stage kt+2 may be in flight
      stage_barrier();
    }
    __builtin_amdgcn_s_waitcnt(0);  // the repeated copies past the last stage
    __syncthreads();
  } else if constexpr (!LUT) {
    // dense operands through two stage slots of 64 KB, the barrier between stages moved
    // before each stage's last k-step (mma_stage_pipe): right after it the copies of stage
    // kt+2 go into stage kt's slot, a full stage ahead of the barrier that completes them.
    // Past the last stage the copies repeat stage nfull-1 into the idle slot, so every
    // stage issues the same instructions.
    auto slot = [&](int kt) { return lbase + (kt & 1) * 2 * TILE_BYTES; };
    auto copy = [&](int kt, lds_u8* as) {
      const int ks = kt < nfull ? kt : nfull - 1;
      copy_stage(as, as + TILE_BYTES, rbeg + (int64_t)ks * BK);
    };
    bf16x8 a0[WT_I], b0[WT_J];
    if (nfull > 0) {
      copy(0, slot(0));
      copy(1, slot(1));
      wait_vmcnt<2 * COPY_INSTS>();  // stage 0 has landed; stage 1 may be in flight
      stage_barrier();
      load_frags<A_COL, B_COL>(slot(0), slot(0) + TILE_BYTES, 0, wi, wj, lane, a0, b0);
    }
    for (int kt = 0; kt < nfull; ++kt) {
      lds_u8* const cs = slot(kt);
      const lds_u8* const ns = slot(kt + 1);
      mma_stage_pipe<A_COL, B_COL>(
          cs, cs + TILE_BYTES, ns, ns + TILE_BYTES, cs, cs + TILE_BYTES, acc, wi, wj, lane, a0,
          b0,
          [&] {
            wait_vmcnt<0>();  // this wave's copies of stage kt+1
            stage_barrier();
          },
          [&](lds_u8* da, lds_u8*) { copy(kt + 2, da); });
    }
    __builtin_amdgcn_s_waitcnt(0);  // the repeated copies past the last stage
    __syncthreads();
  } else {
  if (nfull > 0) {
    issue(0, 0);
    if (LUT) {
      lut_load(0, lr_cur);
      if (nfull > 1) lut_load(1, lr_next);
      uint4* Bs = (uint4*)(lbase + TILE_BYTES);
      if (KB == OP_LUT_ROW) lut_row_store(Bs, lr_cur);
      if (KB == OP_LUT_COL) lut_col_store(Bs, lr_cur);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int kt = 0; kt < nfull; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nfull;
    if (LUT) {
      lr_cur = lr_next;  // stage kt+1's words, loaded a stage ago
      if (kt + 2 < nfull) lut_load(kt + 2, lr_next);
    }
    const lds_u8* As = lbase + cur * 2 * TILE_BYTES;
    // copies of stage kt+1 are issued inside the first k-step (interleaved with its MFMAs);
    // the last stage reloads itself into the idle buffer, which keeps the instruction stream
    // identical (the stage-end wait covers the copies before the buffers are reused)
    lds_u8* An = lbase + (cur ^ 1) * 2 * TILE_BYTES;
    const int64_t r_next = rbeg + (int64_t)(more ? kt + 1 : kt) * BK;
    auto dma = [&](lds_u8* na, lds_u8* nb) { copy_stage(na, nb, r_next); };
    if constexpr (KB == OP_LUT_REG) {
      mma_stage_lutreg(As, As + TILE_BYTES, An, An + TILE_BYTES, acc, wi, wj, lane, dma);
    } else {
      // the next stage's palette dequantisation runs between this stage's MFMA groups
      mma_stage<A_COL, B_COL, LUT>(As, As + TILE_BYTES, An, An + TILE_BYTES, acc, wi, wj, lane,
                                   dma, [&](int part, lds_u8* nb) {
        if (!LUT || !more) return;
        if (KB == OP_LUT_ROW) lut_row_store_part((uint4*)nb, lr_cur, part);
        if (KB == OP_LUT_COL) lut_col_store_part((uint4*)nb, lr_cur, part);
      });
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  }  // RING5
  for (int kt = nfull; kt < nst; ++kt) {
    issue(0, kt);  // register copies (zero-filled past the end)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // reduction length of this stage: the ragged tail of R, or the LoRA rank
    const int len = tail && kt == nfull ? (int)(rend - (rbeg + (int64_t)nfull * BK)) : g.R2;
    mma_stage_sync<A_COL, B_COL>(lbase, lbase + TILE_BYTES, acc, wi, wj, lane, (len + 15) / 16);
    __syncthreads();
  }

  // ---- epilogues ----------------------------------------------------------------------
  // acc[ti][tj][e]: row wi*128 + 32*ti + 8*(e/4) + 4*(lane/32) + e%4,
  //                 col wj*64 + 32*tj + lane%32
  if (EPI == EPI_BF16) {
    if (tail_part) {  // this part's accumulators, coalesced: [part][32 float4][thread]
      float4* dst = reinterpret_cast<float4*>(g.tail_ws) +
                    ((int64_t)(bid - g.tail_first) * g.tail_split + part) * (TILE * TILE / 4);
#pragma unroll
      for (int ti = 0; ti < WT_I; ++ti)
#pragma unroll
        for (int tj = 0; tj < WT_J; ++tj)
#pragma unroll
          for (int e4 = 0; e4 < 4; ++e4)
            dst[((ti * WT_J + tj) * 4 + e4) * NTHR + threadIdx.x] =
                make_float4(acc[ti][tj][4 * e4], acc[ti][tj][4 * e4 + 1],
                            acc[ti][tj][4 * e4 + 2], acc[ti][tj][4 * e4 + 3]);
      return;
    }
    store_tile_bf16(g, acc, lbase, i0, j0, wi, wj, lane);
    return;
  }
  if (EPI == EPI_SWIGLU) {
    store_tile_swiglu(g, acc, lbase, i0, j0, wi, wj, lane);
    return;
  }

  // LoRA weight gradients (dW epilogues: hard grad_palette, soft backward): grad_A's share
  // from the accumulators before they are staged (B^T of the tile's rows through LDS past the
  // staging area)
  const bool wgrad = (EPI == EPI_PAL || EPI == EPI_SOFT || EPI == EPI_F32) && g.wg_r > 0;
  if (wgrad) {
    stage_lora_operands(g, lbase, i0, j0);
    __syncthreads();
    f32x16 ca[WT_J];
    lora_grad_a(g, acc, lbase, wi, lane, ca);
    // the two wave rows' shares of the same k columns meet in LDS (the staging area, free until
    // the staging below): [wj][tj][register][lane]
    float* xs = reinterpret_cast<float*>(smem);
    if (wi == 1)
#pragma unroll
      for (int tj = 0; tj < WT_J; ++tj)
#pragma unroll
        for (int e = 0; e < 16; ++e) xs[((wj * WT_J + tj) * 16 + e) * 64 + lane] = ca[tj][e];
    __syncthreads();
    const int jr = lane & 31, hr = lane >> 5;
    if (wi == 0 && jr < g.wg_r) {
      // ca[tj]: rows k = 8 (e / 4) + 4 h + e % 4 of the wave's k-block tj, column j
      float* dst = g.wg_part_a + (((int64_t)zsl * g.tiles_i + tile_i) * g.wg_r + jr) * g.J;
#pragma unroll
      for (int tj = 0; tj < WT_J; ++tj)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          float v[4];
#pragma unroll
          for (int u = 0; u < 4; ++u)
            v[u] = ca[tj][4 * e4 + u] + xs[((wj * WT_J + tj) * 16 + 4 * e4 + u) * 64 + lane];
          const int64_t k = j0 + wj * (32 * WT_J) + 32 * tj + 8 * e4 + 4 * hr;
          if (k < g.J) *reinterpret_cast<float4*>(dst + k) = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
    __syncthreads();  // the staging below overwrites xs
  }

  // dW tile (rows n = i, cols k = j) staged in two passes of 128 rows of fp32: pass p holds
  // rows wi*128 + 64p .. +64 of every wave (staging row sr <-> tile row
  // (sr/64)*128 + 64p + sr%64), so half of each wave's accumulators are dead after pass 0.
  float* sC = reinterpret_cast<float*>(smem);
  const int64_t segs = g.J / 128;
#pragma unroll
  for (int half = 0; half < 2; ++half) {  // unrolled: acc must only see constant indices
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int ti = 2 * half + tt;
#pragma unroll
      for (int tj = 0; tj < WT_J; ++tj)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          sC[ptile(wi * 64 + 32 * tt + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3),
                   wj * (32 * WT_J) + 32 * tj + (lane & 31))] = acc[ti][tj][e];
    }
    __syncthreads();
    if (EPI == EPI_PAL) {
      // class sums: thread pair (2i, 2i+1) owns one (row, 128-k segment), 64 k each. A class
      // mask comes from the sign-extended index bits (0 or all ones), so each value is routed
      // with bitwise ANDs instead of compares and selects; the pair's halves are added in order.
      const int row = (threadIdx.x >> 2) & 127, h = (threadIdx.x >> 1) & 1, sub = threadIdx.x & 1;
      const int64_t n = i0 + (row >> 6) * 128 + 64 * half + (row & 63);
      const int64_t kseg = j0 + 128 * h;
      const bool live = n < g.I && kseg < g.J;
      float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
      if (live) {
        const uint4 q4 =
            reinterpret_cast<const uint4*>(g.packed + n * (g.Kw / 16) + kseg / 16)[sub];
        const uint32_t qs[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
#pragma unroll
          for (int cc = 0; cc < 4; ++cc) {
            const int col = 128 * h + 64 * sub + 16 * w + 4 * cc;
            const float4 v = *reinterpret_cast<const float4*>(&sC[ptile(row, col)]);
            const uint32_t vb[4] = {__float_as_uint(v.x), __float_as_uint(v.y),
                                    __float_as_uint(v.z), __float_as_uint(v.w)};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int bit = 2 * (4 * cc + e);
              const uint32_t m0 = (uint32_t)((int32_t)(qs[w] << (31 - bit)) >> 31);  // index bit 0
              const uint32_t m1 = (uint32_t)((int32_t)(qs[w] << (30 - bit)) >> 31);  // index bit 1
              s0 += __uint_as_float(vb[e] & ~m0 & ~m1);
              s1 += __uint_as_float(vb[e] & m0 & ~m1);
              s2 += __uint_as_float(vb[e] & ~m0 & m1);
              s3 += __uint_as_float(vb[e] & m0 & m1);
            }
          }
        }
      }
      const float o0 = __shfl_xor(s0, 1), o1 = __shfl_xor(s1, 1);
      const float o2 = __shfl_xor(s2, 1), o3 = __shfl_xor(s3, 1);
      if (live && sub == 0) {
        float* dst = g.partial + (((int64_t)zsl * g.I + n) * segs + kseg / 128) * 4;
        *reinterpret_cast<float4*>(dst) = make_float4(s0 + o0, s1 + o1, s2 + o2, s3 + o3);
      }
      // waves 4..7: grad_B's share of the staged half
      if (wgrad && threadIdx.x >= 256)
        lora_grad_b(g, sC, lbase, i0, half, zsl, tile_j, wave - 4, lane);
    } else {  // EPI_SOFT / EPI_F32: waves walk (row, 128-k segment) items; lane = 2 k
      // with the LoRA weight gradients, waves 4..7 take grad_B's share of the staged half: beside
      // the four waves that store the F32 items (cheap), after all eight walked the soft ones
      const int walkers = wgrad && EPI == EPI_F32 ? 4 : NTHR / 64;
      // item -> (row n, segment kseg); false past the tile's 256 items or the matrix edge
      auto item_at = [&](int item, int64_t& n, int64_t& kseg) {
        const int row = item >> 1;
        n = i0 + (row >> 6) * 128 + 64 * half + (row & 63);
        kseg = j0 + 128 * (item & 1);
        return item < 256 && n < g.I && kseg < g.J;
      };
      if (EPI == EPI_SOFT) {
        // each wave's items in turn, the next item's logits / palette / noise loads issued
        // before this item's math, so their latency is covered by it
        int64_t n, kseg;
        bool live = item_at(wave, n, kseg);
        SoftIn cur;
        if (live) cur = soft_load(g, n, kseg, lane);
        for (int item = wave; item < 256; item += walkers) {
          int64_t n2, k2;
          const bool live2 = item_at(item + walkers, n2, k2);
          SoftIn nxt = cur;
          if (live2) nxt = soft_load(g, n2, k2, lane);
          if (live) {
            const float2 gw =
                *reinterpret_cast<const float2*>(&sC[ptile(item >> 1, 128 * (item & 1) + 2 * lane)]);
            soft_math(g, n, kseg, lane, gw, cur);
          }
          cur = nxt;
          live = live2;
          n = n2;
          kseg = k2;
        }
      } else {
        for (int item = wave; wave < walkers && item < 256; item += walkers) {
          int64_t n, kseg;
          if (!item_at(item, n, kseg)) continue;
          const float2 gw =
              *reinterpret_cast<const float2*>(&sC[ptile(item >> 1, 128 * (item & 1) + 2 * lane)]);
          // this split's partial dW rows, [split][N][K] fp32
          *reinterpret_cast<float2*>(g.acc_ws + ((int64_t)zsl * g.I + n) * g.J + kseg + 2 * lane) = gw;
        }
      }
      if (wgrad && threadIdx.x >= 256)
        lora_grad_b(g, sC, lbase, i0, half, zsl, tile_j, wave - 4, lane);
    }
    __syncthreads();
  }
}

// Soft backward of a split launch: dW = the sum of the Z partial [N][K] fp32 slices, summed in
// split order (deterministic), then the per-item soft math. One wave per (row, 128-k segment).
__global__ __launch_bounds__(256) void soft_split_epilogue_kernel(const Args g, int Z) {
  const int lane = threadIdx.x & 63;
  const int64_t segs = g.J / 128;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // wave-uniform
  if (item >= g.I * segs) return;
  const int64_t n = item / segs, kseg = (item % segs) * 128;
  const SoftIn in = soft_load(g, n, kseg, lane);  // issued beside the partial loads
  const float* p = g.acc_ws + n * g.J + kseg + 2 * lane;
  float2 gw = make_float2(0.f, 0.f);
  for (int z = 0; z < Z; ++z) {
    const float2 v = *reinterpret_cast<const float2*>(p + (int64_t)z * g.I * g.J);
    gw.x += v.x;
    gw.y += v.y;
  }
  soft_math(g, n, kseg, lane, gw, in);
}

// Tail tiles of a split launch: sum each tile's reduction parts in part order (deterministic)
// and store it as the unsplit kernel would. Four workgroups of 256 threads per tile, one per
// 64-row slab q: thread t holds what GEMM thread (q / 2) * 256 + t held for its accumulator
// blocks ti = 2 (q % 2), +1 (rows 64 q .. 64 q + 63), so the slabs read and write disjoint
// parts and the launch fills every CU.
constexpr int TAIL_SLABS = 4;
constexpr int TAIL_THREADS = NTHR / 2;
constexpr size_t kLdsTail = (size_t)(TILE / TAIL_SLABS) * EPI_RS;
__global__ __launch_bounds__(TAIL_THREADS) void tail_reduce_kernel(const Args g) {
  extern __shared__ uint4 smem[];
  lds_u8* st = (lds_u8*)smem;
  const int tt = (int)blockIdx.x / TAIL_SLABS, q = (int)blockIdx.x % TAIL_SLABS;
  int tile_i, tile_j;
  tile_of(g, g.tail_first + tt, tile_i, tile_j);
  const int wi = q >> 1, ti0 = 2 * (q & 1);
  const int gt = wi * TAIL_THREADS + threadIdx.x;  // the GEMM thread of these accumulators
  const int wj = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const float4* src = reinterpret_cast<const float4*>(g.tail_ws) +
                      (int64_t)tt * g.tail_split * (TILE * TILE / 4);
  float a[2][WT_J][16];
#pragma unroll
  for (int tl = 0; tl < 2; ++tl)
#pragma unroll
    for (int tj = 0; tj < WT_J; ++tj)
#pragma unroll
      for (int e = 0; e < 16; ++e) a[tl][tj][e] = 0.f;
  for (int p = 0; p < g.tail_split; ++p) {
#pragma unroll
    for (int tl = 0; tl < 2; ++tl)
#pragma unroll
      for (int tj = 0; tj < WT_J; ++tj)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          const float4 v = src[(int64_t)p * (TILE * TILE / 4) +
                               (((ti0 + tl) * WT_J + tj) * 4 + e4) * NTHR + gt];
          a[tl][tj][4 * e4] += v.x;
          a[tl][tj][4 * e4 + 1] += v.y;
          a[tl][tj][4 * e4 + 2] += v.z;
          a[tl][tj][4 * e4 + 3] += v.w;
        }
  }
  // bf16 (alpha * acc + bias) of the slab's 64 rows in LDS, as stage_tile_bf16 computes it
  const int64_t i0 = (int64_t)tile_i * TILE + (TILE / TAIL_SLABS) * q, j0 = (int64_t)tile_j * TILE;
#pragma unroll
  for (int tj = 0; tj < WT_J; ++tj) {
    const int col = wj * (32 * WT_J) + 32 * tj + (lane & 31);
    const float bj = (g.bias && j0 + col < g.J) ? bf2f(g.bias[j0 + col]) : 0.f;
#pragma unroll
    for (int tl = 0; tl < 2; ++tl)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = 32 * tl + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        *reinterpret_cast<__attribute__((address_space(3))) uint16_t*>(st + row * EPI_RS + col * 2) =
            (uint16_t)f2bf(g.alpha * a[tl][tj][e] + bj);
      }
  }
  __syncthreads();
  uint16_t* C = reinterpret_cast<uint16_t*>(g.c);
#pragma unroll
  for (int it = 0; it < (TILE / TAIL_SLABS) * TILE / 8 / TAIL_THREADS; ++it) {
    const int ch = it * TAIL_THREADS + threadIdx.x;  // 32 chunks of 8 columns per row
    const int row = ch >> 5, c8 = (ch & 31) * 8;
    const int64_t i = i0 + row, j = j0 + c8;
    if (i < g.I && j < g.J) {  // streaming store, as store_tile_bf16
      u32x4 v = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(st + row * EPI_RS + c8 * 2);
      if (g.res) v = add_residual8(v, g.res + i * g.ldres + j);
      if (g.sw_pre)
        store_swiglu_bwd8(g, v, C, i, j);
      else
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(C + i * g.ldc + j));
    }
  }
}

constexpr size_t kLds = 256 * 528;  // 132 KB: two pipeline stages (128 KB) or the padded bf16 output tile
constexpr size_t kLdsRing = RING_SLOTS * TILE_BYTES;  // 160 KB: 5 operand slots (or 3 + 2)

template <int KA, int KB, int EPI>
static int launch(Args g, int splits, hipStream_t stream, const char* what) {
  g.tiles_i = (int)((g.I + TILE - 1) / TILE);
  g.tiles_j = (int)((g.J + TILE - 1) / TILE);
  if (g.r_split <= 0) g.r_split = g.R;
  if (g.group == 0) g.group = 8;
  auto kern = gemm2_kernel<KA, KB, EPI>;
  static uint64_t lds_done = 0;
  const size_t lds = (KA == OP_COL && KB == OP_COL) || KB == OP_LUT_COL ? kLdsRing : kLds;
  if (int rc = reserve_lds((const void*)kern, lds, lds_done, what)) return rc;
  const int64_t tiles = (int64_t)g.tiles_i * g.tiles_j;
  if (tiles == 0 || splits == 0) return PLZ_OK;
  // the copies address each operand through a 32-bit buffer offset
  const int64_t lim = (int64_t)1 << 32;
  const int64_t a_bytes = (KA == OP_ROW ? g.I : g.R) * g.lda * 2;
  const int64_t b_bytes = KB == OP_ROW ? g.J * g.ldb * 2 : KB == OP_COL ? g.R * g.ldb * 2 : 0;
  const int64_t l_bytes = KB == OP_LUT_REG ? g.Nw * (g.Kw / 4) : 0;
  if (a_bytes >= lim || b_bytes >= lim || l_bytes >= lim) {
    set_error("%s: an operand spans 4 GiB or more", what);
    return PLZ_EUNSUPPORTED;
  }
  const bool tail = EPI == EPI_BF16 && g.tail_split > 1;
  const int64_t gx = tail ? g.tail_first + (tiles - g.tail_first) * g.tail_split : tiles;
  hipLaunchKernelGGL(kern, dim3((unsigned)gx, 1, (unsigned)splits), dim3(NTHR), lds, stream, g);
  int rc = check_launch(what);
  if (rc != PLZ_OK || !tail) return rc;
  hipLaunchKernelGGL(tail_reduce_kernel, dim3((unsigned)((tiles - g.tail_first) * TAIL_SLABS)),
                     dim3(TAIL_THREADS), kLdsTail, stream, g);
  return check_launch(what);
}

static int cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        v <= 0)
      v = 256;
    cache[dev] = v;
  }
  return cache[dev];
}

static TailPlan tail_plan(int64_t I, int64_t J, int64_t R) {
  return tail_plan_on(I, J, R, cu_count());
}
static size_t tail_bytes(int64_t I, int64_t J, int64_t R) {
  const TailPlan t = tail_plan(I, J, R);
  if (t.split < 2) return 0;
  const int64_t tiles = ((I + TILE - 1) / TILE) * ((J + TILE - 1) / TILE);
  return (size_t)(tiles - t.first) * t.split * TILE * TILE * sizeof(float);
}
// Sets g's tail fields from the plan; no workspace means no split.
static int set_tail(Args& g, void* workspace, size_t workspace_bytes, const char* what) {
  g.tail_split = 1;
  if (!workspace) return PLZ_OK;
  const size_t need = tail_bytes(g.I, g.J, g.R);
  if (need == 0) return PLZ_OK;
  if (workspace_bytes < need) {
    set_error("%s: workspace of %zu bytes needed, %zu given", what, need, workspace_bytes);
    return PLZ_EWORKSPACE;
  }
  const TailPlan t = tail_plan(g.I, g.J, g.R);
  g.tail_first = t.first;
  g.tail_split = t.split;
  g.tail_len = t.len;
  g.tail_ws = reinterpret_cast<float*>(workspace);
  return PLZ_OK;
}

__device__ __forceinline__ void reduce_pal(const float* __restrict__ partial,
                                           float* __restrict__ out, int64_t N, int64_t G, int Z,
                                           int64_t t) {
  if (t >= N * G) return;
  const int64_t n = t / G, gg = t % G;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int z = 0; z < Z; ++z) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float4 v = *reinterpret_cast<const float4*>(
          partial + (((int64_t)z * N + n) * 2 * G + 2 * gg + h) * 4);
      s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
    }
  }
  *reinterpret_cast<float4*>(out + t * 4) = s;
}
__global__ void reduce_pal_kernel(const float* __restrict__ partial, float* __restrict__ out,
                                  int64_t N, int64_t G, int Z) {
  reduce_pal(partial, out, N, G, Z, (int64_t)blockIdx.x * blockDim.x + threadIdx.x);
}

// grad_A [r, K] and grad_B [N, r] = scale x the sum of their partials, in partial order
// (threads 0 .. la-1: grad_A from [p][r][K]; then grad_B from the j-major [p][r][N], thread
// j * N + n writing grad_B[n][j]); bf16 (out_bf16) or fp32 out.
struct WgRed {
  const float* pa; const float* pb;
  void* ga; void* gb;
  int64_t la, lb, N;
  int na, nb, r, out_bf16;
  float scale;
};
__device__ __forceinline__ void wg_reduce(const WgRed& w, int64_t t) {
  const float* __restrict__ pa = w.pa;
  const float* __restrict__ pb = w.pb;
  const int64_t la = w.la, lb = w.lb, N = w.N;
  const int na = w.na, nb = w.nb, r = w.r;
  const bool second = t >= la;
  if (second) t -= la;
  const int64_t L = second ? lb : la;
  if (t >= L) return;
  const float* src = (second ? pb : pa) + t;
  const int np = second ? nb : na;
  // the loads of 16 partials are issued together (the last batch predicated), the adds stay
  // in partial order
  float s = 0.f;
  for (int p = 0; p < np; p += 16) {
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = p + u < np ? src[(int64_t)(p + u) * L] : 0.f;
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (p + u < np) s += v[u];
  }
  s *= w.scale;
  const int64_t o = second ? (t % N) * r + t / N : t;
  void* out = second ? w.gb : w.ga;
  if (w.out_bf16)
    reinterpret_cast<uint16_t*>(out)[o] = (uint16_t)f2bf(s);
  else
    reinterpret_cast<float*>(out)[o] = s;
}
// one launch for both sums of the LoRA grad_palette call: blocks [0, pal_blocks) reduce the
// palette partials, the rest the LoRA weight-gradient partials
__global__ void pal_wg_reduce_kernel(const float* __restrict__ partial,
                                     float* __restrict__ out, int64_t N, int64_t G, int Z,
                                     int pal_blocks, const WgRed w) {
  if ((int)blockIdx.x < pal_blocks)
    reduce_pal(partial, out, N, G, Z, (int64_t)blockIdx.x * blockDim.x + threadIdx.x);
  else
    wg_reduce(w, (int64_t)(blockIdx.x - pal_blocks) * blockDim.x + threadIdx.x);
}

static bool a16(const void* p) { return ((uintptr_t)p & 15) == 0; }

static int palette_splits(int64_t M, int64_t N, int64_t K) {
  return palette_splits_on(M, N, K, cu_count());
}

// The class-reduced dW GEMM over z splits of M (fp32 partials [z][N][K/128][4] in `partial`,
// every entry written by the GEMM), then the fixed-order sum of the partials.
// LoRA weight gradients riding on the hard grad_palette GEMM (optional)
struct WgradArgs {
  const uint16_t* lora_a = nullptr;  // [r, K]
  const uint16_t* lora_b = nullptr;  // [N, r]
  int rank = 0;
  float scale = 1.f;
  void* grad_a = nullptr;  // [r, K]
  void* grad_b = nullptr;  // [N, r]
  int out_bf16 = 1;
  float* part_a = nullptr;
  float* part_b = nullptr;
};
static size_t wg_part_a_floats(int z, int64_t N, int64_t K, int r) {
  return (size_t)z * ((N + TILE - 1) / TILE) * r * K;
}
static size_t wg_part_b_floats(int z, int64_t N, int64_t K, int r) {
  return (size_t)z * ((K + TILE - 1) / TILE) * N * r;
}

static int bwd_palette(const uint16_t* x, const uint16_t* grad_y, const int32_t* packed,
                       float* grad_palette, float* partial, int z, int64_t M, int64_t N,
                       int64_t K, hipStream_t stream, const char* what,
                       const WgradArgs& wg = WgradArgs()) {
  Args g = {};
  g.a = grad_y; g.lda = N;   // A(i=n, r=m) = grad_y[m, n]   (Col tile)
  g.b = x; g.ldb = K;        // B(j=k, r=m) = x[m, k]        (Col tile)
  g.packed = packed; g.Nw = N; g.Kw = K;
  g.I = N; g.J = K; g.R = M; g.r_split = split_len(M, z);
  g.partial = partial;
  g.wg_r = wg.rank;
  g.wg_a = wg.lora_a; g.wg_b = wg.lora_b;
  g.wg_part_a = wg.part_a; g.wg_part_b = wg.part_b;
  // XCD-contiguous item ranges walk the panels of the larger operand: a range then reads a
  // slice of that operand and all of the smaller one (down_proj dW 966 -> 1056 TFLOP/s)
  g.group = K > N ? -1 : 1;
  int rc = launch<OP_COL, OP_COL, EPI_PAL>(g, z, stream, what);
  if (rc != PLZ_OK) return rc;
  const int64_t G = K / 256, n_out = N * G;
  const int pal_blocks = (int)((n_out + 255) / 256);
  if (wg.rank > 0) {
    WgRed w;
    w.pa = wg.part_a; w.pb = wg.part_b; w.ga = wg.grad_a; w.gb = wg.grad_b;
    w.la = (int64_t)wg.rank * K; w.lb = N * wg.rank; w.N = N;
    w.na = z * (int)((N + TILE - 1) / TILE); w.nb = z * (int)((K + TILE - 1) / TILE);
    w.r = wg.rank; w.out_bf16 = wg.out_bf16; w.scale = wg.scale;
    const int wg_blocks = (int)((w.la + w.lb + 255) / 256);
    hipLaunchKernelGGL(pal_wg_reduce_kernel, dim3((unsigned)(pal_blocks + wg_blocks)), dim3(256),
                       0, stream, g.partial, grad_palette, N, G, z, pal_blocks, w);
  } else {
    hipLaunchKernelGGL(reduce_pal_kernel, dim3((unsigned)pal_blocks), dim3(256), 0, stream,
                       g.partial, grad_palette, N, G, z);
  }
  return check_launch(what);
}

// Scratch of plz_lut_linear_bwd_palette_noalloc: the split-M partials live in this
// file-scope device array instead of a caller workspace, so that entry point allocates
// nothing. Each device holds its own copy (at its own address) from the library's load on
// that device until the process ends. In host code `pal_scratch_buf` names a host-side
// stand-in, never device memory: kernels get the device address that hipGetSymbolAddress
// returns for the current device, looked up once per device and kept in pal_scratch_addr.
constexpr size_t kPalScratchBytes = (size_t)32 << 20;  // 32 MiB
__device__ __align__(256) unsigned char pal_scratch_buf[kPalScratchBytes];
static std::mutex pal_scratch_mu;
static void* pal_scratch_addr[64] = {};

static int pal_scratch(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= 64) {
    set_error("plz_lut_linear_bwd_palette_noalloc: no current device (%s)",
              hipGetErrorString(e));
    return PLZ_EHIP;
  }
  std::lock_guard<std::mutex> lock(pal_scratch_mu);
  if (!pal_scratch_addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(pal_scratch_buf));
    if (e != hipSuccess || !p) {
      set_error("plz_lut_linear_bwd_palette_noalloc: hipGetSymbolAddress of the scratch "
                "failed on device %d: %s", dev, hipGetErrorString(e));
      return PLZ_EHIP;
    }
    pal_scratch_addr[dev] = p;
  }
  *out = reinterpret_cast<float*>(pal_scratch_addr[dev]);
  return PLZ_OK;
}

static size_t soft_pal_bytes(int64_t N, int64_t K) { return (size_t)N * (K / 128) * 4 * sizeof(float); }

}  // namespace g2
}  // namespace plz

using namespace plz;
using namespace plz::g2;

// From this many rows the forward and grad_x dequantise W into the workspace and run the
// dense GEMM on it: the LUT GEMMs rebuild each W tile once per 256-row tile of the activations
// (the forward in registers, grad_x in LDS; 10-25% of their time), while dequantising once
// costs N*K*(0.25 + 2) bytes written and read back, which a 4096-row GEMM hides several times
// over.
constexpr int64_t kStagedRows = 4096;
// Tile-rows walked together by the dense GEMMs (consecutive workgroups share an x / grad_y
// panel within groups of this many tile-rows). Measured on the hard step at M = 16384: 4 (and
// 2, 6) 1085-1092 TFLOP/s against 1081 for 8, 1067-1069 for 16, 1053 for a column walk.
constexpr int kDenseGroup = 4;

static size_t staged_w_bytes(int64_t N, int64_t K) {
  return ((size_t)N * (size_t)K * sizeof(uint16_t) + 255) & ~(size_t)255;
}

// Dequantises W into the head of the workspace when it holds W and the tail partials behind
// it; then points g at W (Row tile for the forward, Col tile for grad_x) and the tail
// partials. Returns false (g untouched) when the rows are too few or the workspace too small;
// when it returns true, *rc holds the status of the dequantisation and of the tail set-up.
static bool stage_w(Args& g, const int32_t* packed, const float* palette, int64_t N, int64_t K,
                    void* workspace, size_t workspace_bytes, const char* what, void* stream,
                    int* rc) {
  const size_t wbytes = staged_w_bytes(N, K);
  if (!(N > 0 && workspace && a16(workspace) && g.I >= kStagedRows &&
        workspace_bytes >= wbytes + tail_bytes(g.I, g.J, g.R)))
    return false;
  uint16_t* w = reinterpret_cast<uint16_t*>(workspace);
  *rc = plz_dequant(packed, palette, w, N, K, stream);
  if (*rc != PLZ_OK) return true;
  g.b = w; g.ldb = K;
  g.group = kDenseGroup;
  *rc = set_tail(g, static_cast<uint8_t*>(workspace) + wbytes, workspace_bytes - wbytes, what);
  return true;
}

extern "C" {

size_t plz_lut_linear_fwd_workspace(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  if (M >= kStagedRows) return staged_w_bytes(N, K) + tail_bytes(M, N, K);
  return tail_bytes(M, N, K);
}

int plz_lut_linear_fwd(const uint16_t* x, const int32_t* packed, const float* palette,
                       const uint16_t* bias, const uint16_t* lora_t, const uint16_t* lora_b,
                       int rank, uint16_t* y, void* workspace, size_t workspace_bytes, int64_t M,
                       int64_t N, int64_t K, void* stream) {
  PLZ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "plz_lut_linear_fwd: negative shape");
  PLZ_REQUIRE(K % 256 == 0, "plz_lut_linear_fwd: K (%lld) must be a multiple of 256", (long long)K);
  PLZ_REQUIRE(N % 8 == 0, "plz_lut_linear_fwd: N (%lld) must be a multiple of 8", (long long)N);
  PLZ_REQUIRE(rank >= 0 && rank <= BK && rank % 8 == 0,
              "plz_lut_linear_fwd: rank (%d) must be a multiple of 8 in [0, 64]", rank);
  if (M == 0 || N == 0) return PLZ_OK;
  PLZ_REQUIRE(x && packed && palette && y, "plz_lut_linear_fwd: null pointer");
  PLZ_REQUIRE(a16(x) && a16(palette) && a16(packed),
              "plz_lut_linear_fwd: x, packed and palette must be 16-byte aligned");
  PLZ_REQUIRE(rank == 0 || (lora_t && lora_b && a16(lora_t) && a16(lora_b)),
              "plz_lut_linear_fwd: rank > 0 needs 16-byte aligned lora_t and lora_b");
  Args g = {};
  g.a = x; g.lda = K;
  g.I = M; g.J = N; g.R = K;
  g.a2 = lora_t; g.b2 = lora_b; g.R2 = rank;
  g.c = y; g.ldc = N; g.bias = bias; g.alpha = 1.f;
  int rc = PLZ_OK;
  if (stage_w(g, packed, palette, N, K, workspace, workspace_bytes, "plz_lut_linear_fwd", stream,
              &rc)) {
    if (rc != PLZ_OK) return rc;  // B(j=n, r=k) = w[n, k]   (Row tile)
    return launch<OP_ROW, OP_ROW, EPI_BF16>(g, 1, (hipStream_t)stream, "plz_lut_linear_fwd");
  }
  g.packed = packed; g.pal = palette; g.Nw = N; g.Kw = K;
  g.group = 1;
  rc = set_tail(g, workspace, workspace_bytes, "plz_lut_linear_fwd");
  if (rc != PLZ_OK) return rc;
  return launch<OP_ROW, OP_LUT_REG, EPI_BF16>(g, 1, (hipStream_t)stream, "plz_lut_linear_fwd");
}

size_t plz_lut_linear_bwd_x_workspace(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  if (M >= kStagedRows) return staged_w_bytes(N, K) + tail_bytes(M, K, N);
  return tail_bytes(M, K, N);
}

int plz_lut_linear_bwd_x(const uint16_t* grad_y, const int32_t* packed, const float* palette,
                         const uint16_t* lora_gt, const uint16_t* lora_a, int rank,
                         uint16_t* grad_x, void* workspace, size_t workspace_bytes, int64_t M,
                         int64_t N, int64_t K, void* stream) {
  PLZ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "plz_lut_linear_bwd_x: negative shape");
  PLZ_REQUIRE(K % 256 == 0, "plz_lut_linear_bwd_x: K (%lld) must be a multiple of 256",
              (long long)K);
  PLZ_REQUIRE(N % 8 == 0, "plz_lut_linear_bwd_x: N (%lld) must be a multiple of 8", (long long)N);
  PLZ_REQUIRE(rank >= 0 && rank <= BK && rank % 8 == 0,
              "plz_lut_linear_bwd_x: rank (%d) must be a multiple of 8 in [0, 64]", rank);
  if (M == 0 || K == 0) return PLZ_OK;
  PLZ_REQUIRE(grad_y && packed && palette && grad_x, "plz_lut_linear_bwd_x: null pointer");
  PLZ_REQUIRE(a16(grad_y) && a16(palette) && a16(packed),
              "plz_lut_linear_bwd_x: grad_y, packed and palette must be 16-byte aligned");
  PLZ_REQUIRE(rank == 0 || (lora_gt && lora_a && a16(lora_gt) && a16(lora_a)),
              "plz_lut_linear_bwd_x: rank > 0 needs 16-byte aligned lora_gt and lora_a");
  Args g = {};
  g.a = grad_y; g.lda = N;
  g.I = M; g.J = K; g.R = N;
  g.a2 = lora_gt; g.b2 = lora_a; g.R2 = rank;
  g.c = grad_x; g.ldc = K; g.alpha = 1.f;
  int rc = PLZ_OK;
  if (stage_w(g, packed, palette, N, K, workspace, workspace_bytes, "plz_lut_linear_bwd_x",
              stream, &rc)) {
    if (rc != PLZ_OK) return rc;  // B(j=k, r=n) = w[n, k]   (Col tile)
    return launch<OP_ROW, OP_COL, EPI_BF16>(g, 1, (hipStream_t)stream, "plz_lut_linear_bwd_x");
  }
  g.packed = packed; g.pal = palette; g.Nw = N; g.Kw = K;
  g.group = 1;
  rc = set_tail(g, workspace, workspace_bytes, "plz_lut_linear_bwd_x");
  if (rc != PLZ_OK) return rc;
  return launch<OP_ROW, OP_LUT_COL, EPI_BF16>(g, 1, (hipStream_t)stream, "plz_lut_linear_bwd_x");
}

size_t plz_lut_linear_bwd_palette_workspace(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return (size_t)palette_splits(M, N, K) * N * (K / 128) * 4 * sizeof(float);
}

int plz_lut_linear_bwd_palette(const uint16_t* x, const uint16_t* grad_y, const int32_t* packed,
                               float* grad_palette, void* workspace, size_t workspace_bytes,
                               int64_t M, int64_t N, int64_t K, void* stream) {
  PLZ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "plz_lut_linear_bwd_palette: negative shape");
  PLZ_REQUIRE(K % 256 == 0, "plz_lut_linear_bwd_palette: K (%lld) must be a multiple of 256",
              (long long)K);
  PLZ_REQUIRE(N % 8 == 0, "plz_lut_linear_bwd_palette: N (%lld) must be a multiple of 8",
              (long long)N);
  if (N == 0 || K == 0) return PLZ_OK;
  PLZ_REQUIRE(packed && grad_palette, "plz_lut_linear_bwd_palette: null pointer");
  if (M == 0) {
    zero_async(grad_palette, (size_t)N * (K / 256) * 16, (hipStream_t)stream);
    return check_launch("plz_lut_linear_bwd_palette");
  }
  PLZ_REQUIRE(x && grad_y && a16(x) && a16(grad_y) && a16(packed),
              "plz_lut_linear_bwd_palette: x, grad_y and packed must be non-null, 16-byte aligned");
  const size_t need = plz_lut_linear_bwd_palette_workspace(M, N, K);
  if (!workspace || workspace_bytes < need) {
    set_error("plz_lut_linear_bwd_palette: workspace of %zu bytes needed, %zu given", need,
              workspace_bytes);
    return PLZ_EWORKSPACE;
  }
  return bwd_palette(x, grad_y, packed, grad_palette, reinterpret_cast<float*>(workspace),
                     palette_splits(M, N, K), M, N, K, (hipStream_t)stream,
                     "plz_lut_linear_bwd_palette");
}

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// An empty weight (N == 0 or K == 0) has an empty palette gradient, but the LoRA factor of
// the other side is not empty: grad_a [rank, K] is zero when N == 0 (no output row contributes)
// and grad_b [N, rank] is zero when K == 0 (x A^T is zero).
static int lora_grads_of_empty_weight(void* grad_a, void* grad_b, int rank, int grads_dtype,
                                      int64_t N, int64_t K, hipStream_t stream, const char* what) {
  const size_t esz = grads_dtype == PLZ_DT_BF16 ? 2 : 4;
  PLZ_REQUIRE((K == 0 || grad_a) && (N == 0 || grad_b), "%s: null pointer", what);
  if (K > 0) zero_async(grad_a, (size_t)rank * K * esz, stream);
  if (N > 0) zero_async(grad_b, (size_t)N * rank * esz, stream);
  return check_launch(what);
}

size_t plz_lut_linear_bwd_palette_lora_workspace(int64_t M, int64_t N, int64_t K, int rank) {
  if (M <= 0 || N <= 0 || K <= 0 || rank <= 0) return plz_lut_linear_bwd_palette_workspace(M, N, K);
  const int z = palette_splits(M, N, K);
  return align256(plz_lut_linear_bwd_palette_workspace(M, N, K)) +
         align256(wg_part_a_floats(z, N, K, rank) * sizeof(float)) +
         align256(wg_part_b_floats(z, N, K, rank) * sizeof(float));
}

int plz_lut_linear_bwd_palette_lora(const uint16_t* x, const uint16_t* grad_y,
                                    const int32_t* packed, const uint16_t* lora_a,
                                    const uint16_t* lora_b, int rank, float scale,
                                    float* grad_palette, void* grad_a, void* grad_b,
                                    int grads_dtype, void* workspace, size_t workspace_bytes,
                                    int64_t M, int64_t N, int64_t K, void* stream) {
  const char* what = "plz_lut_linear_bwd_palette_lora";
  PLZ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "%s: negative shape", what);
  PLZ_REQUIRE(K % 256 == 0, "%s: K (%lld) must be a multiple of 256", what, (long long)K);
  PLZ_REQUIRE(N % 8 == 0, "%s: N (%lld) must be a multiple of 8", what, (long long)N);
  PLZ_REQUIRE(rank > 0 && rank <= 32 && rank % 8 == 0,
              "%s: rank (%d) must be a multiple of 8 in [8, 32]", what, rank);
  PLZ_REQUIRE(grads_dtype == PLZ_DT_BF16 || grads_dtype == PLZ_DT_FP32,
              "%s: grads_dtype must be PLZ_DT_BF16 or PLZ_DT_FP32", what);
  if (N == 0 || K == 0) return lora_grads_of_empty_weight(grad_a, grad_b, rank, grads_dtype, N,
                                                          K, (hipStream_t)stream, what);
  PLZ_REQUIRE(packed && grad_palette && lora_a && lora_b && grad_a && grad_b,
              "%s: null pointer", what);
  PLZ_REQUIRE(a16(lora_a) && a16(lora_b), "%s: lora_a and lora_b must be 16-byte aligned", what);
  const size_t esz = grads_dtype == PLZ_DT_BF16 ? 2 : 4;
  if (M == 0) {  // empty reduction: every gradient is zero
    zero_async(grad_palette, (size_t)N * (K / 256) * 16, (hipStream_t)stream);
    zero_async(grad_a, (size_t)rank * K * esz, (hipStream_t)stream);
    zero_async(grad_b, (size_t)N * rank * esz, (hipStream_t)stream);
    return check_launch(what);
  }
  PLZ_REQUIRE(x && grad_y && a16(x) && a16(grad_y) && a16(packed),
              "%s: x, grad_y and packed must be non-null, 16-byte aligned", what);
  const size_t need = plz_lut_linear_bwd_palette_lora_workspace(M, N, K, rank);
  if (!workspace || !a16(workspace) || workspace_bytes < need) {
    set_error("%s: workspace of %zu bytes (16-byte aligned) needed, %zu given", what, need,
              workspace_bytes);
    return PLZ_EWORKSPACE;
  }
  const int z = palette_splits(M, N, K);
  uint8_t* w = static_cast<uint8_t*>(workspace);
  WgradArgs wg;
  wg.lora_a = lora_a; wg.lora_b = lora_b; wg.rank = rank; wg.scale = scale;
  wg.grad_a = grad_a; wg.grad_b = grad_b; wg.out_bf16 = grads_dtype == PLZ_DT_BF16;
  const size_t pal_bytes = align256(plz_lut_linear_bwd_palette_workspace(M, N, K));
  wg.part_a = reinterpret_cast<float*>(w + pal_bytes);
  wg.part_b = reinterpret_cast<float*>(
      w + pal_bytes + align256(wg_part_a_floats(z, N, K, rank) * sizeof(float)));
  return bwd_palette(x, grad_y, packed, grad_palette, reinterpret_cast<float*>(w), z, M, N, K,
                     (hipStream_t)stream, what, wg);
}

int plz_lut_linear_bwd_palette_noalloc(const uint16_t* x, const uint16_t* grad_y,
                                       const int32_t* packed, float* grad_palette, int64_t M,
                                       int64_t N, int64_t K, void* stream) {
  PLZ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "plz_lut_linear_bwd_palette_noalloc: negative shape");
  PLZ_REQUIRE(K % 256 == 0,
              "plz_lut_linear_bwd_palette_noalloc: K (%lld) must be a multiple of 256",
              (long long)K);
  PLZ_REQUIRE(N % 8 == 0, "plz_lut_linear_bwd_palette_noalloc: N (%lld) must be a multiple of 8",
              (long long)N);
  if (N == 0 || K == 0) return PLZ_OK;
  // the split-M partials of one split: N x K/128 class sums of 16 bytes
  const size_t per_split = (size_t)N * (size_t)(K / 128) * 4 * sizeof(float);
  PLZ_REQUIRE(per_split <= kPalScratchBytes,
              "plz_lut_linear_bwd_palette_noalloc: N x K = %lld x %lld needs %zu bytes of "
              "partials per split, above its %zu-byte scratch (N * K at most %zu); use "
              "plz_lut_linear_bwd_palette with a workspace",
              (long long)N, (long long)K, per_split, kPalScratchBytes, kPalScratchBytes * 8);
  PLZ_REQUIRE(packed && grad_palette, "plz_lut_linear_bwd_palette_noalloc: null pointer");
  if (M == 0) {
    zero_async(grad_palette, (size_t)N * (K / 256) * 16, (hipStream_t)stream);
    return check_launch("plz_lut_linear_bwd_palette_noalloc");
  }
  PLZ_REQUIRE(x && grad_y && a16(x) && a16(grad_y) && a16(packed),
              "plz_lut_linear_bwd_palette_noalloc: x, grad_y and packed must be non-null, "
              "16-byte aligned");
  float* partial = nullptr;
  if (int rc = pal_scratch(&partial)) return rc;
  // the workspace variant's split count, lowered until its partials fit the scratch (a lower
  // count only changes the order of the fp32 sums)
  int z = palette_splits(M, N, K);
  const int zfit = (int)(kPalScratchBytes / per_split);
  z = z < zfit ? z : zfit;
  return bwd_palette(x, grad_y, packed, grad_palette, partial, z, M, N, K, (hipStream_t)stream,
                     "plz_lut_linear_bwd_palette_noalloc");
}

size_t plz_linear_fwd_dense_workspace(int64_t M, int64_t N, int64_t K) {
  return M > 0 && N > 0 && K > 0 ? tail_bytes(M, N, K) : 0;
}

static int linear_fwd_dense(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                            const uint16_t* lora_t, const uint16_t* lora_b, int rank,
                            const uint16_t* residual, uint16_t* y, void* workspace,
                            size_t workspace_bytes, int64_t M, int64_t N, int64_t K, void* stream,
                            const char* what) {
  PLZ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "%s: negative shape", what);
  PLZ_REQUIRE(K % 8 == 0 && N % 8 == 0, "%s: K and N must be multiples of 8", what);
  PLZ_REQUIRE(rank >= 0 && rank <= BK && rank % 8 == 0,
              "%s: rank (%d) must be a multiple of 8 in [0, 64]", what, rank);
  if (M == 0 || N == 0) return PLZ_OK;
  PLZ_REQUIRE(x && w && y && a16(x) && a16(w),
              "%s: x, w, y must be non-null; x, w 16-byte aligned", what);
  PLZ_REQUIRE(rank == 0 || (lora_t && lora_b && a16(lora_t) && a16(lora_b)),
              "%s: rank > 0 needs 16-byte aligned lora_t and lora_b", what);
  Args g = {};
  g.a = x; g.lda = K; g.b = w; g.ldb = K;
  g.I = M; g.J = N; g.R = K;
  g.a2 = lora_t; g.b2 = lora_b; g.R2 = rank;
  g.c = y; g.ldc = N; g.bias = bias; g.alpha = 1.f;
  g.res = residual; g.ldres = N;
  g.group = kDenseGroup;
  const int rc = set_tail(g, workspace, workspace_bytes, what);
  if (rc != PLZ_OK) return rc;
  return launch<OP_ROW, OP_ROW, EPI_BF16>(g, 1, (hipStream_t)stream, what);
}

int plz_linear_fwd_dense(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                         const uint16_t* lora_t, const uint16_t* lora_b, int rank, uint16_t* y,
                         void* workspace, size_t workspace_bytes, int64_t M, int64_t N, int64_t K,
                         void* stream) {
  return linear_fwd_dense(x, w, bias, lora_t, lora_b, rank, nullptr, y, workspace,
                          workspace_bytes, M, N, K, stream, "plz_linear_fwd_dense");
}

int plz_linear_fwd_dense_residual(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                  const uint16_t* lora_t, const uint16_t* lora_b, int rank,
                                  const uint16_t* residual, uint16_t* y, void* workspace,
                                  size_t workspace_bytes, int64_t M, int64_t N, int64_t K,
                                  void* stream) {
  PLZ_REQUIRE(M == 0 || N == 0 || (residual && a16(residual) && a16(y)),
              "plz_linear_fwd_dense_residual: residual and y must be non-null, 16-byte aligned");
  return linear_fwd_dense(x, w, bias, lora_t, lora_b, rank, residual, y, workspace,
                          workspace_bytes, M, N, K, stream, "plz_linear_fwd_dense_residual");
}

int plz_linear_fwd_dense_swiglu(const uint16_t* x, const uint16_t* w_gate_up, uint16_t* h,
                                int64_t M, int64_t N, int64_t K, void* stream) {
  PLZ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "plz_linear_fwd_dense_swiglu: negative shape");
  PLZ_REQUIRE(K % 8 == 0 && N % 128 == 0,
              "plz_linear_fwd_dense_swiglu: K must be a multiple of 8 and N of 128");
  if (M == 0 || N == 0) return PLZ_OK;
  PLZ_REQUIRE(x && w_gate_up && h && a16(x) && a16(w_gate_up) && a16(h),
              "plz_linear_fwd_dense_swiglu: x, w_gate_up, h must be non-null, 16-byte aligned");
  Args g = {};
  g.a = x; g.lda = K; g.b = w_gate_up; g.ldb = K;
  g.I = M; g.J = 2 * N; g.R = K;
  g.c = h; g.ldc = N; g.alpha = 1.f;
  g.group = 8;
  return launch<OP_ROW, OP_ROW, EPI_SWIGLU>(g, 1, (hipStream_t)stream,
                                            "plz_linear_fwd_dense_swiglu");
}

int plz_linear_fwd_dense_swiglu_cat(const uint16_t* x, const uint16_t* w, const uint16_t* lora_t,
                                    const uint16_t* lora_b, int rank, uint16_t* y, uint16_t* h,
                                    int64_t M, int64_t F, int64_t K, void* stream) {
  const char* what = "plz_linear_fwd_dense_swiglu_cat";
  PLZ_REQUIRE(M >= 0 && F >= 0 && K >= 0, "%s: negative shape", what);
  PLZ_REQUIRE(K % 8 == 0 && F % 128 == 0, "%s: K must be a multiple of 8 and F of 128", what);
  PLZ_REQUIRE(rank >= 0 && rank <= BK && rank % 8 == 0,
              "%s: rank (%d) must be a multiple of 8 in [0, 64]", what, rank);
  if (M == 0 || F == 0) return PLZ_OK;
  PLZ_REQUIRE(x && w && h && a16(x) && a16(w) && a16(h) && (!y || a16(y)),
              "%s: x, w, h must be non-null; x, w, h, y 16-byte aligned", what);
  PLZ_REQUIRE(rank == 0 || (lora_t && lora_b && a16(lora_t) && a16(lora_b)),
              "%s: rank > 0 needs 16-byte aligned lora_t and lora_b", what);
  Args g = {};
  g.a = x; g.lda = K; g.b = w; g.ldb = K;
  g.I = M; g.J = 2 * F; g.R = K;
  g.a2 = lora_t; g.b2 = lora_b; g.R2 = rank;
  g.c = h; g.ldc = F; g.alpha = 1.f;
  g.b_half = F; g.c2 = y; g.ldc2 = 2 * F;
  g.group = kDenseGroup;
  return launch<OP_ROW, OP_ROW, EPI_SWIGLU>(g, 1, (hipStream_t)stream, what);
}

size_t plz_linear_bwd_x_dense_workspace(int64_t M, int64_t N, int64_t K) {
  return M > 0 && N > 0 && K > 0 ? tail_bytes(M, K, N) : 0;
}

static int linear_bwd_x_dense(const uint16_t* grad_y, const uint16_t* w, const uint16_t* lora_gt,
                              const uint16_t* lora_a, int rank, const uint16_t* sw_pre,
                              uint16_t* grad_x, void* workspace, size_t workspace_bytes, int64_t M,
                              int64_t N, int64_t K, void* stream, const char* what) {
  PLZ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "%s: negative shape", what);
  PLZ_REQUIRE(K % 8 == 0 && N % 8 == 0, "%s: K and N must be multiples of 8", what);
  PLZ_REQUIRE(rank >= 0 && rank <= BK && rank % 8 == 0,
              "%s: rank (%d) must be a multiple of 8 in [0, 64]", what, rank);
  if (M == 0 || K == 0) return PLZ_OK;
  PLZ_REQUIRE(grad_y && w && grad_x && a16(grad_y) && a16(w),
              "%s: grad_y, w, grad_x must be non-null; grad_y, w aligned", what);
  PLZ_REQUIRE(rank == 0 || (lora_gt && lora_a && a16(lora_gt) && a16(lora_a)),
              "%s: rank > 0 needs 16-byte aligned lora_gt and lora_a", what);
  Args g = {};
  g.a = grad_y; g.lda = N;
  g.b = w; g.ldb = K;  // B(j=k, r=n) = w[n, k]   (Col tile)
  g.I = M; g.J = K; g.R = N;
  g.a2 = lora_gt; g.b2 = lora_a; g.R2 = rank;
  g.c = grad_x; g.ldc = sw_pre ? 2 * K : K; g.alpha = 1.f;
  g.sw_pre = sw_pre; g.ld_sw = 2 * K;
  g.group = kDenseGroup;
  const int rc = set_tail(g, workspace, workspace_bytes, what);
  if (rc != PLZ_OK) return rc;
  return launch<OP_ROW, OP_COL, EPI_BF16>(g, 1, (hipStream_t)stream, what);
}

int plz_linear_bwd_x_dense(const uint16_t* grad_y, const uint16_t* w, const uint16_t* lora_gt,
                           const uint16_t* lora_a, int rank, uint16_t* grad_x, void* workspace,
                           size_t workspace_bytes, int64_t M, int64_t N, int64_t K,
                           void* stream) {
  return linear_bwd_x_dense(grad_y, w, lora_gt, lora_a, rank, nullptr, grad_x, workspace,
                            workspace_bytes, M, N, K, stream, "plz_linear_bwd_x_dense");
}

int plz_linear_bwd_x_dense_swiglu(const uint16_t* grad_y, const uint16_t* w,
                                  const uint16_t* lora_gt, const uint16_t* lora_a, int rank,
                                  const uint16_t* gate_up, uint16_t* grad_gate_up, void* workspace,
                                  size_t workspace_bytes, int64_t M, int64_t N, int64_t K,
                                  void* stream) {
  PLZ_REQUIRE(M == 0 || K == 0 || (gate_up && grad_gate_up && a16(gate_up) && a16(grad_gate_up)),
              "plz_linear_bwd_x_dense_swiglu: gate_up and grad_gate_up must be non-null, "
              "16-byte aligned");
  return linear_bwd_x_dense(grad_y, w, lora_gt, lora_a, rank, gate_up, grad_gate_up, workspace,
                            workspace_bytes, M, N, K, stream, "plz_linear_bwd_x_dense_swiglu");
}

size_t plz_soft_bwd_workspace(int64_t M, int64_t N, int64_t K) {
  if (N <= 0 || K <= 0) return 0;
  const int z = soft_splits(M, N, K);
  return soft_pal_bytes(N, K) + (z > 1 ? (size_t)z * N * K * sizeof(float) : 0);
}

// wg.rank > 0: the LoRA weight gradients from the same dW tiles (their partials in wg.part_a /
// wg.part_b, past the soft workspace), summed with the palette by pal_wg_reduce_kernel
static int soft_bwd(const uint16_t* x, const uint16_t* grad_y, const uint16_t* logits,
                    int logits_dtype, bool gen, const float* noise, uint64_t seed, uint64_t offset,
                    const float* palette, float tau, int scale_grad_by_inv_tau,
                    uint16_t* grad_logits, float* grad_palette, void* workspace,
                    size_t workspace_bytes, int64_t M, int64_t N, int64_t K, void* stream,
                    const WgradArgs& wg = WgradArgs(), float* gsq = nullptr,
                    const uint16_t* probs = nullptr) {
  PLZ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "plz_soft_bwd: negative shape");
  PLZ_REQUIRE(K % 256 == 0, "plz_soft_bwd: K (%lld) must be a multiple of 256", (long long)K);
  PLZ_REQUIRE(N % 8 == 0, "plz_soft_bwd: N (%lld) must be a multiple of 8", (long long)N);
  PLZ_REQUIRE(logits_dtype == PLZ_DT_BF16 || logits_dtype == PLZ_DT_FP16,
              "plz_soft_bwd: logits dtype must be bf16 or fp16");
  PLZ_REQUIRE(tau > 0.f, "plz_soft_bwd: tau must be positive");
  if (N == 0 || K == 0) return PLZ_OK;
  PLZ_REQUIRE((logits || probs) && palette && grad_logits && grad_palette &&
                  (gen || noise || probs),
              "plz_soft_bwd: null pointer");
  if (M == 0) {  // empty reduction: every gradient is zero
    zero_async(grad_logits, (size_t)N * K * 4 * 2, (hipStream_t)stream);
    zero_async(grad_palette, (size_t)N * (K / 256) * 16, (hipStream_t)stream);
    if (wg.rank > 0) {
      const size_t esz = wg.out_bf16 ? 2 : 4;
      zero_async(wg.grad_a, (size_t)wg.rank * K * esz, (hipStream_t)stream);
      zero_async(wg.grad_b, (size_t)N * wg.rank * esz, (hipStream_t)stream);
    }
    if (gsq) zero_async(gsq, (size_t)N * (K / 128) * sizeof(float), (hipStream_t)stream);
    return check_launch("plz_soft_bwd");
  }
  PLZ_REQUIRE(x && grad_y, "plz_soft_bwd: null pointer");
  PLZ_REQUIRE(a16(x) && a16(grad_y) && a16(logits) && a16(noise) && a16(palette) &&
                  a16(grad_logits) && a16(probs),
              "plz_soft_bwd: operands must be 16-byte aligned");
  const size_t need = plz_soft_bwd_workspace(M, N, K);
  if (!workspace || workspace_bytes < need) {
    set_error("plz_soft_bwd: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
    return PLZ_EWORKSPACE;
  }
  const int z = soft_splits(M, N, K);
  Args g = {};
  g.a = grad_y; g.lda = N;
  g.b = x; g.ldb = K;
  g.pal = palette; g.Nw = N; g.Kw = K;
  g.I = N; g.J = K; g.R = M; g.r_split = z > 1 ? split_len(M, z) : (M > 0 ? M : 1);
  g.partial = reinterpret_cast<float*>(workspace);
  g.acc_ws = z > 1 ? reinterpret_cast<float*>((char*)workspace + soft_pal_bytes(N, K)) : nullptr;
  g.logits = logits; g.noise = noise; g.inv_tau = 1.f / tau;
  g.noise_seed = seed; g.noise_offset = offset;
  g.glog_scale = scale_grad_by_inv_tau ? 1.f / tau : 1.f;
  g.grad_logits = grad_logits; g.logits_f16 = logits_dtype == PLZ_DT_FP16;
  g.group = K > N ? -1 : 1;  // walk the larger operand's panels, as the hard grad_palette GEMM
  g.wg_r = wg.rank;
  g.wg_a = wg.lora_a; g.wg_b = wg.lora_b;
  g.wg_part_a = wg.part_a; g.wg_part_b = wg.part_b;
  g.gsq = gsq;
  g.pin = probs;
  int rc;
  if (z == 1) {
    rc = launch<OP_COL, OP_COL, EPI_SOFT>(g, 1, (hipStream_t)stream, "plz_soft_bwd");
  } else {
    rc = launch<OP_COL, OP_COL, EPI_F32>(g, z, (hipStream_t)stream, "plz_soft_bwd");
    if (rc != PLZ_OK) return rc;
    const int64_t items = N * (K / 128);
    hipLaunchKernelGGL(soft_split_epilogue_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256),
                       0, (hipStream_t)stream, g, z);
    rc = check_launch("plz_soft_bwd/epilogue");
  }
  if (rc != PLZ_OK) return rc;
  const int64_t G = K / 256, n_out = N * G;
  const int pal_blocks = (int)((n_out + 255) / 256);
  if (wg.rank > 0) {
    WgRed w;
    w.pa = wg.part_a; w.pb = wg.part_b; w.ga = wg.grad_a; w.gb = wg.grad_b;
    w.la = (int64_t)wg.rank * K; w.lb = N * wg.rank; w.N = N;
    w.na = z * (int)((N + TILE - 1) / TILE); w.nb = z * (int)((K + TILE - 1) / TILE);
    w.r = wg.rank; w.out_bf16 = wg.out_bf16; w.scale = wg.scale;
    const int wg_blocks = (int)((w.la + w.lb + 255) / 256);
    hipLaunchKernelGGL(pal_wg_reduce_kernel, dim3((unsigned)(pal_blocks + wg_blocks)), dim3(256),
                       0, (hipStream_t)stream, g.partial, grad_palette, N, G, 1, pal_blocks, w);
  } else {
    hipLaunchKernelGGL(reduce_pal_kernel, dim3((unsigned)pal_blocks), dim3(256), 0,
                       (hipStream_t)stream, g.partial, grad_palette, N, G, 1);
  }
  return check_launch("plz_soft_bwd/reduce");
}

int plz_soft_bwd(const uint16_t* x, const uint16_t* grad_y, const uint16_t* logits,
                 int logits_dtype, const float* noise, const float* palette, float tau,
                 int scale_grad_by_inv_tau, uint16_t* grad_logits, float* grad_palette,
                 void* workspace, size_t workspace_bytes, int64_t M, int64_t N, int64_t K,
                 void* stream) {
  return soft_bwd(x, grad_y, logits, logits_dtype, false, noise, 0, 0, palette, tau,
                  scale_grad_by_inv_tau, grad_logits, grad_palette, workspace, workspace_bytes, M,
                  N, K, stream);
}

int plz_soft_bwd_probs(const uint16_t* x, const uint16_t* grad_y, const uint16_t* probs,
                       const float* palette, float tau, int scale_grad_by_inv_tau,
                       uint16_t* grad_logits, int grad_logits_dtype, float* grad_palette,
                       void* workspace, size_t workspace_bytes, int64_t M, int64_t N, int64_t K,
                       void* stream) {
  PLZ_REQUIRE(N == 0 || K == 0 || probs, "plz_soft_bwd_probs: null probs");
  return soft_bwd(x, grad_y, nullptr, grad_logits_dtype, false, nullptr, 0, 0, palette, tau,
                  scale_grad_by_inv_tau, grad_logits, grad_palette, workspace, workspace_bytes, M,
                  N, K, stream, WgradArgs(), nullptr, probs);
}

size_t plz_soft_bwd_lora_workspace(int64_t M, int64_t N, int64_t K, int rank) {
  if (N <= 0 || K <= 0 || rank <= 0) return plz_soft_bwd_workspace(M, N, K);
  const int z = soft_splits(M, N, K);
  return align256(plz_soft_bwd_workspace(M, N, K)) +
         align256(wg_part_a_floats(z, N, K, rank) * sizeof(float)) +
         align256(wg_part_b_floats(z, N, K, rank) * sizeof(float));
}

int plz_soft_bwd_lora(const uint16_t* x, const uint16_t* grad_y, const uint16_t* logits,
                      int logits_dtype, const float* noise, uint64_t seed, uint64_t offset,
                      const uint16_t* probs, const float* palette, float tau,
                      int scale_grad_by_inv_tau,
                      const uint16_t* lora_a, const uint16_t* lora_b, int rank, float scale,
                      uint16_t* grad_logits, float* grad_palette, void* grad_a, void* grad_b,
                      int grads_dtype, float* grad_sq, void* workspace, size_t workspace_bytes,
                      int64_t M, int64_t N, int64_t K, void* stream) {
  const char* what = "plz_soft_bwd_lora";
  PLZ_REQUIRE(((uintptr_t)grad_sq & 3) == 0, "%s: grad_sq must be 4-byte aligned", what);
  PLZ_REQUIRE(rank > 0 && rank <= 32 && rank % 8 == 0,
              "%s: rank (%d) must be a multiple of 8 in [8, 32]", what, rank);
  PLZ_REQUIRE(grads_dtype == PLZ_DT_BF16 || grads_dtype == PLZ_DT_FP32,
              "%s: grads_dtype must be PLZ_DT_BF16 or PLZ_DT_FP32", what);
  PLZ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "%s: negative shape", what);
  if (N == 0 || K == 0) return lora_grads_of_empty_weight(grad_a, grad_b, rank, grads_dtype, N,
                                                          K, (hipStream_t)stream, what);
  PLZ_REQUIRE(lora_a && lora_b && grad_a && grad_b && a16(lora_a) && a16(lora_b),
              "%s: lora_a, lora_b, grad_a, grad_b must be non-null; lora_a, lora_b 16-byte "
              "aligned", what);
  const size_t need = plz_soft_bwd_lora_workspace(M, N, K, rank);
  if (!workspace || !a16(workspace) || workspace_bytes < need) {
    set_error("%s: workspace of %zu bytes (16-byte aligned) needed, %zu given", what, need,
              workspace_bytes);
    return PLZ_EWORKSPACE;
  }
  const int z = soft_splits(M, N, K);
  uint8_t* w = static_cast<uint8_t*>(workspace);
  WgradArgs wg;
  wg.lora_a = lora_a; wg.lora_b = lora_b; wg.rank = rank; wg.scale = scale;
  wg.grad_a = grad_a; wg.grad_b = grad_b; wg.out_bf16 = grads_dtype == PLZ_DT_BF16;
  const size_t soft_bytes = align256(plz_soft_bwd_workspace(M, N, K));
  wg.part_a = reinterpret_cast<float*>(w + soft_bytes);
  wg.part_b = reinterpret_cast<float*>(
      w + soft_bytes + align256(wg_part_a_floats(z, N, K, rank) * sizeof(float)));
  return soft_bwd(x, grad_y, logits, logits_dtype, noise == nullptr, noise, seed, offset, palette,
                  tau, scale_grad_by_inv_tau, grad_logits, grad_palette, workspace,
                  soft_bytes, M, N, K, stream, wg, grad_sq, probs);
}

int plz_soft_bwd_philox(const uint16_t* x, const uint16_t* grad_y, const uint16_t* logits,
                        int logits_dtype, uint64_t seed, uint64_t offset, const float* palette,
                        float tau, int scale_grad_by_inv_tau, uint16_t* grad_logits,
                        float* grad_palette, void* workspace, size_t workspace_bytes, int64_t M,
                        int64_t N, int64_t K, void* stream) {
  return soft_bwd(x, grad_y, logits, logits_dtype, true, nullptr, seed, offset, palette, tau,
                  scale_grad_by_inv_tau, grad_logits, grad_palette, workspace, workspace_bytes, M,
                  N, K, stream);
}

}  // extern "C"
