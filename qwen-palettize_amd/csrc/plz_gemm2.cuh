// Large-tile MFMA GEMM core for gfx950 (the M = 16384 training shapes).
//
// C[I,J] = sum_r A(i,r) B(j,r), bf16 operands, fp32 accumulation, 512 threads = 8 wave64s
// in a 2x4 grid (two per SIMD, so that one wave's LDS and memory waits are covered by the
// other's MFMAs), workgroup tile 256x256, 128x64 per wave (4x2 blocks of
// v_mfma_f32_32x32x16_bf16, 128 accumulator registers), reduction stages of BK = 64,
// double-buffered in LDS (2 x 64 KB).
//
// Each operand tile sits in LDS in one of two layouts:
//   Row tile  [row][r]: 16-byte chunks of 8 consecutive r, chunk index XOR ((row >> 1) & 7).
//             Fragments: one ds_read_b128 per lane (row = lane%32, chunk = 2*ks + lane/32),
//             free of bank conflicts with this swizzle.
//   Col tile  [r][row]: the operand's own memory order when rows are contiguous
//             (MN-contiguous: grad_y and x in dW, W in grad_x). Chunks of 8 consecutive
//             rows, chunk index XOR col_swz(r). Fragments: two ds_read_b64_tr_b16 per lane.
//             Within each 16-lane group lane i points at rows 4*(i%4)..+3 of reduction
//             index kbase + i/4; the instruction hands lane j elements j, j+16, j+32, j+48
//             of the group's 64 loaded values, i.e. row j at kbase..kbase+3 -- the MFMA
//             operand order (k-slots 8*(lane/32) + s), the same as a Row-tile fragment.
// Dense operands are copied global -> LDS by global_load_lds_dwordx4 (no VGPR staging;
// lane l of an instruction writes LDS bytes base + 16*l, so the swizzle is applied to the
// global address each lane reads). The palettized operand W[n,k] is dequantised by all
// threads into a Row tile (forward, rows = n) or a Col tile (grad_x, rows = k, reduction n).
#pragma once
#include "plz_common.h"

namespace plz {
namespace g2 {

constexpr int BK = 64;
constexpr int TILE = 256;            // BI = BJ
constexpr int TILE_BYTES = TILE * BK * 2;  // 32 KB per operand per stage
constexpr int NTHR = 512;            // 8 waves
constexpr int WAVES_I = 2, WAVES_J = 4;
constexpr int WT_I = TILE / WAVES_I / 32;  // 32x32 MFMA blocks per wave along i (4)
constexpr int WT_J = TILE / WAVES_J / 32;  // ... along j (2)
constexpr int COPY_INSTS = TILE * BK / 8 / NTHR;  // 16-byte copies per thread per operand (4)
constexpr int RING_SLOTS = 5;  // operand tiles in a copy ring (5 x 32 KB = 160 KB of LDS)

// Workgroup barrier after this wave's LDS reads have completed, without the release fence of
// __syncthreads() (which waits for every outstanding copy): the caller's wait_vmcnt decides
// which copies must have landed. The empty asm statements keep the compiler from moving
// memory accesses across it.
__device__ __forceinline__ void stage_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xF | (3 << 14) | (7 << 4));  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// wait until at most N vector-memory operations of this wave are outstanding
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
typedef __attribute__((address_space(3))) uint8_t lds_u8;

__device__ __forceinline__ int row_swz(int row) { return (row >> 1) & 7; }
__device__ __forceinline__ int row_chunk(int row, int c) { return row * (BK / 8) + (c ^ row_swz(row)); }
// kr ^ 4*(kr & 3): the tr16 fragment reads (4 consecutive kr x 4 chunks per 32 lanes) and
// the 16-byte dequant stores (16 consecutive kr per wave) are both free of bank conflicts
// on gfx950 (measured with SQ_LDS_BANK_CONFLICT).
__device__ __forceinline__ int col_swz(int kr) { return (kr ^ ((kr & 3) << 2)) & 15; }
__device__ __forceinline__ int col_chunk(int kr, int c) { return kr * (TILE / 8) + (c ^ col_swz(kr)); }

struct Args {
  const uint16_t* a; int64_t lda;   // dense A
  const uint16_t* b; int64_t ldb;   // dense B
  const int32_t* packed; const float* pal; int64_t Nw, Kw;  // palettized operand
  int64_t I, J, R, r_split;
  // rank-r second segment (R2 <= BK): A2 row-major [I, R2]; B2 row-major [J, R2] when the
  // main B is a Row tile, reduction-major [R2, J] when it is a Col tile
  const uint16_t* a2; const uint16_t* b2; int R2;
  // epilogue
  void* c; int64_t ldc; const uint16_t* bias; float alpha; float* partial;
  // EPI_BF16: bf16 [I, J] (row stride ldres) added to the stored bf16 values and rounded
  // again, as a bf16 tensor add after the GEMM would (NULL: none)
  const uint16_t* res; int64_t ldres;
  // EPI_BF16: the [gate | up] pre-activations [I, 2J] (row stride ld_sw) of a SwiGLU whose
  // output gradient this GEMM computes; the stored values are then the SwiGLU's gate / up
  // gradients, into c [I, 2J] (NULL: none)
  const uint16_t* sw_pre; int64_t ld_sw;
  const uint16_t* logits; const float* noise; float inv_tau, glog_scale; uint16_t* grad_logits;
  uint64_t noise_seed, noise_offset;  // noise == nullptr: Philox at noise_offset + n*K + k
  int logits_f16;
  float* acc_ws;  // EPI_F32: partial dW rows of each reduction split, [split][I][J] fp32
  // EPI_PAL with wg_r > 0: the LoRA weight gradients from the dW tile (wg_a = lora_a [r, K],
  // wg_b = lora_b [N, r]); partials [split][tiles_i][r][K] and [split][tiles_j][r][N]
  const uint16_t* wg_a; const uint16_t* wg_b; int wg_r;
  float* wg_part_a; float* wg_part_b;
  // EPI_BF16 tail split: tiles [tail_first, tiles) run as tail_split reduction parts of
  // tail_len each, whose fp32 accumulators go to tail_ws (accumulator layout, 256 KB per part);
  // tail_reduce_kernel sums them and stores the tiles
  int tail_first, tail_split;
  int64_t tail_len;
  float* tail_ws;
  int tiles_i, tiles_j;
  int group;  // tile-rows walked together (1: consecutive workgroups share the A panel);
              // < 0: column-major walk (consecutive workgroups share the B panel)
  // EPI_SWIGLU over a [gate | up] weight: b_half = F gate rows, so that a tile's 256 columns
  // are gate rows j0/2 .. j0/2+127 and the matching up rows F + j0/2 .. (half_row); c2, when
  // set, receives the pre-activations [I, 2F] in that natural layout (row pitch ldc2)
  int64_t b_half;
  uint16_t* c2; int64_t ldc2;
  // soft epilogues: the sum of squares of each item's stored grad_logits (512 values: row n,
  // 128 k), [I][J / 128] fp32, or NULL
  float* gsq;
  // soft epilogues: the forward's P [I][J][4] fp16, read in place of logits + noise, or NULL
  const uint16_t* pin;
};

// B row (and output column) of the tile-local logical column j when b_half > 0: the first 128
// of every 256 columns are gate rows, the next 128 the up rows at the same offset
__device__ __forceinline__ int64_t half_row(int64_t j, int64_t half) {
  return half > 0 ? (j >> 8) * 128 + (j & 127) + ((j & 128) ? half : 0) : j;
}

// ---- dense operand copy, global -> LDS ---------------------------------------------------
// Each lane's byte offsets of its COPY_INSTS 16-byte chunks are fixed for a tile; a stage adds
// a wave-uniform offset (the buffer instruction's soffset), so the main loop's copies need no
// per-lane address arithmetic. The host checks that every operand spans < 4 GiB.
struct TileDma {
  BufRsrc r;
  uint32_t off[COPY_INSTS];
};
// Row tile from p[row*ld + r] (r contiguous): 2048 chunks; lane l of an instruction writes
// LDS bytes base + 16*l, so the swizzle is applied to the global address each lane reads.
// Stage offset: 2*r0 bytes.
__device__ __forceinline__ TileDma row_tile_dma(const uint16_t* p, int64_t ld, int64_t row0,
                                                int64_t nrows, int64_t half = 0) {
  TileDma d;
  d.r = make_rsrc(p, (uint32_t)(nrows * ld * 2));
#pragma unroll
  for (int it = 0; it < COPY_INSTS; ++it) {
    const int pch = it * NTHR + threadIdx.x;         // physical chunk written by this lane
    const int row = pch >> 3, c = (pch & 7) ^ row_swz(row);
    int64_t gr = row0 + row;
    gr = gr < nrows ? gr : nrows - 1;                 // rows past the end: any valid row
    gr = half_row(gr, half);
    d.off[it] = (uint32_t)((gr * ld + c * 8) * 2);
  }
  return d;
}
// Col tile from p[r*ld + row] (rows contiguous): 64 reduction rows x 32 chunks. Stage offset:
// 2*r0*ld bytes.
__device__ __forceinline__ TileDma col_tile_dma(const uint16_t* p, int64_t ld, int64_t row0,
                                                int64_t nrows, int64_t rtotal) {
  TileDma d;
  d.r = make_rsrc(p, (uint32_t)(rtotal * ld * 2));
#pragma unroll
  for (int it = 0; it < COPY_INSTS; ++it) {
    const int pch = it * NTHR + threadIdx.x;
    const int kr = pch >> 5, c = (pch & 31) ^ col_swz(kr);
    int64_t gr = row0 + c * 8;
    gr = gr < nrows ? gr : 0;                          // chunks past the end: any valid chunk
    d.off[it] = (uint32_t)((kr * ld + gr) * 2);
  }
  return d;
}
__device__ __forceinline__ void tile_copy(lds_u8* lds, const TileDma& d, uint32_t soff) {
  const int wbase = __builtin_amdgcn_readfirstlane((threadIdx.x >> 6) * 1024);
#pragma unroll
  for (int it = 0; it < COPY_INSTS; ++it)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(d.r, lds + it * NTHR * 16 + wbase, 16, d.off[it],
                                             soff, 0, 0);
}

// ---- palettized operand: one thread per (row n, 32 k) -------------------------------------
struct LutRegs {
  uint2 q;   // two packed words = 32 indices
  float4 p;  // the palette of their group
};
// Forward: tile rows are n (256 rows x 64 k); thread t owns row lut_row_of(t % 256), half
// t / 256 of the 64 k. The row permutation within groups of 8 makes the 4 lanes of each
// store group write rows with distinct (row >> 1) & 3, i.e. distinct 16-byte columns of a
// 64-byte window (no bank conflicts).
__device__ __forceinline__ int lut_row_of(int t) {
  return (t & ~7) | ((t & 3) << 1) | ((t >> 2) & 1);
}
__device__ __forceinline__ void lut_row_load(const Args& g, int64_t n0, int64_t k0, LutRegs& r) {
  const int64_t n = n0 + lut_row_of(threadIdx.x & 255);
  const int h = threadIdx.x >> 8;
  r.q = make_uint2(0, 0);
  r.p = make_float4(0.f, 0.f, 0.f, 0.f);
  if (n < g.Nw) {
    r.q = *reinterpret_cast<const uint2*>(g.packed + n * (g.Kw / 16) + k0 / 16 + 2 * h);
    r.p = *reinterpret_cast<const float4*>(g.pal + (n * (g.Kw / 256) + k0 / 256) * 4);
  }
}
// part = word of the thread's 32 k: two 16-byte chunks
__device__ __forceinline__ void lut_row_store_part(uint4* lds, const LutRegs& r, int part) {
  const PalLut t = make_lut(r.p.x, r.p.y, r.p.z, r.p.w);
  const int row = lut_row_of(threadIdx.x & 255), cb = 4 * (threadIdx.x >> 8);
  uint32_t o[8];
  dequant16(part == 0 ? r.q.x : r.q.y, t, o);
  lds[row_chunk(row, cb + 2 * part)] = make_uint4(o[0], o[1], o[2], o[3]);
  lds[row_chunk(row, cb + 2 * part + 1)] = make_uint4(o[4], o[5], o[6], o[7]);
}
__device__ __forceinline__ void lut_row_store(uint4* lds, const LutRegs& r) {
  lut_row_store_part(lds, r, 0);
  lut_row_store_part(lds, r, 1);
}
// grad_x: tile rows are k (256), reduction n (64). Thread t owns n = n0 + t%64 and
// k = k0 + 32*(t/64) .. +32: 4 consecutive lanes store 4 consecutive reduction rows, whose
// col_swz low bits differ (no bank conflicts). The tile's k range lies in one palette group
// (k0 % 256 == 0).
__device__ __forceinline__ int lut_col_kr() { return threadIdx.x & 63; }
__device__ __forceinline__ int lut_col_seg() { return threadIdx.x >> 6; }
__device__ __forceinline__ void lut_col_load(const Args& g, int64_t k0, int64_t n0, LutRegs& r) {
  const int64_t n = n0 + lut_col_kr();
  const int64_t k = k0 + 32 * lut_col_seg();
  r.q = make_uint2(0, 0);
  r.p = make_float4(0.f, 0.f, 0.f, 0.f);
  if (n < g.Nw && k < g.Kw) {
    r.q = *reinterpret_cast<const uint2*>(g.packed + n * (g.Kw / 16) + k / 16);
    r.p = *reinterpret_cast<const float4*>(g.pal + (n * (g.Kw / 256) + k / 256) * 4);
  }
}
__device__ __forceinline__ void lut_col_store_part(uint4* lds, const LutRegs& r, int part) {
  const PalLut t = make_lut(r.p.x, r.p.y, r.p.z, r.p.w);
  const int kr = lut_col_kr(), cb = 4 * lut_col_seg();
  uint32_t o[8];
  dequant16(part == 0 ? r.q.x : r.q.y, t, o);
  lds[col_chunk(kr, cb + 2 * part)] = make_uint4(o[0], o[1], o[2], o[3]);
  lds[col_chunk(kr, cb + 2 * part + 1)] = make_uint4(o[4], o[5], o[6], o[7]);
}
__device__ __forceinline__ void lut_col_store(uint4* lds, const LutRegs& r) {
  lut_col_store_part(lds, r, 0);
  lut_col_store_part(lds, r, 1);
}

// Forward, register-dequant variant: the stage's palettized operand travels raw, 256 rows x
// (4 packed words = 64 k | the row's palette), one 16-byte global->LDS copy per thread
// (threads 0..255 the words of row t, threads 256..511 the palette of row t-256). Each wave
// then dequantises its own B fragments in registers: no dequantised tile is written to or
// read from LDS (16-byte LDS writes cost ~2.7x the reads per byte on gfx950).
constexpr int LUT_RAW_PAL = 256 * 16;  // byte offset of the palettes in the raw slot
struct LutDma {
  BufRsrc r;
  uint32_t off;
};
__device__ __forceinline__ LutDma lut_raw_dma(const Args& g, int64_t n0) {
  const int t = threadIdx.x, r = t & 255;
  int64_t n = n0 + r;
  n = n < g.Nw ? n : g.Nw - 1;  // rows past the end: any valid row (never stored)
  LutDma d;
  if (__builtin_amdgcn_readfirstlane(t >> 8) == 0) {
    d.r = make_rsrc(g.packed, (uint32_t)(g.Nw * (g.Kw / 4)));
    d.off = (uint32_t)(n * (g.Kw / 16) * 4);
  } else {
    d.r = make_rsrc(g.pal, (uint32_t)(g.Nw * (g.Kw / 256) * 16));
    d.off = (uint32_t)(n * (g.Kw / 256) * 16);
  }
  return d;
}
// stage at k0: 16 bytes of words (k0/4 bytes into the row) or the row's palette of group k0/256
__device__ __forceinline__ void copy_lut_raw(lds_u8* lds, const LutDma& d, int64_t k0) {
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t soff = w < 4 ? (uint32_t)(k0 / 4) : (uint32_t)((k0 / 256) * 16);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(d.r, lds + w * 1024, 16, d.off, soff, 0, 0);
}

// ---- fragments (v_mfma_f32_32x32x16_bf16: lane l holds row l%32, k-slots 8*(l/32)..+7) --
typedef float f32x16 __attribute__((ext_vector_type(16)));

// One ds_read_b128 per lane: with the row swizzle the 64 lanes hit no bank twice (two
// ds_read_b64 halves of the same chunks conflict 2-way: half of every chunk sits in the
// same banks).
__device__ __forceinline__ bf16x8 frag_row(const uint4* lds, int rowbase, int ks, int lane) {
  const int ch = row_chunk(rowbase + (lane & 31), 2 * ks + (lane >> 5));
  return __builtin_bit_cast(bf16x8, lds[ch]);
}
// Row tile fragment of an explicit chunk per lane (8 consecutive r of row rowbase + lane%32).
__device__ __forceinline__ bf16x8 frag_row_chunk(const uint4* lds, int rowbase, int chunk, int lane) {
  return __builtin_bit_cast(bf16x8, lds[row_chunk(rowbase + (lane & 31), chunk)]);
}
// Col tile: per 16-lane group j = lane/16 the rows 16*(j&1)..+15 at k-group j>>1.
// col_swz sees only the low 4 bits of the reduction row, so k-step ks moves both reads by
// the constant 16*ks rows: the lane-dependent part is formed for ks = 0 and the k-step
// becomes the read instruction's immediate offset (one address per fragment and stage
// instead of one per k-step).
__device__ __forceinline__ bf16x8 frag_col(const lds_u8* lds, int rowbase, int ks, int lane) {
  const int j = lane >> 4, i = lane & 15, t = i >> 2, q = i & 3;
  const int row = rowbase + 16 * (j & 1) + 4 * q;
  const int kr1 = 8 * (j >> 1) + t, kr2 = kr1 + 4;
  const int c = row >> 3, off = (row & 7) * 2;
  const lds_u8* kb = lds + ks * (16 * TILE * 2);
  const v4i16 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16*)(kb + col_chunk(kr1, c) * 16 + off));
  const v4i16 v2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16*)(kb + col_chunk(kr2, c) * 16 + off));
  typedef short v8i16 __attribute__((ext_vector_type(8)));
  const v8i16 v = __builtin_shufflevector(v1, v2, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, v);
}

// Read addresses of a Col tile's fragments for one stage: two per 32-row block, at k-step 0.
// The empty asm statement makes each address an opaque register value, so that the k-steps
// use the read instruction's immediate offset (+16*ks rows) and the compiler does not keep
// one precomputed address per k-step and re-add the stage's slot base to every one of them.
template <int NB>
struct ColBases {
  uint32_t p1[NB], p2[NB];
};
template <int NB>
__device__ __forceinline__ void col_bases(const lds_u8* lds, int rowbase0, int lane,
                                          ColBases<NB>& cb) {
  const int j = lane >> 4, i = lane & 15, t = i >> 2, q = i & 3;
  const int kr1 = 8 * (j >> 1) + t, kr2 = kr1 + 4;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int row = rowbase0 + 32 * b + 16 * (j & 1) + 4 * q;
    const int c = row >> 3, off = (row & 7) * 2;
    uint32_t p1 = (uint32_t)(uintptr_t)lds + col_chunk(kr1, c) * 16 + off;
    uint32_t p2 = (uint32_t)(uintptr_t)lds + col_chunk(kr2, c) * 16 + off;
    asm volatile("" : "+v"(p1), "+v"(p2));
    cb.p1[b] = p1;
    cb.p2[b] = p2;
  }
}
__device__ __forceinline__ bf16x8 frag_col_at(uint32_t p1, uint32_t p2, int ks) {
  const v4i16 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16*)(uintptr_t)(p1 + ks * (16 * TILE * 2)));
  const v4i16 v2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16*)(uintptr_t)(p2 + ks * (16 * TILE * 2)));
  typedef short v8i16 __attribute__((ext_vector_type(8)));
  const v8i16 v = __builtin_shufflevector(v1, v2, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, v);
}

// ---- work-item map and launch planning (shared by the kernels and a host-side check) -------
// A launch has tiles_i x tiles_j output tiles and gridDim.z reduction splits; a tail-split
// launch (bf16 epilogue, tail_split > 1) runs its first tail_first tiles whole and each later
// tile as tail_split reduction parts in the last, partial wave.
struct Item {
  int zsl, bid, part;  // reduction split, tile index, tail part
  bool tail_part;
};
// Workgroups go to the 8 XCDs round-robin by linear id, and each XCD has its own L2: the
// (split, tile) items are renumbered so that XCD x runs one contiguous range of them.
__host__ __device__ __forceinline__ Item map_item(int tiles, bool tail, int tail_first,
                                                  int tail_split, int bx, int bz, int gz) {
  Item it{0, 0, 0, false};
  if (tail && bx >= tail_first) {
    const int u = bx - tail_first;
    it.bid = tail_first + u / tail_split;
    it.part = u % tail_split;
    it.tail_part = true;
    return it;
  }
  const int whole = tail ? tail_first : tiles;
  const int total = whole * gz;
  const int lin = bx + whole * bz;
  const int xcd = lin % 8, q8 = total / 8, r8 = total % 8;
  const int item = xcd * q8 + (xcd < r8 ? xcd : r8) + lin / 8;
  it.zsl = item / whole;
  it.bid = item % whole;
  return it;
}
// Tile of item bid: tile-columns are walked within groups of `group` tile-rows, or, with
// group < 0, tile-rows within each tile-column (column-major).
__host__ __device__ __forceinline__ void tile_coords(int group, int tiles_i, int tiles_j, int bid,
                                                     int& tile_i, int& tile_j) {
  if (group < 0) {
    tile_i = bid % tiles_i;
    tile_j = bid / tiles_i;
    return;
  }
  const int per_group = group * tiles_j;
  const int first_i = (bid / per_group) * group;
  const int gsz = tiles_i - first_i < group ? tiles_i - first_i : group;
  tile_i = first_i + (bid % per_group) % gsz;
  tile_j = (bid % per_group) / gsz;
}

// reduction length of each of z splits, a whole number of stages
inline int64_t split_len(int64_t R, int z) {
  const int64_t per = (R + z - 1) / z;
  return (per + BK - 1) / BK * BK;
}

// Reduction splits of the grad_palette GEMM on C CUs. Its time is modelled as (waves of
// `tiles * z` workgroups) x (stages per split + the per-tile prologue and epilogue, worth
// about 4 stages); the smallest modelled time wins. On the Qwen-4B shapes at M = 16384 this
// picks 2 splits for the MLP shapes, 3 for q/o and 6 for k/v (measured: k/v 631 -> 861
// TFLOP/s against the fill-the-waves choice of 19 splits).
inline int palette_splits_on(int64_t M, int64_t N, int64_t K, int64_t C) {
  const int64_t tiles = ((N + TILE - 1) / TILE) * ((K + TILE - 1) / TILE);
  if (tiles == 0 || M <= 0) return 1;
  int best = 1;
  double best_t = 1e300;
  for (int z = 1; z <= 32; ++z) {
    const int64_t len = split_len(M, z);
    if (z > 1 && (len < 8 * BK || (int64_t)(z - 1) * len >= M)) break;  // >= 8 stages, none empty
    const double t = (double)((tiles * z + C - 1) / C) * ((double)len / BK + 4.0);
    if (t < best_t * 0.99) {
      best_t = t;
      best = z;
    }
  }
  return best;
}

// Tail split of a one-workgroup-per-tile GEMM (one workgroup per CU) on C CUs: when the tiles
// leave a last, partial wave of rem < C/2 tiles, those tiles run as s = C/rem reduction parts
// each, so the last wave takes 1/s of a tile-time. Taken when the time saved (2.15 us per
// 256x256x64 stage) exceeds the cost of the fp32 partials (256 KB per part written and read
// at ~5 TB/s) and one more launch.
struct TailPlan {
  int first = 0, split = 1;
  int64_t len = 0;
};
inline TailPlan tail_plan_on(int64_t I, int64_t J, int64_t R, int64_t C) {
  TailPlan t;
  const int64_t tiles = ((I + TILE - 1) / TILE) * ((J + TILE - 1) / TILE);
  const int64_t rem = tiles % C;
  if (rem == 0 || R <= 0) return t;
  const int64_t stages = (R + BK - 1) / BK;
  int s = (int)(C / rem);
  s = s < 16 ? s : 16;
  while (s > 1 && (stages / s < 8 || (int64_t)(s - 1) * split_len(R, s) >= R)) --s;
  if (s < 2) return t;
  const double gain = (double)stages * 2.15 * (1.0 - 1.0 / s);
  const double cost = (double)rem * s * 2.0 * TILE * TILE * 4 / 5.0e6 + 5.0;
  if (gain <= cost) return t;
  t.first = (int)(tiles - rem);
  t.split = s;
  t.len = split_len(R, s);
  return t;
}

// Splits of the soft backward's reduction over M. The fused epilogue needs the whole sum, so
// an unsplit launch has one workgroup per 256x256 output tile: 40 for k/v_proj, 160 for
// q/o_proj, 380 for the MLP shapes, i.e. whole or partial waves on 256 CUs. A split launch
// writes each split's partial dW rows in fp32 and a streaming kernel sums them and runs the
// soft epilogue. The count minimises a model of the two: (waves of 256 workgroups) x (stages
// per split) x 2.4 us, plus, when split, 32 B per weight of epilogue traffic and 8 B per weight
// and split of partials, at 5 TB/s. On the Qwen-4B shapes at M = 16384 it picks 6 / 3 / 2
// splits, the measured optimum of each.
inline int soft_splits(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ((N + TILE - 1) / TILE) * ((K + TILE - 1) / TILE);
  if (tiles == 0 || M <= 0) return 1;
  const double weights = (double)N * (double)K;
  const double stage_us = 2.4, epi_us = 32.0 * weights / 5.0e6, part_us = 8.0 * weights / 5.0e6;
  int best = 1;
  double best_t = (double)((tiles + 255) / 256) * (double)((M + BK - 1) / BK) * stage_us;
  for (int z = 2; z <= 16; ++z) {
    const int64_t len = split_len(M, z);
    if (len < 8 * BK || (int64_t)(z - 1) * len >= M) break;  // >= 8 stages, no empty split
    const double t = (double)((tiles * z + 255) / 256) * (double)(len / BK) * stage_us + epi_us +
                     z * part_us;
    if (t < best_t * 0.97) {
      best_t = t;
      best = z;
    }
  }
  return best;
}
}  // namespace g2
}  // namespace plz
