// Decode GEMV for 1 <= M <= 16 tokens: y[M,N] = x[M,K] W^T, one pass over packed W.
//
// The reference has no decode path; at M = 1 it would run the 64-row-tile forward kernel
// (fused_lut_kernel.cu:309-518). Here the work is bandwidth-bound: 2 bits of index plus
// 0.5 bit of fp32 palette per weight are streamed once, and everything else is arranged so
// that the stream never stops:
//
// * Persistent workgroups, a few per CU. The work items (128 rows of one linear, all of K) of
//   a launch are cut into one contiguous range per workgroup, balanced by bytes (K per item);
//   each XCD runs one contiguous block of ranges (xcd_range).
// * A workgroup walks its items as one sequence of stages (128 rows x 256 k = one palette
//   group), with the loads of the next item in flight while this one finishes.
// * Wave w owns rows 32w..32w+31 of the item (two MFMA row blocks of 16). Lane (row n%16,
//   quarter q) dequantises 4 consecutive packed words (64 k) of its row per block and stage
//   through v_perm_b32 byte tables into bf16 fragments (in a permuted k order that the x
//   fragments repeat); v_mfma_f32_16x16x32_bf16 computes C[n][m] for all M <= 16 tokens at
//   once (fragment lanes of tokens m >= M read token M-1; their columns are never stored).
//   x fragments come from the stage's x slice in LDS and serve both row blocks.
// * Native layouts (gemv_kernel): each stage's packed indices, palettes and x slice go
//   global->LDS by buffer_load ... lds (1 KB per wave instruction, whole cache lines), NS-1
//   stages ahead in an NS-slot ring; LDS layouts are XOR-swizzled on the global side of the
//   copies so that every fragment read is bank-conflict free.
// * Decode layouts (plz_gemv_pack_indices, plz_gemv_pack_palettes; gemv_reg_kernel): each
//   stage's 8 KB of words lie contiguous in the order the lanes read them, every word's 2-bit
//   fields permuted so that the dequantiser emits natural k order, and the palettes are ready
//   lookup words (8 B per row and stage). Words and lookup words go straight into registers,
//   RD stages ahead; only the x slice goes through LDS.
#include "plz_common.h"
#include "palettize_hip.h"

namespace plz {
namespace gv {

// Dequantise one packed word (16 indices) into two MFMA fragments in the cheapest byte-permute
// order: a = k {0,4,1,5,2,6,3,7}, b = k {8,12,9,13,10,14,11,15} (23 VALU per 16 weights).
__device__ __forceinline__ void dequant16_slots(uint32_t q, PalLut t, u32x4& a, u32x4& b) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t u = (q >> (2 * j)) & 0x03030303u;  // indices j, j+4, j+8, j+12
    const uint32_t l = perm(0, t.lo, u), h = perm(0, t.hi, u);
    a[j] = perm(h, l, 0x05010400u);  // {w_j, w_j+4}
    b[j] = perm(h, l, 0x07030602u);  // {w_j+8, w_j+12}
  }
}

// Decode-layout word: field (8B + 2j) (j, B = 0..3) holds the index of k = kmap(B, j), so that
// dequant16_slots returns a = k {0..7}, b = k {8..15} in order.
__host__ __device__ constexpr int decode_k(int B, int j) {
  return (B < 2 ? 0 : 8) + 2 * j + (B & 1);
}
__device__ __forceinline__ uint32_t decode_word(uint32_t w) {
  uint32_t o = 0;
#pragma unroll
  for (int B = 0; B < 4; ++B)
#pragma unroll
    for (int j = 0; j < 4; ++j) o |= ((w >> (2 * decode_k(B, j))) & 3u) << (8 * B + 2 * j);
  return o;
}

typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;

#ifndef PLZ_GV_WAVES
#define PLZ_GV_WAVES 4
#endif
constexpr int WAVES = PLZ_GV_WAVES;           // waves per workgroup
constexpr int RB = 8 / WAVES;                 // MFMA row blocks of 16 per wave
constexpr int ROWS = WAVES * 16 * RB;         // rows per work item: 128
constexpr int KC = 256;                       // k per stage: one palette group
constexpr int W_WAVE = 16 * RB * (KC / 4);    // packed bytes per wave and stage: RB KB
constexpr int W_BYTES = WAVES * W_WAVE;       // 8 KB
constexpr int X_TOKEN = KC * 2;               // x bytes per token and stage: 512 B
// Besides the packed words (2 copies per wave), each stage copies the item's palettes (128 rows
// x 16 B = 2 KB) and the x slice (M x 512 B) in 1 KB copy slots g = 4j + wave (j < NPX): slots
// 0-1 palettes, then two tokens per slot; slots past the data copy zeros.
template <int NPX>
constexpr int stage_bytes() { return W_BYTES + NPX * WAVES * 1024; }
// LDS ring slots (NS - 1 stages in flight) and the workgroups that share a CU's 160 KB
#ifndef PLZ_GV_NS
#define PLZ_GV_NS 4
#endif
template <int NPX>
constexpr int ring() { return PLZ_GV_NS; }
template <int NPX>
constexpr int lds_bytes() { return ring<NPX>() * stage_bytes<NPX>(); }
template <int NPX>
constexpr int wgs_per_cu() {
  return 160 * 1024 / lds_bytes<NPX>() < 16 / WAVES ? 160 * 1024 / lds_bytes<NPX>() : 16 / WAVES;
}
__host__ __device__ constexpr int npx_for(int M) { return (2 + (M + 1) / 2 + WAVES - 1) / WAVES; }

// swizzles (16-byte chunk index XOR): packed rows of 64 B (4 chunks), x rows of 512 B (32 chunks)
__device__ __forceinline__ int w_swz(int row) { return (row >> 2) & 3; }
__device__ __forceinline__ int x_swz(int m) { return m & 15; }

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xF | (3 << 14) | (7 << 4));  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ void dma16(BufRsrc r, uint32_t off, lds_u8* lds_wave_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_wave_base, 16, off, 0, 0, 0);
}

// The item list of a launch: items [block_begin, block_begin + ceil(N/ROWS)) belong to
// descriptor d; item j of d starts at byte-cost cost_begin + j*K.
template <bool GROUPED>
struct Table {
  const plz_gemv_desc* descs;
  int n;
  plz_gemv_desc single;
  __device__ __forceinline__ plz_gemv_desc at(int i) const { return GROUPED ? descs[i] : single; }
  __device__ __forceinline__ int find_item(int64_t item) const {  // descriptor of an item
    if (!GROUPED) return 0;
    int lo = 0, hi = n - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (descs[mid].block_begin <= item) lo = mid; else hi = mid - 1;
    }
    return lo;
  }
  // the item whose start cost is nearest to c (ties to the later one)
  __device__ __forceinline__ int64_t item_at_cost(int64_t c) const {
    int lo = 0;
    if (GROUPED) {
      int hi = n - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (descs[mid].cost_begin <= c) lo = mid; else hi = mid - 1;
      }
    }
    const plz_gemv_desc d = at(lo);
    const int64_t items = d.K > 0 ? (d.N + ROWS - 1) / ROWS : 0;
    if (items == 0) return d.block_begin;
    const int64_t j = (c - d.cost_begin + d.K / 2) / d.K;
    return d.block_begin + (j < items ? j : items);
  }
  __device__ __forceinline__ int64_t total_cost() const {
    const plz_gemv_desc d = at(GROUPED ? n - 1 : 0);
    const int64_t items = d.K > 0 ? (d.N + ROWS - 1) / ROWS : 0;
    return d.cost_begin + items * d.K;
  }
};

// Workgroups go to the 8 XCDs round-robin by linear id, and each XCD has its own L2. Range r
// (the byte-balanced ranges in cost order) is given to workgroup id so that XCD x runs one
// contiguous block of ranges: the few workgroups that share a linear then sit on one XCD, and
// since they reach the same 256-k stage at about the same time, its x slice is read from HBM
// once per linear instead of once per workgroup.
__device__ __forceinline__ int64_t xcd_range(int64_t id, int64_t G) {
  const int64_t x = id % 8, q8 = G / 8, r8 = G % 8;
  return x * q8 + (x < r8 ? x : r8) + id / 8;
}

// Position in a workgroup's stage sequence.
struct Cursor {
  int64_t item, end;
  int kc, nkc;
  plz_gemv_desc d;
  int64_t row0;  // first row of the item
  int di;        // descriptor index of the item
};
template <bool GROUPED>
__device__ __forceinline__ void cursor_load(Cursor& c, const Table<GROUPED>& tb) {
  c.kc = 0;
  if (c.item >= c.end) {  // finished (or empty) range: a harmless, never-live cursor
    c.nkc = 1;
    c.d = plz_gemv_desc{};
    c.row0 = 0;
    c.di = 0;
    return;
  }
  const int di = tb.find_item(c.item);
  c.di = di;
  c.d = tb.at(di);
  c.row0 = (c.item - c.d.block_begin) * ROWS;
  c.nkc = (int)((c.d.K + KC - 1) / KC);
}
template <bool GROUPED>
__device__ __forceinline__ void cursor_next(Cursor& c, const Table<GROUPED>& tb) {
  if (++c.kc < c.nkc) return;
  ++c.item;
  cursor_load(c, tb);
}

// The native layouts (packed indices [N, K/16], fp32 palettes); the decode layouts run
// gemv_reg_kernel below.
template <int NPX, bool GROUPED>
__global__ __launch_bounds__(64 * WAVES) void gemv_kernel(const plz_gemv_desc* __restrict__ descs,
                                                          int n_desc, plz_gemv_desc single,
                                                          int M) {
  extern __shared__ uint4 smem[];
  lds_u8* lds = (lds_u8*)smem;
  constexpr int NS = ring<NPX>();
  const Table<GROUPED> tb{descs, n_desc, single};
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int nl = lane & 15, q = lane >> 4;

  // this workgroup's items: those whose start cost lies in [wid*T/G, (wid+1)*T/G)
  const int64_t T = tb.total_cost(), G = gridDim.x, wid = xcd_range(blockIdx.x, G);
  Cursor pc, cc;
  pc.item = cc.item = tb.item_at_cost(wid * T / G);
  pc.end = cc.end = tb.item_at_cost((wid + 1) * T / G);
  cursor_load(pc, tb);
  cursor_load(cc, tb);

  // Copies of the producer's stage into ring slot `slot` (out-of-range lanes write zeros;
  // a stage past the workgroup's last item is all zeros and keeps the copy count uniform).
  // Per item, each lane's byte offsets without the k term are computed once; rows past N and
  // tokens past M fall outside the buffer ranges.
  // packed copy i of this lane: row 16i + lane/4 of the wave's rows, 16-byte chunk lane%4
  const int wrow = lane >> 2;
  static_assert(KC == kPalGroup, "one palette group per stage");
  uint32_t wbase[RB], mbase[NPX];
  BufRsrc rq = make_rsrc(nullptr, 0), rp = rq, rx = rq;
  int64_t p_item = -1;
  auto issue = [&](int slot) {
    lds_u8* st = lds + slot * stage_bytes<NPX>();
    const bool live = pc.item < pc.end;
    const int64_t N = pc.d.N, K = pc.d.K;
    const int gpr = (int)(K / kPalGroup);
    if (pc.item != p_item) {  // new item: descriptors and per-lane base offsets
      p_item = pc.item;
      // indices [N, K/16] words; palettes fp32 [N, K/256, 4] (16 B per row and stage, rows
      // gpr*16 B apart)
      rq = make_rsrc(pc.d.packed, live && pc.d.packed ? (uint32_t)(N * K / 4) : 0u);
      rp = make_rsrc(pc.d.palette, live && pc.d.palette ? (uint32_t)(N * gpr * 16) : 0u);
      rx = make_rsrc(pc.d.x, live ? (uint32_t)(M * K * 2) : 0u);
      const uint32_t r0 = (uint32_t)pc.row0;
#pragma unroll
      for (int i = 0; i < RB; ++i)
        wbase[i] = (r0 + 16 * RB * wave + 16 * i + wrow) * (uint32_t)(K / 4) +
                   16u * ((lane & 3) ^ w_swz(16 * i + wrow));
#pragma unroll
      for (int j = 0; j < NPX; ++j) {
        const int g = WAVES * j + wave;
        if (g < 2) {  // palettes of rows 64g + lane
          mbase[j] = (r0 + 64 * g + lane) * (uint32_t)gpr * 16u;
        } else {      // x tokens 2(g-2), 2(g-2)+1
          const int m = 2 * (g - 2) + (lane >> 5);
          mbase[j] = m < 16 ? ((uint32_t)m * (uint32_t)K + 8u * ((lane & 31) ^ x_swz(m))) * 2u
                            : kBufOob;
        }
      }
    }
    // K is a multiple of 256 = KC, so every stage is whole
    const uint32_t k0 = (uint32_t)pc.kc * KC;
    const uint32_t wk = k0 / 4;
#pragma unroll
    for (int i = 0; i < RB; ++i) dma16(rq, wbase[i] + wk, st + wave * W_WAVE + i * 1024);
#pragma unroll
    for (int j = 0; j < NPX; ++j) {
      const int g = WAVES * j + wave;
      lds_u8* dst = st + W_BYTES + g * 1024;
      if (g < 2)
        dma16(rp, mbase[j] + (uint32_t)pc.kc * 16u, dst);
      else
        dma16(rx, mbase[j] == kBufOob ? kBufOob : mbase[j] + k0 * 2u, dst);
    }
  };

  const int mx = nl < M ? nl : M - 1;  // token whose x this fragment lane reads

#pragma unroll
  for (int s = 0; s < NS - 1; ++s) {
    issue(s);
    cursor_next(pc, tb);
  }
  int s = 0;
  while (cc.item < cc.end) {  // one item (128 rows, all of K) per pass
    f32x4 acc[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int kc = 0; kc < cc.nkc; ++kc, ++s) {
      wait_vmcnt<(RB + NPX) * (NS - 2)>();  // this lane's copies of stage s have landed
      lds_barrier();                        // everyone's have; slot (s - 1) % NS is free
      issue((s + NS - 1) % NS);
      cursor_next(pc, tb);

      const lds_u8* st = lds + (s % NS) * stage_bytes<NPX>();
      const lds_u8* xs = st + W_BYTES + 2048 + mx * X_TOKEN;
      // x fragments of this lane: k = 64q + 16t + 8h .. +7 (t = 0..3, h = 0..1), permuted
      // into the dequantiser's slot order {k0, k4, k1, k5, k2, k6, k3, k7}
      u32x4 xf[8];
#pragma unroll
      for (int f = 0; f < 8; ++f) {
        const u32x4 v = *(const lds_u32x4*)(xs + (((8 * q + f) ^ x_swz(mx)) << 4));
        xf[f] = u32x4{perm(v[2], v[0], 0x05040100u), perm(v[2], v[0], 0x07060302u),
                      perm(v[3], v[1], 0x05040100u), perm(v[3], v[1], 0x07060302u)};
      }
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int row = 16 * r + nl;
        const u32x4 wv =
            *(const lds_u32x4*)(st + wave * W_WAVE + row * 64 + ((q ^ w_swz(row)) << 4));
        const u32x4 pv = *(const lds_u32x4*)(st + W_BYTES + (16 * RB * wave + row) * 16);
        const PalLut t = make_lut(__uint_as_float(pv[0]), __uint_as_float(pv[1]),
                                  __uint_as_float(pv[2]), __uint_as_float(pv[3]));
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          u32x4 a0, a1;
          dequant16_slots(wv[w], t, a0, a1);
          acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8, a0), __builtin_bit_cast(bf16x8, xf[2 * w]), acc[r], 0,
              0, 0);
          acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8, a1), __builtin_bit_cast(bf16x8, xf[2 * w + 1]), acc[r],
              0, 0, 0);
        }
      }
    }
    // item done: acc lane l holds C[row 4q + e][token nl]
    if (nl < M) {
#pragma unroll
      for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t n = cc.row0 + 16 * RB * wave + 16 * r + 4 * q + e;
          if (n < cc.d.N) cc.d.y[(int64_t)nl * cc.d.N + n] = (uint16_t)f2bf(acc[r][e]);
        }
    }
    ++cc.item;
    cursor_load(cc, tb);
  }
  __builtin_amdgcn_s_waitcnt(0);  // drain the trailing (empty) copies before the wave ends
}

// ---- register-ring kernel for the decode layouts ---------------------------------------
// The same items, stages, dequantiser and MFMAs as gemv_kernel, but a stage's packed words
// and lookup words go from global memory straight into registers: each lane loads exactly
// the 16 B of words per row block and the 8 B lookup words it dequantises (both layouts put
// them where the lane reads them), RD stages ahead in a ring of registers. Only the stage's
// x slice goes through LDS (shared by the four waves, one barrier per stage). The words in
// flight are then bounded by registers, not by LDS: RD-1 stages of 2 KB per wave, against the
// LDS ring's three stages of 8 KB per workgroup (which also held the x and palette slots).
#ifndef PLZ_GV_RD
#define PLZ_GV_RD 6
#endif
constexpr int RD = PLZ_GV_RD;
template <int NX>
constexpr int xstage_bytes() { return NX * WAVES * 1024; }  // x slots of one stage

template <int NX, bool GROUPED>
__global__ __launch_bounds__(64 * WAVES) void gemv_reg_kernel(const plz_gemv_desc* __restrict__ descs,
                                                              int n_desc, plz_gemv_desc single,
                                                              int M) {
  extern __shared__ uint4 smem[];
  lds_u8* lds = (lds_u8*)smem;
  constexpr int XS = xstage_bytes<NX>();
  constexpr int LOADS = 2 * RB + NX;  // vector-memory operations per lane and stage
  const Table<GROUPED> tb{descs, n_desc, single};
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int nl = lane & 15, q = lane >> 4;

  const int64_t T = tb.total_cost(), G = gridDim.x, wid = xcd_range(blockIdx.x, G);
  Cursor pc, cc;
  pc.item = cc.item = tb.item_at_cost(wid * T / G);
  pc.end = cc.end = tb.item_at_cost((wid + 1) * T / G);
  cursor_load(pc, tb);
  cursor_load(cc, tb);

  // the issue cursor's per-item state; dead stages (past the range) read zeros
  BufRsrc rq = make_rsrc(nullptr, 0), rp = rq, rx = rq;
  uint32_t qbase = 0, pbase = 0, mbase[NX];
  int64_t p_item = -1;
  const uint32_t wlane = (uint32_t)(wave * W_WAVE + lane * 16);       // words of this lane
  const uint32_t plane = (uint32_t)((16 * RB * wave + nl) * 8);       // lookup words of its row
  uint4 wr[RD][RB];  // words, [ring slot][row block]
  uint2 lr[RD][RB];  // lookup words {lo, hi}
  auto issue = [&](int slot, lds_u8* __restrict__ xdst) {
    const bool live = pc.item < pc.end;
    const int64_t N = pc.d.N, K = pc.d.K;
    if (pc.item != p_item) {
      p_item = pc.item;
      const int64_t rows = (N + ROWS - 1) / ROWS * ROWS;
      rq = make_rsrc(pc.d.packed_items, live && pc.d.packed_items ? (uint32_t)(rows * (K / 4)) : 0u);
      rp = make_rsrc(pc.d.palette_items,
                     live && pc.d.palette_items ? (uint32_t)(rows * (K / kPalGroup) * 8) : 0u);
      rx = make_rsrc(pc.d.x, live ? (uint32_t)(M * K * 2) : 0u);
      qbase = (uint32_t)pc.row0 * (uint32_t)(K / 4);
      pbase = (uint32_t)pc.row0 * (uint32_t)(K / kPalGroup) * 8u;
#pragma unroll
      for (int j = 0; j < NX; ++j) {  // x tokens 2g, 2g+1 of slot g = WAVES j + wave
        const int m = 2 * (WAVES * j + wave) + (lane >> 5);
        mbase[j] = m < 16 ? ((uint32_t)m * (uint32_t)K + 8u * ((lane & 31) ^ x_swz(m))) * 2u
                          : kBufOob;
      }
    }
    const uint32_t kc = (uint32_t)pc.kc;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
          rq, (int)wlane, (int)(qbase + kc * (uint32_t)W_BYTES + (uint32_t)r * 1024u), 0);
      wr[slot][r] = make_uint4(v.x, v.y, v.z, v.w);
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(
          rp, (int)plane, (int)(pbase + kc * (uint32_t)(ROWS * 8) + (uint32_t)r * 128u), 0);
      lr[slot][r] = make_uint2(v.x, v.y);
    }
#pragma unroll
    for (int j = 0; j < NX; ++j)
      dma16(rx, mbase[j] == kBufOob ? kBufOob : mbase[j] + kc * (uint32_t)(KC * 2),
            xdst + (WAVES * j + wave) * 1024);
  };

  const int mx = nl < M ? nl : M - 1;  // token whose x this fragment lane reads
  f32x4 acc[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
  // One stage: the copies of stage s + RD - 1 (registers of slot sw, x into xw), then the
  // MFMAs of stage s (registers of slot u, x from xr). xr and xw are distinct LDS slots, and
  // saying so (__restrict__) keeps the compiler from waiting for the x copy just issued --
  // and with it for every register load in flight -- before the x fragment reads.
  auto stage = [&](int u, int sw, const lds_u8* __restrict__ xr, lds_u8* __restrict__ xw) {
    issue(sw, xw);
    cursor_next(pc, tb);
    const lds_u8* xs = xr + mx * X_TOKEN;
    u32x4 xf[8];
#pragma unroll
    for (int f = 0; f < 8; ++f) xf[f] = *(const lds_u32x4*)(xs + (((8 * q + f) ^ x_swz(mx)) << 4));
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      PalLut t;
      t.lo = lr[u][r].x;
      t.hi = lr[u][r].y;
      const uint4 wv = wr[u][r];
      const uint32_t wq[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        u32x4 a0, a1;
        dequant16_slots(wq[w], t, a0, a1);
        acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, a0), __builtin_bit_cast(bf16x8, xf[2 * w]), acc[r], 0, 0, 0);
        acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, a1), __builtin_bit_cast(bf16x8, xf[2 * w + 1]), acc[r], 0,
            0, 0);
      }
    }
  };

#pragma unroll
  for (int p = 0; p < RD - 1; ++p) {
    issue(p, lds + p * XS);
    cursor_next(pc, tb);
  }
  // RD stages per pass, unrolled so that ring slots are constants. A pass runs whole even when
  // the range ends inside it (the stages past the end read zeros and store nothing): a break out
  // of the unrolled body makes the compiler wait for most of the ring at the next pass.
  while (cc.item < cc.end) {
#pragma unroll
    for (int u = 0; u < RD; ++u) {
      wait_vmcnt<(RD - 2) * LOADS>();  // this lane's loads of stage s have landed
      lds_barrier();                   // everyone's x copies have; slot (s - 1) % RD is free
      stage(u, (u + RD - 1) % RD, lds + u * XS, lds + ((u + RD - 1) % RD) * XS);
      if (++cc.kc == cc.nkc) {  // item done: acc lane l holds C[row 4q + e][token nl]
        if (nl < M) {
#pragma unroll
          for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int64_t n = cc.row0 + 16 * RB * wave + 16 * r + 4 * q + e;
              if (n < cc.d.N) cc.d.y[(int64_t)nl * cc.d.N + n] = (uint16_t)f2bf(acc[r][e]);
            }
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
        ++cc.item;
        cursor_load(cc, tb);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // drain the trailing (empty) loads before the wave ends
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

template <int NPX, bool GROUPED>
static int launch_nx(int64_t items, hipStream_t st, const plz_gemv_desc* descs, int n,
                     plz_gemv_desc single, int M, const char* what) {
  auto kern = gemv_kernel<NPX, GROUPED>;
  static uint64_t lds_done = 0;
  if (int rc = reserve_lds((const void*)kern, (size_t)lds_bytes<NPX>(), lds_done, what)) return rc;
  const int64_t slots = wgs_per_cu<NPX>() * (int64_t)cu_count();
  const int64_t g = items < slots ? items : slots;
  hipLaunchKernelGGL(kern, dim3((unsigned)g), dim3(64 * WAVES), lds_bytes<NPX>(), st, descs, n,
                     single, M);
  return check_launch(what);
}
template <bool GROUPED>
static int launch_native(int64_t items, hipStream_t st, const plz_gemv_desc* descs, int n,
                         plz_gemv_desc single, int M, const char* what) {
  switch (npx_for(M)) {
    case 1: return launch_nx<1, GROUPED>(items, st, descs, n, single, M, what);
    case 2: return launch_nx<2, GROUPED>(items, st, descs, n, single, M, what);
    case 3: return launch_nx<3, GROUPED>(items, st, descs, n, single, M, what);
    case 4: return launch_nx<4, GROUPED>(items, st, descs, n, single, M, what);
    default: return launch_nx<5, GROUPED>(items, st, descs, n, single, M, what);
  }
}
// decode layouts: the register-ring kernel; x slots for 8 tokens per stage (M <= 8) or 16
template <int NX, bool GROUPED>
static int launch_reg_nx(int64_t items, hipStream_t st, const plz_gemv_desc* descs, int n,
                         plz_gemv_desc single, int M, const char* what) {
  auto kern = gemv_reg_kernel<NX, GROUPED>;
  const size_t lds = (size_t)RD * xstage_bytes<NX>();
  static uint64_t lds_done = 0;
  if (int rc = reserve_lds((const void*)kern, lds, lds_done, what)) return rc;
  static int per_cu[64] = {0};  // resident workgroups per CU, per device
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (per_cu[dev] == 0) {
    int v = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, (const void*)kern, 64 * WAVES, lds) !=
            hipSuccess ||
        v < 1)
      v = 1;
    per_cu[dev] = v;
  }
  const int64_t slots = per_cu[dev] * (int64_t)cu_count();
  const int64_t g = items < slots ? items : slots;
  hipLaunchKernelGGL(kern, dim3((unsigned)g), dim3(64 * WAVES), lds, st, descs, n, single, M);
  return check_launch(what);
}
template <bool GROUPED>
static int launch(int64_t items, hipStream_t st, const plz_gemv_desc* descs, int n,
                  plz_gemv_desc single, int M, bool dec, const char* what) {
  if (dec)
    return M <= 8 ? launch_reg_nx<1, GROUPED>(items, st, descs, n, single, M, what)
                  : launch_reg_nx<2, GROUPED>(items, st, descs, n, single, M, what);
  return launch_native<GROUPED>(items, st, descs, n, single, M, what);
}

// palette [N, G, 4] -> lookup tables [ceil(N/ROWS)][G][ROWS][lo, hi] (make_lut of the row's
// group, rows past N zero): one row and group per thread
__global__ void pack_palettes_kernel(const float4* __restrict__ pal, uint2* __restrict__ out,
                                     int64_t N, int64_t G) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t items = (N + ROWS - 1) / ROWS;
  if (t >= items * G * ROWS) return;
  const int64_t row = t % ROWS, g = (t / ROWS) % G, item = t / (ROWS * G);
  const int64_t n = item * ROWS + row;
  uint2 v = make_uint2(0u, 0u);
  if (n < N) {
    const float4 p = pal[n * G + g];
    const PalLut lut = make_lut(p.x, p.y, p.z, p.w);
    v = make_uint2(lut.lo, lut.hi);
  }
  out[t] = v;
}

// packed [N, K/16] -> decode layout [ceil(N/ROWS)][K/256][WAVES][RB][64 lanes][4 words]: lane
// l = 16q + nl of block i of wave w holds words 4q..4q+3 (k 64q .. 64q+63 of the stage) of row
// 16 RB w + 16 i + nl, each through decode_word; rows past N are zero. One 16-byte chunk per
// thread.
__global__ void pack_indices_kernel(const uint4* __restrict__ packed, uint4* __restrict__ out,
                                    int64_t N, int64_t K) {
  constexpr int CH = W_BYTES / 16;  // chunks per stage
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stages = K / KC, items = (N + ROWS - 1) / ROWS;
  if (t >= items * stages * CH) return;
  const int c = (int)(t % CH);
  const int64_t st = (t / CH) % stages, item = t / (CH * stages);
  const int w = c / (W_WAVE / 16), i = (c / 64) % RB, l = c & 63;
  const int64_t n = item * ROWS + 16 * RB * w + 16 * i + (l & 15);
  uint4 v = make_uint4(0u, 0u, 0u, 0u);
  if (n < N) {
    const uint4 src = packed[n * (K / 64) + st * 4 + (l >> 4)];
    v = make_uint4(decode_word(src.x), decode_word(src.y), decode_word(src.z), decode_word(src.w));
  }
  out[t] = v;
}


// ---- bit-plane kernel (layout PLZ_GEMV_PLANES) -------------------------------------------
// A weight with index b = b0 + 2 b1 is w = p0 + d1 b0 + d2 b1 + d3 b0 b1 (d1 = p1 - p0,
// d2 = p2 - p0, d3 = p3 - p2 - p1 + p0). So per row n and palette group g
//   sum_k x_k w_k = p0 X + d1 S(b0) + d2 S(b1) + d3 S(b0 b1),   S(f) = sum_k x_k f_k,
// and the three bit planes go into the B operand of the scaled FP8 x FP4 MFMA
// (v_mfma_scale_f32_16x16x128_f8f6f4) straight from the packed word: a plane nibble is 0 or one
// FP4 power of two, cut out of the word by a mask or a 3-input AND -- 7 VALU per 16 weights,
// where dequantising to bf16 takes 23. X, the group sum of
// x, comes with the x pieces from the prep kernel. x is the A operand, in two
// e4m3 pieces per element, x = 2^s (x1 + x2) exactly (4 + 4 significant bits), with an E8M0
// scale 2^s per token and stage that the MFMA applies: A row m = 2 t + piece, so one 16-row
// operand holds 8 tokens. At the end of a stage p0 X + d1 S(b0) + d2 S(b1) + d3 S(b0 b1) is
// folded into the row's fp32 sum (the MFMA's B scales turn every plane into 0/1); the two pieces
// of a token are added when the item is stored.
//
// Operand layouts of the 16x16x128 MFMA (A fp8, B fp4), checked on the device: A lane l holds
// row l % 16, k = 16 (l/16) + e for bytes e < 16 and k = 64 + 16 (l/16) + e - 16 above; B lane
// l holds column l % 16, k = 32 (l/16) + e for nibble e; a lane's scale byte covers its row or
// column over k in [32 (l/16), 32 (l/16) + 32); C lane l holds rows 4 (l/16) + i, column l % 16.
//
// Planes layout of the indices (plz_gemv_pack_planes): the decode layout's blocks (8 KB per
// 128-row item and 256-k stage, 16 B per lane and 16-row block), where lane l = 16 g + nl of
// block r of wave w holds row 16 (RB w + r) + nl in four words: nibble i of word j holds the
// index of k = 32 g + 8 j + i in bits 4i, 4i+1 (MFMA half 0) and that of k = 128 + 32 g + 8 j + i
// in bits 4i+2, 4i+3 (half 1). With t = q >> 1, the planes of a word are then one mask or one
// 3-input AND each -- half 0: b0 = q & 0x11.. (0.5), b1 = q & 0x22.. (1.0), b0 b1 = q & t &
// 0x11.. (0.5); half 1: b0 = q & 0x44.. (2.0), b1 = t & 0x44.. (2.0), b0 b1 = q & t & 0x44..
// (2.0) -- 7 VALU per 16 weights, and the MFMA's B scale brings every plane to 0 / 1.
__host__ __device__ inline uint32_t plane_word(uint32_t src_a, uint32_t src_b, int off) {
  uint32_t o = 0;  // src_a / src_b: natural 16-index words holding the two halves' indices
  for (int i = 0; i < 8; ++i)
    o |= (((src_a >> (2 * (off + i))) & 3u) << (4 * i)) |
         (((src_b >> (2 * (off + i))) & 3u) << (4 * i + 2));
  return o;
}

// x prep, one chunk per (linear d, stage s) of the workspace at (d * max_stages + s) * chunk:
// A rows m = 2 t + piece, 256 B each (the fragments of both MFMA halves: 16-byte piece
// c = 8 h + 2 j + half, holding stage k = 128 h + 64 half + 16 j + (0..15), stored at
// c ^ (m & 15)); then the tokens' E8M0 scale bytes (16 B), their stage sums X as fp32 (64 B)
// and 48 B of padding.
__host__ __device__ constexpr int pl_chunk(int M) { return 512 * M + 128; }
__host__ __device__ constexpr int pl_nx(int M) {
  return (pl_chunk(M) + WAVES * 1024 - 1) / (WAVES * 1024);
}
typedef int i32x8 __attribute__((ext_vector_type(8)));

// One wave per linear, PREP_STAGES stages and PREP_TOKENS tokens: lane 16 g + c makes 16-byte
// piece c of work item 4 i + g, the items being the (token, stage) pairs of the wave's tokens
// and stages (at most 4 rounds of loads in sequence per wave).
constexpr int PREP_STAGES = 4, PREP_TOKENS = 4;
__host__ __device__ constexpr int prep_blocks_per_desc(int M, int max_stages) {
  return ((max_stages + PREP_STAGES - 1) / PREP_STAGES) * ((M + PREP_TOKENS - 1) / PREP_TOKENS);
}
template <bool GROUPED>
__global__ __launch_bounds__(64) void gemv_pl_prep_kernel(const plz_gemv_desc* __restrict__ descs,
                                                          int n_desc, plz_gemv_desc single,
                                                          int M, int max_stages,
                                                          uint8_t* __restrict__ ws) {
  const int tgroups = (M + PREP_TOKENS - 1) / PREP_TOKENS;
  const int blocks_per_desc = prep_blocks_per_desc(M, max_stages);
  const int d = blockIdx.x / blocks_per_desc, r = blockIdx.x % blocks_per_desc;
  const int s0 = (r / tgroups) * PREP_STAGES, t0 = (r % tgroups) * PREP_TOKENS;
  const int mt = M - t0 < PREP_TOKENS ? M - t0 : PREP_TOKENS;
  const Table<GROUPED> tb{descs, n_desc, single};
  const plz_gemv_desc dd = tb.at(d);
  const int stages = (int)(dd.K / KC);
  if (s0 >= stages || dd.N == 0) return;  // uniform per block
  const int ns = stages - s0 < PREP_STAGES ? stages - s0 : PREP_STAGES;
  const int lane = threadIdx.x, c = lane & 15, g = lane >> 4;
  const int k0 = 128 * (c >> 3) + 64 * (c & 1) + 16 * ((c >> 1) & 3);
  for (int w0 = 0; w0 < mt * ns; w0 += 4) {
    const int w = w0 + g, t = t0 + w % mt, s = s0 + w / mt;
    const bool live = w < mt * ns;
    uint32_t b[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (live) {
      const uint4* src = reinterpret_cast<const uint4*>(dd.x + (int64_t)t * dd.K + (int64_t)s * KC + k0);
      const uint4 v0 = src[0], v1 = src[1];
      b[0] = v0.x; b[1] = v0.y; b[2] = v0.z; b[3] = v0.w;
      b[4] = v1.x; b[5] = v1.y; b[6] = v1.z; b[7] = v1.w;
    }
    float v[16];
    int emax = 0;
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t h = (b[i / 2] >> (16 * (i & 1))) & 0xffffu;
      v[i] = bf2f(h);
      const int e = (int)((h >> 7) & 0xffu);
      emax = e != 0xff && e > emax ? e : emax;  // the finite values set the scale
      sum += v[i];
    }
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) {  // over the 16 lanes of the item, fixed order
      const int oe = __shfl_xor(emax, off);
      emax = oe > emax ? oe : emax;
      sum += __shfl_xor(sum, off);
    }
    if (!live) continue;
    uint8_t* ch = ws + ((int64_t)d * max_stages + s) * pl_chunk(M);
    // scale 2^s = 2^(E - 7), E the unbiased exponent of the stage's largest finite |x| plus
    // one: |x| / 2^s < 256, well inside e4m3's 448; e8 = s + 127
    const int e8 = emax >= 7 ? emax - 7 : 0;
    const float inv = __builtin_bit_cast(float, (uint32_t)(254 - e8) << 23);  // 2^-s
    uint32_t w1[4] = {0, 0, 0, 0}, w2[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float xs = v[i] * inv;
      uint32_t p1 = 0x7fu, p2 = 0x7fu;  // NaN and +-inf: e4m3 NaN, the token's outputs go NaN
      if (__builtin_isfinite(xs)) {
        const int q1 = __builtin_amdgcn_cvt_pk_fp8_f32(xs, 0.f, 0, false);
        const float r = xs - __builtin_amdgcn_cvt_f32_fp8(q1, 0);  // exact
        p1 = (uint32_t)q1 & 0xffu;
        p2 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(r, 0.f, 0, false) & 0xffu;
      }
      w1[i / 4] |= p1 << (8 * (i & 3));
      w2[i / 4] |= p2 << (8 * (i & 3));
    }
    const int m0 = 2 * t, m1 = 2 * t + 1;
    *reinterpret_cast<uint4*>(ch + m0 * 256 + ((c ^ (m0 & 15)) << 4)) =
        make_uint4(w1[0], w1[1], w1[2], w1[3]);
    *reinterpret_cast<uint4*>(ch + m1 * 256 + ((c ^ (m1 & 15)) << 4)) =
        make_uint4(w2[0], w2[1], w2[2], w2[3]);
    if (c == 0) {
      ch[512 * M + t] = (uint8_t)e8;
      reinterpret_cast<float*>(ch + 512 * M + 16)[t] = sum;
    }
  }
}

// NX: 1 KB x-chunk copies per wave and stage (pl_nx(M)); NSET: 16-row A operands (8 tokens
// each); NI: C rows per lane that can hold a token's piece (2 at M = 1).
//
// Outputs are staged in LDS (YBYTES per workgroup) and written when the staging is full or at
// the end: a global store pending beside the register ring's loads would make the compiler
// drain the ring (s_waitcnt vmcnt(0)) at the next wait, since it cannot order stores against
// loads on the one counter.
constexpr int YBYTES = 16384;
#ifndef PLZ_GV_RDP
#define PLZ_GV_RDP 5
#endif
constexpr int RDP = PLZ_GV_RDP;  // register-ring depth (stages) of the bit-plane kernel
template <int NX, int NSET, int NI, bool GROUPED>
__global__ __launch_bounds__(64 * WAVES) void gemv_pl_kernel(const plz_gemv_desc* __restrict__ descs,
                                                             int n_desc, plz_gemv_desc single,
                                                             int M, int max_stages,
                                                             const uint8_t* __restrict__ ws,
                                                             uint32_t ws_bytes) {
  extern __shared__ uint4 smem[];
  lds_u8* lds = (lds_u8*)smem;
  constexpr int XS = NX * WAVES * 1024;
  constexpr int LOADS = 2 * RB + NX;  // vector-memory operations per lane and stage
  typedef __attribute__((address_space(3))) uint16_t lds_u16;
  typedef __attribute__((address_space(3))) int64_t lds_i64;
  lds_u16* ybuf = (lds_u16*)(lds + RDP * XS);                 // [ycap][M][ROWS] bf16
  lds_i64* yitem = (lds_i64*)(lds + RDP * XS + YBYTES);       // [ycap] item of each slot
  const int ycap = YBYTES / (ROWS * M * 2);
  const Table<GROUPED> tb{descs, n_desc, single};
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int nl = lane & 15, q = lane >> 4;
  const uint32_t CH = (uint32_t)pl_chunk(M);

  const int64_t T = tb.total_cost(), G = gridDim.x, wid = xcd_range(blockIdx.x, G);
  Cursor pc, cc;
  pc.item = cc.item = tb.item_at_cost(wid * T / G);
  pc.end = cc.end = tb.item_at_cost((wid + 1) * T / G);
  cursor_load(pc, tb);
  cursor_load(cc, tb);

  BufRsrc rq = make_rsrc(nullptr, 0), rp = rq;
  const BufRsrc rx = make_rsrc(ws, ws_bytes);
  uint32_t qbase = 0, pbase = 0, xbase = 0;
  int64_t p_item = -1;
  const uint32_t wlane = (uint32_t)(wave * W_WAVE + lane * 16);  // words of this lane
  const uint32_t plane = (uint32_t)((16 * RB * wave + nl) * 8);  // lookup words of its row
  uint4 wr[RDP][RB];  // words, [ring slot][row block]
  uint2 lr[RDP][RB];  // lookup words {lo, hi}
  auto issue = [&](int slot, lds_u8* __restrict__ xdst) {
    const bool live = pc.item < pc.end;
    const int64_t N = pc.d.N, K = pc.d.K;
    if (pc.item != p_item) {
      p_item = pc.item;
      const int64_t rows = (N + ROWS - 1) / ROWS * ROWS;
      rq = make_rsrc(pc.d.packed_items, live && pc.d.packed_items ? (uint32_t)(rows * (K / 4)) : 0u);
      rp = make_rsrc(pc.d.palette_items,
                     live && pc.d.palette_items ? (uint32_t)(rows * (K / kPalGroup) * 8) : 0u);
      qbase = (uint32_t)pc.row0 * (uint32_t)(K / 4);
      pbase = (uint32_t)pc.row0 * (uint32_t)(K / kPalGroup) * 8u;
      xbase = live ? (uint32_t)pc.di * (uint32_t)max_stages * CH : kBufOob;
    }
    const uint32_t kc = (uint32_t)pc.kc;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
          rq, (int)wlane, (int)(qbase + kc * (uint32_t)W_BYTES + (uint32_t)r * 1024u), 0);
      wr[slot][r] = make_uint4(v.x, v.y, v.z, v.w);
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(
          rp, (int)plane, (int)(pbase + kc * (uint32_t)(ROWS * 8) + (uint32_t)r * 128u), 0);
      lr[slot][r] = make_uint2(v.x, v.y);
    }
#pragma unroll
    for (int j = 0; j < NX; ++j) {
      const uint32_t g = (uint32_t)(WAVES * j + wave);
      dma16(rx, xbase == kBufOob ? kBufOob : xbase + kc * CH + g * 1024u + (uint32_t)lane * 16u,
            xdst + g * 1024);
    }
  };

  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 yacc[RB][NSET];
#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int S = 0; S < NSET; ++S) yacc[r][S] = zero;
  // E8M0 scales 1.0, 2.0 and 0.5 (every plane bit of half 1 sits at nibble bit 2, value 2.0)
  constexpr int kScale1 = 127, kScale2 = 128, kScaleH = 126;
  constexpr uint32_t M1 = 0x11111111u, M2 = 0x22222222u, M4 = 0x44444444u;

  // One stage: the loads of stage s + RDP - 1 (registers of slot sw, x chunk into xw), then the
  // MFMAs of stage s (registers of slot u, x chunk from xr).
  auto stage = [&](int u, int sw, const lds_u8* __restrict__ xr, lds_u8* __restrict__ xw) {
    issue(sw, xw);
    cursor_next(pc, tb);
    i32x8 a[NSET][2];
    int sc[NSET];
    float xsum[NSET][NI / 2];  // X of the tokens whose first piece this lane's C rows hold
#pragma unroll
    for (int S = 0; S < NSET; ++S) {
      const int mr = 16 * S + nl, m = mr < 2 * M ? mr : 2 * M - 1;  // rows past 2M repeat one
      const lds_u8* row = xr + m * 256;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c0 = 8 * h + 2 * q;
        const u32x4 lo = *(const lds_u32x4*)(row + ((c0 ^ (m & 15)) << 4));
        const u32x4 hi = *(const lds_u32x4*)(row + (((c0 + 1) ^ (m & 15)) << 4));
        a[S][h] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                        (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      }
      sc[S] = (int)xr[512 * M + (m >> 1)];
#pragma unroll
      for (int i = 0; i < NI; i += 2)  // token of C row 16 S + 4 q + i (a stale value past M)
        xsum[S][i / 2] = *(const __attribute__((address_space(3))) float*)(
            xr + 512 * M + 16 + 4 * (8 * S + 2 * q + i / 2));
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      // the row's palette entries as fp32 (bf16 bits: high byte from hi, low byte from lo)
      const uint32_t lo = lr[u][r].x, hi = lr[u][r].y;
      const float p0 = __uint_as_float(perm(hi, lo, 0x04000c0cu));
      const float p1 = __uint_as_float(perm(hi, lo, 0x05010c0cu));
      const float p2 = __uint_as_float(perm(hi, lo, 0x06020c0cu));
      const float p3 = __uint_as_float(perm(hi, lo, 0x07030c0cu));
      const float c1 = p1 - p0, c2 = p2 - p0, c3 = (p3 - p2) - c1;
      const uint4 wv = wr[u][r];
      const uint32_t wq[4] = {wv.x, wv.y, wv.z, wv.w};
      f32x4 cb0[NSET], cb1[NSET], cb3[NSET];
      uint32_t t[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) t[j] = wq[j] >> 1;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t m0 = h ? M4 : M1, m1 = h ? M4 : M2;  // b0 (and b0 b1), b1 masks
        i32x8 B0 = {0, 0, 0, 0, 0, 0, 0, 0}, B1 = B0, B3 = B0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          B0[j] = (int)(wq[j] & m0);
          B1[j] = (int)((h ? t[j] : wq[j]) & m1);
          B3[j] = (int)(wq[j] & t[j] & m0);
        }
        // B scales that make every plane 0 / 1: half 0 planes are 0.5 / 1.0 / 0.5, half 1 2.0
        const int s0 = h ? kScaleH : kScale2, s1 = h ? kScaleH : kScale1, s3 = h ? kScaleH : kScale2;
#pragma unroll
        for (int S = 0; S < NSET; ++S) {
          cb0[S] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[S][h], B0, h ? cb0[S] : zero,
                                                                    0, 4, 0, sc[S], 0, s0);
          cb1[S] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[S][h], B1, h ? cb1[S] : zero,
                                                                    0, 4, 0, sc[S], 0, s1);
          cb3[S] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[S][h], B3, h ? cb3[S] : zero,
                                                                    0, 4, 0, sc[S], 0, s3);
        }
      }
#pragma unroll
      for (int S = 0; S < NSET; ++S)
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          float y = __builtin_fmaf(c1, cb0[S][i], __builtin_fmaf(c2, cb1[S][i],
                                   __builtin_fmaf(c3, cb3[S][i], yacc[r][S][i])));
          if ((i & 1) == 0) y = __builtin_fmaf(p0, xsum[S][i / 2], y);  // first piece only
          yacc[r][S][i] = y;
        }
    }
  };

  // the staged outputs of slots [0, cnt) to y (after a barrier; all waves take part)
  auto flush = [&](int cnt) {
    for (int it = 0; it < cnt; ++it) {
      const int64_t iv = yitem[it];  // the same in every lane: make it scalar
      const int64_t item = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(iv >> 32)) << 32) |
                                     (uint32_t)__builtin_amdgcn_readfirstlane((int)iv));
      const plz_gemv_desc d = tb.at(tb.find_item(item));
      const int64_t row0 = (item - d.block_begin) * ROWS;
      for (int t = wave; t < M; t += WAVES)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int nloc = 2 * lane + h;
          if (row0 + nloc < d.N)
            ((__attribute__((address_space(1))) uint16_t*)d.y)[(int64_t)t * d.N + row0 + nloc] =
                ybuf[(it * M + t) * ROWS + nloc];  // a global store (a flat one would also count
                                                  // on lgkmcnt)
        }
    }
  };

#pragma unroll
  for (int p = 0; p < RDP - 1; ++p) {
    issue(p, lds + p * XS);
    cursor_next(pc, tb);
  }
  int ycount = 0;
  // RDP stages per pass, unrolled so that ring slots are constants. A pass runs whole even when
  // the range ends inside it (the stages past the end read zeros and store nothing): a break out
  // of the unrolled body makes the compiler wait for most of the ring at the next pass.
  while (cc.item < cc.end) {
#pragma unroll
    for (int u = 0; u < RDP; ++u) {
      wait_vmcnt<(RDP - 2) * LOADS>();  // this lane's loads of stage s have landed
      lds_barrier();                   // everyone's x copies have; slot (s - 1) % RDP is free
      stage(u, (u + RDP - 1) % RDP, lds + u * XS, lds + ((u + RDP - 1) % RDP) * XS);
      if (++cc.kc == cc.nkc) {  // item done: C row 16 S + 4 q + i of lane l = piece i & 1 of
                                // token 8 S + 2 q + i / 2, item row 16 (RB w + r) + nl
        if (cc.item < cc.end) {  // a live item (the last pass may run past the range)
#pragma unroll
          for (int r = 0; r < RB; ++r) {
            const int nloc = 16 * RB * wave + 16 * r + nl;
#pragma unroll
            for (int S = 0; S < NSET; ++S)
#pragma unroll
              for (int i = 0; i < NI; i += 2) {
                const int t = 8 * S + 2 * q + i / 2;
                if (t < M)
                  ybuf[(ycount * M + t) * ROWS + nloc] =
                      (uint16_t)f2bf(yacc[r][S][i] + yacc[r][S][i + 1]);
              }
          }
          if (threadIdx.x == 0) yitem[ycount] = cc.item;
          if (++ycount == ycap) {  // the same count in every wave: waves walk the same stages
            __syncthreads();
            flush(ycount);
            __syncthreads();
            ycount = 0;
          }
        }
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
          for (int S = 0; S < NSET; ++S) yacc[r][S] = zero;
        ++cc.item;
        cursor_load(cc, tb);
      }
    }
  }
  __syncthreads();
  flush(ycount);
  __builtin_amdgcn_s_waitcnt(0);  // drain the trailing (empty) loads before the wave ends
}

// packed [N, K/16] -> planes layout: the decode layout's chunk order (one 16-byte chunk per
// thread: lane l = 16 g + nl of block i of wave w, row 16 RB w + 16 i + nl), word j pairing
// k = 32 g + 8 j + (0..7) with 128 + 32 g + 8 j + (0..7) of the stage through plane_word.
__global__ void pack_planes_kernel(const uint32_t* __restrict__ packed, uint4* __restrict__ out,
                                   int64_t N, int64_t K) {
  constexpr int CHK = W_BYTES / 16;  // chunks per stage
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stages = K / KC, items = (N + ROWS - 1) / ROWS;
  if (t >= items * stages * CHK) return;
  const int c = (int)(t % CHK);
  const int64_t st = (t / CHK) % stages, item = t / (CHK * stages);
  const int w = c / (W_WAVE / 16), i = (c / 64) % RB, l = c & 63;
  const int64_t n = item * ROWS + 16 * RB * w + 16 * i + (l & 15);
  uint4 v = make_uint4(0u, 0u, 0u, 0u);
  if (n < N) {
    const uint32_t* src = packed + n * (K / 16) + st * (KC / 16);
    const int g = l >> 4;
    uint32_t w[4];
    for (int j = 0; j < 4; ++j)  // k = 32 g + 8 j lies in source word 2 g + j / 2
      w[j] = plane_word(src[2 * g + j / 2], src[8 + 2 * g + j / 2], 8 * (j & 1));
    v = make_uint4(w[0], w[1], w[2], w[3]);
  }
  out[t] = v;
}

template <int NX, int NSET, int NI, bool GROUPED>
static int launch_pl_nx(int64_t items, hipStream_t st, const plz_gemv_desc* descs, int n,
                        plz_gemv_desc single, int M, int max_stages, uint8_t* ws,
                        size_t ws_bytes, const char* what) {
  hipLaunchKernelGGL(gemv_pl_prep_kernel<GROUPED>,
                     dim3((unsigned)(n * prep_blocks_per_desc(M, max_stages))), dim3(64), 0,
                     st, descs, n, single, M, max_stages, ws);
  auto kern = gemv_pl_kernel<NX, NSET, NI, GROUPED>;
  const size_t lds = (size_t)RDP * NX * WAVES * 1024 + YBYTES + (YBYTES / (ROWS * 2)) * 8;
  static uint64_t lds_done = 0;
  if (int rc = reserve_lds((const void*)kern, lds, lds_done, what)) return rc;
  static int per_cu[64] = {0};  // resident workgroups per CU, per device
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (per_cu[dev] == 0) {
    int v = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, (const void*)kern, 64 * WAVES, lds) !=
            hipSuccess ||
        v < 1)
      v = 1;
    per_cu[dev] = v;
  }
  const int64_t slots = per_cu[dev] * (int64_t)cu_count();
  const int64_t g = items < slots ? items : slots;
  hipLaunchKernelGGL(kern, dim3((unsigned)g), dim3(64 * WAVES), lds, st, descs, n, single, M,
                     max_stages, (const uint8_t*)ws, (uint32_t)ws_bytes);
  return check_launch(what);
}
template <bool GROUPED>
static int launch_pl(int64_t items, hipStream_t st, const plz_gemv_desc* descs, int n,
                     plz_gemv_desc single, int M, int max_stages, uint8_t* ws, size_t ws_bytes,
                     const char* what) {
  if (M == 1)
    return launch_pl_nx<pl_nx(1), 1, 2, GROUPED>(items, st, descs, n, single, M, max_stages, ws,
                                                 ws_bytes, what);
  if (M <= 7)
    return launch_pl_nx<pl_nx(7), 1, 4, GROUPED>(items, st, descs, n, single, M, max_stages, ws,
                                                 ws_bytes, what);
  if (M == 8)
    return launch_pl_nx<pl_nx(8), 1, 4, GROUPED>(items, st, descs, n, single, M, max_stages, ws,
                                                 ws_bytes, what);
  if (M <= 15)
    return launch_pl_nx<pl_nx(15), 2, 4, GROUPED>(items, st, descs, n, single, M, max_stages, ws,
                                                  ws_bytes, what);
  return launch_pl_nx<pl_nx(16), 2, 4, GROUPED>(items, st, descs, n, single, M, max_stages, ws,
                                                ws_bytes, what);
}
static_assert(pl_nx(1) == 1 && pl_nx(7) == 1 && pl_nx(8) == 2 && pl_nx(15) == 2 && pl_nx(16) == 3,
              "x chunk copies per wave");

static int check_desc(const plz_gemv_desc& d, int i) {
  PLZ_REQUIRE(d.N >= 0 && d.K >= 0, "plz_gemv: descriptor %d has a negative shape", i);
  PLZ_REQUIRE(d.K % 256 == 0, "plz_gemv: descriptor %d: K (%lld) must be a multiple of 256", i,
              (long long)d.K);
  PLZ_REQUIRE(d.N == 0 || d.K == 0 ||
                  (d.x && (d.packed || d.packed_items) && (d.palette || d.palette_items) && d.y),
              "plz_gemv: descriptor %d has a null pointer", i);
  PLZ_REQUIRE(d.N * d.K / 4 < (int64_t)kBufOob && d.N * (d.K / 256) * 16 < (int64_t)kBufOob &&
                  16 * d.K * 2 < (int64_t)kBufOob,
              "plz_gemv: descriptor %d is too large (packed or palette above 2 GiB)", i);
  PLZ_REQUIRE((((uintptr_t)d.x | (uintptr_t)d.packed | (uintptr_t)d.palette |
                 (uintptr_t)d.palette_items | (uintptr_t)d.packed_items) & 15) == 0,
              "plz_gemv: descriptor %d: x, packed and palettes must be 16-byte aligned", i);
  PLZ_REQUIRE((d.N + ROWS - 1) / ROWS * ROWS * (d.K / 4) < (int64_t)kBufOob,
              "plz_gemv: descriptor %d: decode-layout indices above 2 GiB", i);
  PLZ_REQUIRE((d.N + ROWS - 1) / ROWS * ROWS * (d.K / 256) * 8 < (int64_t)kBufOob,
              "plz_gemv: descriptor %d: prepacked palettes above 2 GiB", i);
  return PLZ_OK;
}

}  // namespace gv
}  // namespace plz

using namespace plz;
using namespace plz::gv;

extern "C" {

int plz_lut_gemv(const uint16_t* x, const int32_t* packed, const float* palette, uint16_t* y,
                 int64_t M, int64_t N, int64_t K, void* stream) {
  PLZ_REQUIRE(M >= 1 && M <= 16, "plz_lut_gemv: M (%lld) must be in [1, 16]", (long long)M);
  plz_gemv_desc d = {x, packed, palette, y, N, K, 0, 0, nullptr, nullptr};
  PLZ_REQUIRE(N == 0 || K == 0 || (packed && palette), "plz_lut_gemv: null pointer");
  int rc = check_desc(d, 0);
  if (rc) return rc;
  if (N == 0) return PLZ_OK;
  if (K == 0) {
    zero_async(y, (size_t)M * N * 2, (hipStream_t)stream);
    return check_launch("plz_lut_gemv");
  }
  const int64_t items = (N + ROWS - 1) / ROWS;
  return launch<false>(items, (hipStream_t)stream, nullptr, 1, d, (int)M, false, "plz_lut_gemv");
}

int plz_lut_gemv_decode(const uint16_t* x, const int32_t* packed_items,
                        const uint32_t* palette_items, uint16_t* y, int64_t M, int64_t N, int64_t K,
                        void* stream) {
  PLZ_REQUIRE(M >= 1 && M <= 16, "plz_lut_gemv_decode: M (%lld) must be in [1, 16]", (long long)M);
  PLZ_REQUIRE(N == 0 || K == 0 || (packed_items && palette_items),
              "plz_lut_gemv_decode: null pointer");
  plz_gemv_desc d = {x, nullptr, nullptr, y, N, K, 0, 0, palette_items, packed_items};
  int rc = check_desc(d, 0);
  if (rc) return rc;
  if (N == 0) return PLZ_OK;
  if (K == 0) {
    zero_async(y, (size_t)M * N * 2, (hipStream_t)stream);
    return check_launch("plz_lut_gemv_decode");
  }
  const int64_t items = (N + ROWS - 1) / ROWS;
  return launch<false>(items, (hipStream_t)stream, nullptr, 1, d, (int)M, true,
                       "plz_lut_gemv_decode");
}

size_t plz_gemv_packed_items_bytes(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0) return 0;
  return (size_t)((N + ROWS - 1) / ROWS) * ROWS * (size_t)(K / 4);
}

int plz_gemv_pack_indices(const int32_t* packed, int32_t* packed_items, int64_t N, int64_t K,
                          void* stream) {
  PLZ_REQUIRE(N >= 0 && K >= 0 && K % KC == 0,
              "plz_gemv_pack_indices: need N, K >= 0 and K a multiple of 256");
  if (N == 0 || K == 0) return PLZ_OK;
  PLZ_REQUIRE(packed && packed_items && (((uintptr_t)packed | (uintptr_t)packed_items) & 15) == 0,
              "plz_gemv_pack_indices: packed and packed_items must be non-null, 16-byte aligned");
  const int64_t total = (N + ROWS - 1) / ROWS * (K / KC) * (W_BYTES / 16);
  hipLaunchKernelGGL(pack_indices_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, reinterpret_cast<const uint4*>(packed),
                     reinterpret_cast<uint4*>(packed_items), N, K);
  return check_launch("plz_gemv_pack_indices");
}

size_t plz_gemv_palette_items_bytes(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0) return 0;
  return (size_t)((N + ROWS - 1) / ROWS) * ROWS * (K / kPalGroup) * 8;
}

int plz_gemv_pack_palettes(const float* palette, uint32_t* palette_items, int64_t N, int64_t K,
                           void* stream) {
  PLZ_REQUIRE(N >= 0 && K >= 0 && K % kPalGroup == 0,
              "plz_gemv_pack_palettes: need N, K >= 0 and K a multiple of 256");
  if (N == 0 || K == 0) return PLZ_OK;
  PLZ_REQUIRE(palette && palette_items && (((uintptr_t)palette | (uintptr_t)palette_items) & 15) == 0,
              "plz_gemv_pack_palettes: palette and palette_items must be non-null, 16-byte aligned");
  const int64_t G = K / kPalGroup, total = (N + ROWS - 1) / ROWS * G * ROWS;
  hipLaunchKernelGGL(pack_palettes_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, reinterpret_cast<const float4*>(palette),
                     reinterpret_cast<uint2*>(palette_items), N, G);
  return check_launch("plz_gemv_pack_palettes");
}

int64_t plz_gemv_plan(plz_gemv_desc* descs, int n, int M, int layout) {
  if (n < 0 || !descs || M < 1 || M > 16) {
    set_error("plz_gemv_plan: need n >= 0, non-null descriptors and M in [1, 16]");
    return -PLZ_EINVAL;
  }
  if (layout != PLZ_GEMV_NATIVE && layout != PLZ_GEMV_DECODE && layout != PLZ_GEMV_PLANES) {
    set_error("plz_gemv_plan: unknown index layout %d", layout);
    return -PLZ_EINVAL;
  }
  int64_t items = 0, cost = 0;
  for (int i = 0; i < n; ++i) {
    int rc = check_desc(descs[i], i);
    if (rc) return -rc;
    if (descs[i].N > 0 && descs[i].K == 0) {
      set_error("plz_gemv_plan: descriptor %d has K = 0", i);
      return -PLZ_EINVAL;
    }
    // every non-empty linear must hold the arrays the chosen layout streams
    const bool nonempty = descs[i].N > 0 && descs[i].K > 0;
    if (nonempty && layout == PLZ_GEMV_NATIVE && (!descs[i].packed || !descs[i].palette)) {
      set_error("plz_gemv_plan: descriptor %d has a null packed or palette array (native "
                "layout)", i);
      return -PLZ_EINVAL;
    }
    if (nonempty && layout != PLZ_GEMV_NATIVE &&
        (!descs[i].packed_items || !descs[i].palette_items)) {
      set_error("plz_gemv_plan: descriptor %d has a null packed_items or palette_items array "
                "(%s layout)", i, layout == PLZ_GEMV_DECODE ? "decode" : "planes");
      return -PLZ_EINVAL;
    }
    descs[i].block_begin = items;
    descs[i].cost_begin = cost;
    const int64_t it = descs[i].K > 0 ? (descs[i].N + ROWS - 1) / ROWS : 0;
    items += it;
    cost += it * descs[i].K;
  }
  return items;
}

int plz_lut_gemv_grouped(const plz_gemv_desc* descs_device, int n, int64_t total_blocks, int M,
                         int layout, void* stream) {
  PLZ_REQUIRE(M >= 1 && M <= 16, "plz_lut_gemv_grouped: M (%d) must be in [1, 16]", M);
  PLZ_REQUIRE(layout != PLZ_GEMV_PLANES,
              "plz_lut_gemv_grouped: the planes layout runs through plz_lut_gemv_grouped_planes "
              "(it needs a workspace)");
  PLZ_REQUIRE(layout == PLZ_GEMV_NATIVE || layout == PLZ_GEMV_DECODE,
              "plz_lut_gemv_grouped: unknown index layout %d", layout);
  PLZ_REQUIRE(n >= 0 && total_blocks >= 0, "plz_lut_gemv_grouped: negative count");
  if (n == 0 || total_blocks == 0) return PLZ_OK;
  PLZ_REQUIRE(descs_device, "plz_lut_gemv_grouped: null descriptor table");
  plz_gemv_desc dummy = {};
  return launch<true>(total_blocks, (hipStream_t)stream, descs_device, n, dummy, M,
                      layout == PLZ_GEMV_DECODE, "plz_lut_gemv_grouped");
}

int plz_gemv_pack_planes(const int32_t* packed, int32_t* planes_items, int64_t N, int64_t K,
                         void* stream) {
  PLZ_REQUIRE(N >= 0 && K >= 0 && K % KC == 0,
              "plz_gemv_pack_planes: need N, K >= 0 and K a multiple of 256");
  if (N == 0 || K == 0) return PLZ_OK;
  PLZ_REQUIRE(packed && planes_items && (((uintptr_t)packed | (uintptr_t)planes_items) & 15) == 0,
              "plz_gemv_pack_planes: packed and planes_items must be non-null, 16-byte aligned");
  const int64_t total = (N + ROWS - 1) / ROWS * (K / KC) * (W_BYTES / 16);
  hipLaunchKernelGGL(pack_planes_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, reinterpret_cast<const uint32_t*>(packed),
                     reinterpret_cast<uint4*>(planes_items), N, K);
  return check_launch("plz_gemv_pack_planes");
}

size_t plz_gemv_planes_workspace(int n, int64_t max_K, int M) {
  if (n <= 0 || max_K <= 0 || M < 1 || M > 16) return 0;
  return (size_t)n * (size_t)((max_K + KC - 1) / KC) * (size_t)pl_chunk(M);
}

static int planes_ws_check(int n, int64_t max_K, int M, void* workspace, size_t workspace_bytes,
                           const char* what) {
  const size_t need = plz_gemv_planes_workspace(n, max_K, M);
  PLZ_REQUIRE(need < (size_t)kBufOob, "%s: workspace of %zu bytes is above 2 GiB", what, need);
  if (!workspace || ((uintptr_t)workspace & 15) || workspace_bytes < need) {
    set_error("%s: workspace of %zu bytes (16-byte aligned) needed, %zu given", what, need,
              workspace_bytes);
    return PLZ_EWORKSPACE;
  }
  return PLZ_OK;
}

int plz_lut_gemv_planes(const uint16_t* x, const int32_t* planes_items,
                        const uint32_t* palette_items, uint16_t* y, int64_t M, int64_t N, int64_t K,
                        void* workspace, size_t workspace_bytes, void* stream) {
  const char* what = "plz_lut_gemv_planes";
  PLZ_REQUIRE(M >= 1 && M <= 16, "%s: M (%lld) must be in [1, 16]", what, (long long)M);
  PLZ_REQUIRE(N == 0 || K == 0 || (planes_items && palette_items), "%s: null pointer", what);
  plz_gemv_desc d = {x, nullptr, nullptr, y, N, K, 0, 0, palette_items, planes_items};
  int rc = check_desc(d, 0);
  if (rc) return rc;
  if (N == 0) return PLZ_OK;
  if (K == 0) {
    zero_async(y, (size_t)M * N * 2, (hipStream_t)stream);
    return check_launch(what);
  }
  if ((rc = planes_ws_check(1, K, (int)M, workspace, workspace_bytes, what))) return rc;
  const int64_t items = (N + ROWS - 1) / ROWS;
  return launch_pl<false>(items, (hipStream_t)stream, nullptr, 1, d, (int)M, (int)(K / KC),
                          static_cast<uint8_t*>(workspace), workspace_bytes, what);
}

int plz_lut_gemv_grouped_planes(const plz_gemv_desc* descs_device, int n, int64_t total_blocks,
                                int M, int64_t max_K, void* workspace, size_t workspace_bytes,
                                void* stream) {
  const char* what = "plz_lut_gemv_grouped_planes";
  PLZ_REQUIRE(M >= 1 && M <= 16, "%s: M (%d) must be in [1, 16]", what, M);
  PLZ_REQUIRE(n >= 0 && total_blocks >= 0 && max_K >= 0, "%s: negative count", what);
  PLZ_REQUIRE(max_K % KC == 0, "%s: max_K (%lld) must be a multiple of 256", what,
              (long long)max_K);
  if (n == 0 || total_blocks == 0) return PLZ_OK;
  PLZ_REQUIRE(descs_device, "%s: null descriptor table", what);
  PLZ_REQUIRE(max_K > 0, "%s: max_K must be the largest K of the table", what);
  if (int rc = planes_ws_check(n, max_K, M, workspace, workspace_bytes, what)) return rc;
  plz_gemv_desc dummy = {};
  return launch_pl<true>(total_blocks, (hipStream_t)stream, descs_device, n, dummy, M,
                         (int)(max_K / KC), static_cast<uint8_t*>(workspace), workspace_bytes,
                         what);
}

}  // extern "C"
