// Decode GEMV for 1 <= M <= 16 tokens: y[M,N] = x[M,K] W^T, one pass over packed W.
//
// The reference has no decode path; at M = 1 it would run the 64-row-tile forward kernel
// (fused_lut_kernel.cu:309-518). Here the work is bandwidth-bound: 2 bits of index plus
// 0.5 bit of fp32 palette per weight are streamed once, and everything else is arranged so
// that the stream never stops:
//
// * Persistent workgroups, a few per CU. The work items (128 rows of one linear, all of K) of
//   a launch are cut into one contiguous range per workgroup, balanced by bytes (K per item).
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

// Position in a workgroup's stage sequence.
struct Cursor {
  int64_t item, end;
  int kc, nkc;
  plz_gemv_desc d;
  int64_t row0;  // first row of the item
};
template <bool GROUPED>
__device__ __forceinline__ void cursor_load(Cursor& c, const Table<GROUPED>& tb) {
  c.kc = 0;
  if (c.item >= c.end) {  // finished (or empty) range: a harmless, never-live cursor
    c.nkc = 1;
    c.d = plz_gemv_desc{};
    c.row0 = 0;
    return;
  }
  const int di = tb.find_item(c.item);
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
  const int64_t T = tb.total_cost(), G = gridDim.x, wid = blockIdx.x;
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

  const int64_t T = tb.total_cost(), G = gridDim.x, wid = blockIdx.x;
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
  while (cc.item < cc.end) {  // RD stages per pass, unrolled so that ring slots are constants
#pragma unroll
    for (int u = 0; u < RD; ++u) {
      if (cc.item >= cc.end) break;
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
  if (layout != PLZ_GEMV_NATIVE && layout != PLZ_GEMV_DECODE) {
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
    if (nonempty && layout == PLZ_GEMV_DECODE &&
        (!descs[i].packed_items || !descs[i].palette_items)) {
      set_error("plz_gemv_plan: descriptor %d has a null packed_items or palette_items array "
                "(decode layout)", i);
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
  PLZ_REQUIRE(layout == PLZ_GEMV_NATIVE || layout == PLZ_GEMV_DECODE,
              "plz_lut_gemv_grouped: unknown index layout %d", layout);
  PLZ_REQUIRE(n >= 0 && total_blocks >= 0, "plz_lut_gemv_grouped: negative count");
  if (n == 0 || total_blocks == 0) return PLZ_OK;
  PLZ_REQUIRE(descs_device, "plz_lut_gemv_grouped: null descriptor table");
  plz_gemv_desc dummy = {};
  return launch<true>(total_blocks, (hipStream_t)stream, descs_device, n, dummy, M,
                      layout == PLZ_GEMV_DECODE, "plz_lut_gemv_grouped");
}

}  // extern "C"
