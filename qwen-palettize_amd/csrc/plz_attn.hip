// Causal grouped-query attention forward for the decoder-layer step (flash-style, MFMA).
//
//   o[b, s, h, :] = softmax_t<=s(q[b, s, h, :] . k[b, t, h / G, :] * scale) v[b, t, h / G, :]
//   lse[b, h, s]  = log-sum-exp of the scaled scores (natural log), kept for the backward
// with q, o bf16 [B, S, Hq, 128], k, v bf16 [B, S, Hkv, 128], G = Hq / Hkv: the layout the
// q/k/v projections produce and o_proj consumes, so no transposes or repeated k/v are needed.
// Replaces torch scaled_dot_product_attention(is_causal=True) of HF Qwen3 attention
// (transformers models/qwen3/modeling_qwen3.py), which the reference runs through sdpa.
//
// A workgroup (4 waves) owns 128 query rows of one head; wave w owns rows 32w..32w+31 and
// keeps their q fragments in registers. Key/value blocks of 64 rows stream through a
// double-buffered LDS ring (buffer_load ... lds). Each wave computes S^T = K Q^T (kv x q,
// 2 blocks of v_mfma_f32_32x32x16_bf16) so that, after the online softmax, its accumulator
// registers are directly the B operand P^T of O^T += V^T P^T: lane l holds query l%32 and the
// kv indices {4h+0..3, 8+4h+0..3} (h = l/32) of each 16-wide k-step, and the V^T fragments are
// read from LDS (ds_read_b64_tr_b16) in that same kv order. The running max and sum of each
// query live in the two lanes that hold it (l and l^32); the max is moved (and O, l rescaled)
// only when a block exceeds it by more than 8 in log2 units, and the causal mask is applied
// only on blocks that cross the diagonal. O^T is transposed through LDS so that the bf16
// output is written with 16-byte stores.
#include <initializer_list>

#include "plz_common.h"
#include "palettize_hip.h"

namespace plz {
namespace attn {

typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int D = 128;        // head dim
constexpr int BM = 128;       // query rows per workgroup
constexpr int BN = 64;        // kv rows per block
constexpr int NT = 256;       // threads
constexpr int TILE = BN * D * 2;  // 16 KB per K or V block
constexpr int KCH = D / 8;        // 16-byte chunks per row (16)

// K tile [64 kv][128 d]: row-fragment reads (A operand, kv = lane%32, d chunk = 2ks + lane/32);
// chunk c of row r sits at c ^ (r & 15): 16 consecutive rows put a chunk on 16 distinct bank
// groups.
__device__ __forceinline__ int k_off(int r, int c) { return r * (KCH * 16) + ((c ^ (r & 15)) << 4); }
// V tile [64 kv][128 d] read with the transposing instruction (d contiguous): chunk c (8 d) of
// row kv sits at c ^ vswz(kv); the reads of 4 consecutive kv x 4 chunks per 16 lanes and the
// copies are conflict-free.
__device__ __forceinline__ int vswz(int kv) { return (kv ^ ((kv & 3) << 2)) & 15; }
__device__ __forceinline__ int v_off(int kv, int c) { return kv * (KCH * 16) + ((c ^ vswz(kv)) << 4); }

// wait until at most N vector-memory operations of this wave are outstanding
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ void dma16(BufRsrc r, lds_u8* dst, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, off, 0, 0, 0);
}

// V^T fragment for k-step ks (kv 16ks..16ks+15 of the block), d rows dbase..dbase+31, in the
// k-slot order of the S^T accumulators: lane l gets d = dbase + l%32 and kv
// {16ks + 4h + 0..3, 16ks + 8 + 4h + 0..3}, h = l/32.
__device__ __forceinline__ bf16x8 vt_frag(const lds_u8* vs, int dbase, int ks, int lane) {
  const int j = lane >> 4, i = lane & 15, t = i >> 2, q = i & 3;
  const int d = dbase + 16 * (j & 1) + 4 * q;
  const int kv1 = 16 * ks + 4 * (j >> 1) + t, kv2 = kv1 + 8;
  const int c = d >> 3, off = (d & 7) * 2;
  const v4i16 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(vs + v_off(kv1, c) + off));
  const v4i16 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(vs + v_off(kv2, c) + off));
  typedef short v8i16 __attribute__((ext_vector_type(8)));
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}

// 2^x by v_exp_f32 alone. exp2f wraps the same instruction in a rescaling of arguments below
// -126 so that it can return subnormal results; here those probabilities (< 2^-126) become 0,
// and every other result, +-inf and NaN included, is the same.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__global__ __launch_bounds__(NT, 2) void attn_fwd_kernel(const uint16_t* __restrict__ q,
                                                      const uint16_t* __restrict__ k,
                                                      const uint16_t* __restrict__ v,
                                                      uint16_t* __restrict__ o,
                                                      float* __restrict__ lse, int B, int S,
                                                      int Hq, int Hkv, float scale_log2) {
  extern __shared__ uint4 smem[];
  lds_u8* lds = (lds_u8*)smem;
  const int lane = threadIdx.x & 63, h2 = lane >> 5, ql = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  // 1-D grid in longest-first order: the last query blocks see the most kv blocks
  int id = blockIdx.x;
  const int qb = S / BM - 1 - id / (Hq * B);
  id %= Hq * B;
  const int h = id % Hq, b = id / Hq;
  const int hk = h / (Hq / Hkv);
  const int q0 = qb * BM;
  const int qrow = q0 + 32 * wave + ql;  // this lane's query
  const int64_t qstride = (int64_t)Hq * D, kstride = (int64_t)Hkv * D;

  // q fragments (B operand of S^T = K Q^T): query qrow, d = 16 ks + 8 h2 .. +7
  bf16x8 qf[D / 16];
  {
    const uint16_t* qp = q + ((int64_t)b * S + qrow) * qstride + (int64_t)h * D + 8 * h2;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks)
      qf[ks] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(qp + 16 * ks));
  }

  // copies of one kv block: 64 rows x 16 chunks per tensor = 1024 chunks = 4 per thread each
  const int64_t kv_bytes = (int64_t)S * kstride * 2;
  const BufRsrc rk = make_rsrc(k + (int64_t)b * S * kstride + (int64_t)hk * D, (uint32_t)kv_bytes);
  const BufRsrc rv = make_rsrc(v + (int64_t)b * S * kstride + (int64_t)hk * D, (uint32_t)kv_bytes);
  uint32_t koff[4], voff[4];
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int pch = it * NT + threadIdx.x;  // physical chunk: lane l writes LDS base + 16 l
    const int r = pch >> 4;
    const int ck = (pch & 15) ^ (r & 15), cv = (pch & 15) ^ vswz(r);
    koff[it] = (uint32_t)(r * kstride * 2 + ck * 16);
    voff[it] = (uint32_t)(r * kstride * 2 + cv * 16);
  }
  const int wb = __builtin_amdgcn_readfirstlane(wave * 1024);
  auto issue = [&](int slot, int kb) {
    lds_u8* ks_ = lds + slot * 2 * TILE;
    const uint32_t base = (uint32_t)(kb * BN) * (uint32_t)(kstride * 2);
#pragma unroll
    for (int it = 0; it < 4; ++it) dma16(rk, ks_ + it * NT * 16 + wb, koff[it] + base);
#pragma unroll
    for (int it = 0; it < 4; ++it) dma16(rv, ks_ + TILE + it * NT * 16 + wb, voff[it] + base);
  };

  f32x16 ot[D / 32];  // O^T blocks: d rows 32 db .. +31, query columns
#pragma unroll
  for (int db = 0; db < D / 32; ++db) ot[db] = f32x16{};
  float mrun = -INFINITY, lrun = 0.f;  // running max (log2 units) and sum of this query

  const int nkb = (q0 + BM) / BN;  // causal: kv blocks up to the last query of the workgroup
  issue(0, 0);
  for (int kb = 0; kb < nkb; ++kb) {
    const int cur = kb & 1;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // block kb landed for everyone; slot cur^1 (block kb-1) is free
    if (kb + 1 < nkb) issue(cur ^ 1, kb + 1);
    const lds_u8* ks_ = lds + cur * 2 * TILE;
    const lds_u8* vs_ = ks_ + TILE;
    const int kv0 = kb * BN;
    if (kv0 > q0 + 32 * wave + 31) continue;  // every query of this wave is before the block
    // S^T = K Q^T: two 32-kv blocks, 8 k-steps over d
    f32x16 st[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const bf16x8 kf = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
                        ks_ + k_off(32 * nb + ql, 2 * ks + h2)));
        st[nb] = mfma32(kf, qf[ks], st[nb]);
      }
    }
    // causal mask (only blocks that cross this wave's diagonal), online softmax in the log2
    // domain on the raw scores: p = exp2(s * scale_log2 - m)
    if (kv0 + BN - 1 > q0 + 32 * wave) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int kv = kv0 + 32 * nb + 8 * (e >> 2) + 4 * h2 + (e & 3);
          if (kv > qrow) st[nb][e] = -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, st[nb][e]);
    mx = fmaxf(mx, __shfl_xor(mx, 32)) * scale_log2;
    // Lazy rescaling: the reference max m only moves when the block max exceeds it by more
    // than 8 (so every p stays <= 2^8, exact in fp32 and in range for bf16); the first block
    // always sets it (kv 0 <= qrow). O and l are rescaled only when some lane moved.
    if (__builtin_amdgcn_ballot_w64(mx > mrun + 8.f) != 0) {
      const float mnew = mx > mrun + 8.f ? mx : mrun;
      const float alpha = exp2_fast(mrun - mnew);
      mrun = mnew;
      lrun *= alpha;
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) ot[db][e] *= alpha;
    }
    const float nm = -mrun;
    float sum = 0.f;
    bf16x8 pf[4];  // P^T fragments for the 4 k-steps of 16 kv
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      float p[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        p[e] = exp2_fast(fmaf(st[nb][e], scale_log2, nm));
        sum += p[e];
      }
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const uint32_t w0 = f2bf2(p[8 * half + 0], p[8 * half + 1]);
        const uint32_t w1 = f2bf2(p[8 * half + 2], p[8 * half + 3]);
        const uint32_t w2 = f2bf2(p[8 * half + 4], p[8 * half + 5]);
        const uint32_t w3 = f2bf2(p[8 * half + 6], p[8 * half + 7]);
        pf[2 * nb + half] = __builtin_bit_cast(bf16x8, u32x4{w0, w1, w2, w3});
      }
    }
    sum += __shfl_xor(sum, 32);
    lrun += sum;
    // O^T += V^T P^T
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int db = 0; db < D / 32; ++db) ot[db] = mfma32(vt_frag(vs_, 32 * db, ks, lane), pf[ks], ot[db]);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // normalise, transpose through LDS (this wave's 32 queries x 128 d, bf16, rows padded to
  // 272 B), write 16-byte chunks of each query row
  const float inv = 1.f / lrun;
  lds_u8* st_ = lds + wave * (32 * 272);
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // accumulator values 4j..4j+3: 4 consecutive d, one 8-B store
      const int d = 32 * db + 8 * j + 4 * h2;
      *reinterpret_cast<__attribute__((address_space(3))) u32x2*>(st_ + ql * 272 + d * 2) =
          u32x2{f2bf2(ot[db][4 * j] * inv, ot[db][4 * j + 1] * inv),
                f2bf2(ot[db][4 * j + 2] * inv, ot[db][4 * j + 3] * inv)};
    }
  if (h2 == 0) lse[((int64_t)b * Hq + h) * S + qrow] = (mrun + log2f(lrun)) * 0.69314718055994531f;
  __syncthreads();
#pragma unroll
  for (int it = 0; it < 8; ++it) {  // 32 rows x 16 chunks = 512 chunks, 8 per lane
    const int ch = it * 64 + lane, r = ch >> 4, c = ch & 15;
    const u32x4 val = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(st_ + r * 272 + c * 16);
    *reinterpret_cast<u32x4*>(o + ((int64_t)b * S + q0 + 32 * wave + r) * qstride +
                              (int64_t)h * D + 8 * c) = val;
  }
}

constexpr size_t kLds = 4 * TILE;  // 64 KB: two K/V blocks (also holds the output staging)

// ---- backward -----------------------------------------------------------------------------
// Two kernels, no atomics (deterministic):
//   attn_bwd_dq_kernel   per 128 queries of one head: D_i = rowsum(dO o O) (written for the
//                        second kernel), then over kv blocks S^T = K Q^T, dP^T = V dO^T,
//                        dS^T = P^T o (dP^T - D), dQ^T += K^T dS^T; dQ = scale dQ.
//   attn_bwd_dkv_kernel  per 128 kv rows of one kv head, over the G query heads sharing it and
//                        the query blocks at or after the kv rows: S = Q K^T, dP = dO V^T,
//                        P, dS as above, dV^T += dO^T P, dK^T += Q^T dS; dK = scale dK.
// The accumulators of S / S^T are directly the B operands of the following products in the
// permuted k order that tr_frag reads (as in the forward). Every [64][128] tile uses the vswz
// layout, which is conflict-free for both row-fragment and transposing reads.

// A or B operand rows r (= lane % 32 row of the tile), d chunk 2 ks + h2
__device__ __forceinline__ bf16x8 row_frag(const lds_u8* t, int r, int ks, int h2) {
  return __builtin_bit_cast(
      bf16x8, *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(t + v_off(r, 2 * ks + h2)));
}

// per-thread source offsets of a [64 rows][128 d] tile copy into the vswz layout (4 chunks)
__device__ __forceinline__ void tile_offsets(uint32_t row_bytes, uint32_t (&off)[4]) {
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int pch = it * NT + threadIdx.x, r = pch >> 4;
    off[it] = (uint32_t)r * row_bytes + (uint32_t)(((pch & 15) ^ vswz(r)) << 4);
  }
}

__device__ __forceinline__ float dot_bf8(u32x4 a, u32x4 b) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    s += bf2f(a[i] & 0xffffu) * bf2f(b[i] & 0xffffu) + bf2f(a[i] >> 16) * bf2f(b[i] >> 16);
  return s;
}

// bf16 B-operand fragments (k-steps 2 mb, 2 mb + 1) from one 32x32 accumulator's values
__device__ __forceinline__ void pack_frags(const float (&x)[16], bf16x8& lo, bf16x8& hi) {
  lo = __builtin_bit_cast(bf16x8, u32x4{f2bf2(x[0], x[1]), f2bf2(x[2], x[3]), f2bf2(x[4], x[5]),
                                        f2bf2(x[6], x[7])});
  hi = __builtin_bit_cast(bf16x8, u32x4{f2bf2(x[8], x[9]), f2bf2(x[10], x[11]),
                                        f2bf2(x[12], x[13]), f2bf2(x[14], x[15])});
}

// write a wave's transposed accumulators (rows d, columns = 32 output rows) as bf16 rows
// [32][128] times mul, through this wave's LDS staging area (32 rows x 272 B)
__device__ __forceinline__ void store_rows_t(const f32x16 (&acc)[D / 32], float mul, lds_u8* st,
                                             uint16_t* out, int64_t row_stride, int lane) {
  const int h2 = lane >> 5, ql = lane & 31;
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // accumulator values 4j..4j+3: 4 consecutive d, one 8-B store
      const int d = 32 * db + 8 * j + 4 * h2;
      *reinterpret_cast<__attribute__((address_space(3))) u32x2*>(st + ql * 272 + d * 2) =
          u32x2{f2bf2(acc[db][4 * j] * mul, acc[db][4 * j + 1] * mul),
                f2bf2(acc[db][4 * j + 2] * mul, acc[db][4 * j + 3] * mul)};
    }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int ch = it * 64 + lane, r = ch >> 4, c = ch & 15;
    const u32x4 val = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(st + r * 272 + c * 16);
    *reinterpret_cast<u32x4*>(out + (int64_t)r * row_stride + 8 * c) = val;
  }
}

constexpr float kLog2e = 1.4426950408889634f;

// grid: S/128 x Hq x B, in longest-first order (the last query blocks see the most kv blocks)
__global__ __launch_bounds__(NT, 2) void attn_bwd_dq_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ o, const uint16_t* __restrict__ dout,
    const float* __restrict__ lse, uint16_t* __restrict__ dq, float* __restrict__ dsum_out,
    float* __restrict__ nl_out, int B,
    int S, int Hq, int Hkv, float scale_log2, float scale) {
  extern __shared__ uint4 smem[];
  lds_u8* lds = (lds_u8*)smem;
  const int lane = threadIdx.x & 63, h2 = lane >> 5, ql = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int nqb = S / BM;
  int id = blockIdx.x;
  const int qb = nqb - 1 - id / (Hq * B);
  id %= Hq * B;
  const int h = id % Hq, b = id / Hq;
  const int hk = h / (Hq / Hkv);
  const int q0 = qb * BM;
  const int qrow = q0 + 32 * wave + ql;
  const int64_t qstride = (int64_t)Hq * D, kstride = (int64_t)Hkv * D;

  bf16x8 qf[D / 16], df[D / 16];
  float dsum = 0.f;
  {
    const int64_t base = ((int64_t)b * S + qrow) * qstride + (int64_t)h * D + 8 * h2;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      const u32x4 qv = *reinterpret_cast<const u32x4*>(q + base + 16 * ks);
      const u32x4 dv = *reinterpret_cast<const u32x4*>(dout + base + 16 * ks);
      const u32x4 ov = *reinterpret_cast<const u32x4*>(o + base + 16 * ks);
      qf[ks] = __builtin_bit_cast(bf16x8, qv);
      df[ks] = __builtin_bit_cast(bf16x8, dv);
      dsum += dot_bf8(dv, ov);
    }
  }
  dsum += __shfl_xor(dsum, 32);
  const int64_t li = ((int64_t)b * Hq + h) * S + qrow;
  const float nl = -lse[li] * kLog2e;
  if (h2 == 0) {
    dsum_out[li] = dsum;
    nl_out[li] = nl;
  }

  const int64_t kv_bytes = (int64_t)S * kstride * 2;
  const BufRsrc rk = make_rsrc(k + (int64_t)b * S * kstride + (int64_t)hk * D, (uint32_t)kv_bytes);
  const BufRsrc rv = make_rsrc(v + (int64_t)b * S * kstride + (int64_t)hk * D, (uint32_t)kv_bytes);
  uint32_t off[4];
  tile_offsets((uint32_t)(kstride * 2), off);
  const int wb = __builtin_amdgcn_readfirstlane(wave * 1024);
  auto issue = [&](int slot, int kb) {
    lds_u8* ks_ = lds + slot * 2 * TILE;
    const uint32_t base = (uint32_t)(kb * BN) * (uint32_t)(kstride * 2);
#pragma unroll
    for (int it = 0; it < 4; ++it) dma16(rk, ks_ + it * NT * 16 + wb, off[it] + base);
#pragma unroll
    for (int it = 0; it < 4; ++it) dma16(rv, ks_ + TILE + it * NT * 16 + wb, off[it] + base);
  };

  // fragment addresses within a K/V slot (lane-dependent, formed once): row fragments of the K
  // and V tiles (A operands of S^T = K Q^T and dP^T = V dO^T) for k-step ks and kv block nb, and
  // the transposed K fragments (A operands of dQ^T += K^T dS^T) for d block db, whose k-step adds
  // 16 rows = 4096 bytes (vswz sees only the low 4 bits of the row)
  uint32_t roff[D / 16][2], toff[D / 32][2];
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) roff[ks][nb] = (uint32_t)v_off(32 * nb + ql, 2 * ks + h2);
  {
    const int j = lane >> 4, i = lane & 15, t4 = i >> 2, q4 = i & 3;
    const int kv1 = 4 * (j >> 1) + t4, kv2 = kv1 + 8;
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      const int d = 32 * db + 16 * (j & 1) + 4 * q4;
      const int c = d >> 3, o2 = (d & 7) * 2;
      toff[db][0] = (uint32_t)(v_off(kv1, c) + o2);
      toff[db][1] = (uint32_t)(v_off(kv2, c) + o2);
    }
  }
  auto rfrag = [&](const lds_u8* base, int ks, int nb) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
                                          base + roff[ks][nb]));
  };
  auto tfrag = [&](const lds_u8* base, int db, int ks) {
    const v4i16 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(base + ks * 4096 + toff[db][0]));
    const v4i16 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(base + ks * 4096 + toff[db][1]));
    typedef short v8i16 __attribute__((ext_vector_type(8)));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  f32x16 dqt[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) dqt[db] = f32x16{};
  const int nkb = (q0 + BM) / BN;
  issue(0, 0);
  for (int kb = 0; kb < nkb; ++kb) {
    const int cur = kb & 1;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (kb + 1 < nkb) issue(cur ^ 1, kb + 1);
    const lds_u8* ks_ = lds + cur * 2 * TILE;
    const lds_u8* vs_ = ks_ + TILE;
    const int kv0 = kb * BN;
    if (kv0 > q0 + 32 * wave + 31) continue;
    f32x16 st[2], dpt[2];
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        st[nb] = mfma32(rfrag(ks_, ks, nb), qf[ks], ks == 0 ? f32x16{} : st[nb]);
        dpt[nb] = mfma32(rfrag(vs_, ks, nb), df[ks], ks == 0 ? f32x16{} : dpt[nb]);
      }
    const bool diag = kv0 + BN - 1 > q0 + 32 * wave;  // the block crosses this wave's diagonal
    bf16x8 dsf[4];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      float p[16], ds[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) p[e] = exp2_fast(fmaf(st[nb][e], scale_log2, nl));
      if (diag) {  // a wave-uniform branch: the other blocks run no mask code
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (kv0 + 32 * nb + 8 * (e >> 2) + 4 * h2 + (e & 3) > qrow) p[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) ds[e] = p[e] * (dpt[nb][e] - dsum);
      pack_frags(ds, dsf[2 * nb], dsf[2 * nb + 1]);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int db = 0; db < D / 32; ++db) dqt[db] = mfma32(tfrag(ks_, db, ks), dsf[ks], dqt[db]);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  store_rows_t(dqt, scale, lds + wave * (32 * 272),
               dq + ((int64_t)b * S + q0 + 32 * wave) * qstride + (int64_t)h * D, qstride, lane);
}

constexpr int BKV = 128;   // kv rows per dK/dV workgroup (32 per wave)
constexpr int BQ = 64;     // query rows per block of the dK/dV loop
constexpr int QRING = 4;   // q-block slots of the dK/dV ring: copies run two blocks ahead
// one slot: Q tile, dO tile, then per wave 128 B: lse and D of the wave's 16 queries of the block
constexpr int QSLOT = 2 * TILE + 512;
constexpr int QCOPIES = 10;  // copy instructions per slot and wave: 4 Q, 4 dO, lse, D
constexpr size_t kLdsDkv =
    2 * 4 * 32 * 272 > QRING * QSLOT ? 2 * 4 * 32 * 272 : (size_t)QRING * QSLOT;

// 8 MFMAs, each followed by fragment reads: two after each of the first four, one after each
// of the others (12 reads: the next step's fragments)
__device__ __forceinline__ void interleave12() {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
}

// One pipelined iteration of the dK/dV loop (phases A and C; phase B follows in the kernel):
// the copies of a later block into dst, then 8 steps of 8 MFMAs, step st = dV/dK of block i
// (slot cs) for k-step st/2 and d blocks 2(st&1), +1, and S/dP of block i+1 (slot ns) for
// k-step st. The fragments of step st+1 are read before the MFMAs of step st; fc holds the
// dV/dK fragments of step 0 on entry (read before the barrier, from a slot completed by the
// previous one) and those of the next iteration's step 0 on return, read from ns during the
// last step together with the next softmax's -lse log2 e and D (nl, dd). The last step issues
// its S/dP MFMAs first, so that its dV/dK MFMAs cover their latency before the softmax reads
// them. cs, ns and dst are distinct slots, and saying so lets the compiler leave the copies in
// flight across the reads.
template <typename Issue>
__device__ __forceinline__ void dkv_step(const lds_u8* __restrict__ cs,
                                         const lds_u8* __restrict__ ns, lds_u8* __restrict__ dst,
                                         const uint32_t (&roff)[D / 16][2],
                                         const uint32_t (&toff)[D / 32][2], uint32_t loff,
                                         const bf16x8 (&kf)[D / 16], const bf16x8 (&vf)[D / 16],
                                         const bf16x8 (&pf)[4], const bf16x8 (&dsf)[4],
                                         f32x16 (&s)[2], f32x16 (&dp)[2], f32x16 (&dvt)[D / 32],
                                         f32x16 (&dkt)[D / 32], bf16x8 (&fc)[4],
                                         f32x4 (&nl)[2][4], f32x4 (&dd)[2][4], Issue&& issue) {
  auto rfrag = [&](int tile, int ks, int mb) {
    return __builtin_bit_cast(
        bf16x8, *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
                    ns + tile * TILE + roff[ks][mb]));
  };
  auto tfrag = [&](const lds_u8* base, int tile, int db, int ks) {
    const v4i16 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_v4i16*)(base + tile * TILE + ks * 4096 + toff[db][0]));
    const v4i16 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_v4i16*)(base + tile * TILE + ks * 4096 + toff[db][1]));
    typedef short v8i16 __attribute__((ext_vector_type(8)));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7));
  };
  // fragments of one step: [0..1] dO^T (d blocks d0, d0+1), [2..3] Q^T, [4..5] Q rows
  // (mb 0, 1), [6..7] dO rows
  auto load_c = [&](const lds_u8* base, int st, bf16x8 (&f)[4]) {
    const int kc = st >> 1, d0 = 2 * (st & 1);
    f[0] = tfrag(base, 1, d0, kc);
    f[1] = tfrag(base, 1, d0 + 1, kc);
    f[2] = tfrag(base, 0, d0, kc);
    f[3] = tfrag(base, 0, d0 + 1, kc);
  };
  auto load_a = [&](int st, bf16x8 (&f)[4]) {
    f[0] = rfrag(0, st, 0);
    f[1] = rfrag(0, st, 1);
    f[2] = rfrag(1, st, 0);
    f[3] = rfrag(1, st, 1);
  };
  auto mma_c = [&](int st, const bf16x8 (&f)[4]) {
    const int kc = st >> 1, d0 = 2 * (st & 1);
    dvt[d0] = mfma32(f[0], pf[kc], dvt[d0]);
    dkt[d0] = mfma32(f[2], dsf[kc], dkt[d0]);
    dvt[d0 + 1] = mfma32(f[1], pf[kc], dvt[d0 + 1]);
    dkt[d0 + 1] = mfma32(f[3], dsf[kc], dkt[d0 + 1]);
  };
  auto mma_a = [&](int st, const bf16x8 (&f)[4]) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      s[mb] = mfma32(f[mb], kf[st], st == 0 ? f32x16{} : s[mb]);
      dp[mb] = mfma32(f[2 + mb], vf[st], st == 0 ? f32x16{} : dp[mb]);
    }
  };
  bf16x8 ca[4], cb[4], aa[4], ab[4];
  issue(dst);
  load_a(0, aa);
  __builtin_amdgcn_sched_barrier(0);
  // step 0 (dV/dK fragments from fc)
  load_c(cs, 1, cb);
  load_a(1, ab);
  mma_c(0, fc);
  mma_a(0, aa);
  interleave12();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int st = 1; st < 7; st += 2) {
    load_c(cs, st + 1, ca);
    load_a(st + 1, aa);
    mma_c(st, cb);
    mma_a(st, ab);
    interleave12();
    __builtin_amdgcn_sched_barrier(0);
    load_c(cs, st + 2, cb);
    load_a(st + 2, ab);
    mma_c(st + 1, ca);
    mma_a(st + 1, aa);
    interleave12();
    __builtin_amdgcn_sched_barrier(0);
  }
  // step 7: S/dP first; reads of the next iteration's step-0 dV/dK fragments and of the next
  // softmax's -lse log2 e and D (queries r = 32 mb + 8 j + 4 h2 + 0..3 of block i+1)
  load_c(ns, 0, fc);
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const lds_u8* a = ns + 2 * TILE + loff + 128 * (2 * mb + (j >> 1)) + 32 * (j & 1);
      nl[mb][j] = *reinterpret_cast<const __attribute__((address_space(3))) f32x4*>(a);
      dd[mb][j] = *reinterpret_cast<const __attribute__((address_space(3))) f32x4*>(a + 64);
    }
  mma_a(7, ab);
  mma_c(7, cb);
#pragma unroll
  for (int m = 0; m < 8; ++m) {  // 24 reads: three after each MFMA
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
}

// grid: S/128 x Hkv x B, in longest-first order (the first kv blocks see the most queries).
// The loop over the (query head, query block) pairs t is software-pipelined: iteration i issues
// the MFMAs of S, dP for block i+1 (phase A) interleaved with those of dV, dK for block i
// (phase C), then the softmax algebra of block i+1 (phase B: P, dS as bf16 fragments). So the
// VALU work of a block never waits on MFMAs just issued, and the matrix core always has
// independent MFMAs queued. The blocks go through a 4-slot LDS ring, copied two blocks ahead:
// the barrier at the top of iteration i completes block i+1 and frees the slot of block i-1,
// which then receives block i+3. Every wave runs every block; blocks that lie entirely before
// a wave's kv rows are masked to P = 0 like the diagonal ones (about a tenth more MFMAs than
// skipping them, in exchange for one instruction stream).
__global__ __launch_bounds__(NT) void attn_bwd_dkv_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ dout, const float* __restrict__ nlse,
    const float* __restrict__ dsum, uint16_t* __restrict__ dk, uint16_t* __restrict__ dv, int B,
    int S, int Hq, int Hkv, float scale_log2, float scale) {
  extern __shared__ uint4 smem[];
  lds_u8* lds = (lds_u8*)smem;
  const int lane = threadIdx.x & 63, h2 = lane >> 5, ql = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  int id = blockIdx.x;
  const int kb = id / (Hkv * B);
  id %= Hkv * B;
  const int hk = id % Hkv, b = id / Hkv;
  const int G = Hq / Hkv;
  const int kv0 = kb * BKV, kvw = kv0 + 32 * wave, kvrow = kvw + ql;
  const int64_t qstride = (int64_t)Hq * D, kstride = (int64_t)Hkv * D;

  bf16x8 kf[D / 16], vf[D / 16];
  {
    const int64_t base = ((int64_t)b * S + kvrow) * kstride + (int64_t)hk * D + 8 * h2;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      kf[ks] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(k + base + 16 * ks));
      vf[ks] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(v + base + 16 * ks));
    }
  }

  uint32_t off[4];
  tile_offsets((uint32_t)(qstride * 2), off);
  const int wb = __builtin_amdgcn_readfirstlane(wave * 1024);
  const int qstart = kv0 / BQ, nq = S / BQ - qstart, T = G * nq;
  const int64_t q_bytes = (int64_t)S * qstride * 2;
  auto slot = [&](int t) { return lds + (t & (QRING - 1)) * QSLOT; };
  // copies of block t into its slot (past the last block: block T-1 again, so that every
  // iteration issues the same number of copies; its slot is free then)
  auto issue = [&](int t, lds_u8* qs) {
    const int tt = t < T ? t : T - 1;
    const int g = tt / nq, qblk = qstart + tt % nq, h = hk * G + g;
    const int64_t hoff = (int64_t)b * S * qstride + (int64_t)h * D;
    const BufRsrc rq = make_rsrc(q + hoff, (uint32_t)q_bytes);
    const BufRsrc rd = make_rsrc(dout + hoff, (uint32_t)q_bytes);
    const uint32_t base = (uint32_t)(qblk * BQ) * (uint32_t)(qstride * 2);
#pragma unroll
    for (int it = 0; it < 4; ++it) dma16(rq, qs + it * NT * 16 + wb, off[it] + base);
#pragma unroll
    for (int it = 0; it < 4; ++it) dma16(rd, qs + TILE + it * NT * 16 + wb, off[it] + base);
    // lanes 0..3: -lse log2 e of queries 16 wave .. +15 of the block; lanes 4..7: their D
    const int64_t row = ((int64_t)b * Hq + h) * S;
    const uint32_t loff = (uint32_t)(qblk * BQ + 16 * wave + 4 * (lane & 3)) * 4;
    lds_u8* ldst = qs + 2 * TILE + 128 * wave;
    if (lane < 4) dma16(make_rsrc(nlse + row, (uint32_t)S * 4), ldst, loff);
    if (lane >= 4 && lane < 8) dma16(make_rsrc(dsum + row, (uint32_t)S * 4), ldst, loff);
  };

  // fragment addresses within a slot (lane-dependent, formed once): row fragments of the Q and
  // dO tiles (A operands of S = Q K^T and dP = dO V^T) for k-step ks and row block mb, and the
  // transposed fragments (A operands of dV^T += dO^T P and dK^T += Q^T dS) for d block db, whose
  // k-step adds 16 rows = 4096 bytes (vswz sees only the low 4 bits of the row)
  // this lane's queries' -lse log2 e and D within a slot's 512 B: 16 h2 bytes into each
  // 32-byte half of a wave's 128 B (queries r = 32 mb + 8 j + 4 h2 + 0..3)
  const uint32_t loff = 16 * h2;
  uint32_t roff[D / 16][2], toff[D / 32][2];
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks)
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) roff[ks][mb] = (uint32_t)v_off(32 * mb + ql, 2 * ks + h2);
  {
    const int j = lane >> 4, i = lane & 15, t4 = i >> 2, q4 = i & 3;
    const int kv1 = 4 * (j >> 1) + t4, kv2 = kv1 + 8;
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      const int d = 32 * db + 16 * (j & 1) + 4 * q4;
      const int c = d >> 3, o2 = (d & 7) * 2;
      toff[db][0] = (uint32_t)(v_off(kv1, c) + o2);
      toff[db][1] = (uint32_t)(v_off(kv2, c) + o2);
    }
  }
  auto rfrag = [&](const lds_u8* base, int tile, int ks, int mb) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
                                          base + tile * TILE + roff[ks][mb]));
  };
  auto tfrag = [&](const lds_u8* base, int tile, int db, int ks) {
    const v4i16 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_v4i16*)(base + tile * TILE + ks * 4096 + toff[db][0]));
    const v4i16 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_v4i16*)(base + tile * TILE + ks * 4096 + toff[db][1]));
    typedef short v8i16 __attribute__((ext_vector_type(8)));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  f32x16 dvt[D / 32], dkt[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) dvt[db] = dkt[db] = f32x16{};
  f32x16 s[2], dp[2];
  bf16x8 pf[4], dsf[4];

  // phase B: P and dS of block t (its S, dP in s, dp) as bf16 B-operand fragments
  auto softmax = [&](int t, const f32x4 (&L)[2][4], const f32x4 (&Dv)[2][4]) {
    const int qb0 = (qstart + t % nq) * BQ;
    const bool diag = qb0 < kvw + 31;  // some query of the block precedes a kv row of the wave
    float p[2][16];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        p[mb][e] = exp2_fast(fmaf(s[mb][e], scale_log2, L[mb][e >> 2][e & 3]));
    if (diag) {  // a wave-uniform branch: the other blocks run no mask code
      asm volatile("");  // (keeps the compiler from turning the branch into selects for all)
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (qb0 + 32 * mb + 8 * (e >> 2) + 4 * h2 + (e & 3) < kvrow) p[mb][e] = 0.f;
    }
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      float ds[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) ds[e] = p[mb][e] * (dp[mb][e] - Dv[mb][e >> 2][e & 3]);
      pack_frags(p[mb], pf[2 * mb], pf[2 * mb + 1]);
      pack_frags(ds, dsf[2 * mb], dsf[2 * mb + 1]);
    }
  };

  // prologue: blocks 0..2 in flight; block 0 complete; S, dP and P, dS of block 0
  issue(0, slot(0));
  issue(1, slot(1));
  issue(2, slot(2));
  wait_vmcnt<2 * QCOPIES>();
  __syncthreads();
  {
    const lds_u8* qs = slot(0);
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks)
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const f32x16 zs = ks == 0 ? f32x16{} : s[mb];
        const f32x16 zd = ks == 0 ? f32x16{} : dp[mb];
        s[mb] = mfma32(rfrag(qs, 0, ks, mb), kf[ks], zs);
        dp[mb] = mfma32(rfrag(qs, 1, ks, mb), vf[ks], zd);
      }
    f32x4 L[2][4], Dv[2][4];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const lds_u8* a = qs + 2 * TILE + loff + 128 * (2 * mb + (j >> 1)) + 32 * (j & 1);
        L[mb][j] = *reinterpret_cast<const __attribute__((address_space(3))) f32x4*>(a);
        Dv[mb][j] = *reinterpret_cast<const __attribute__((address_space(3))) f32x4*>(a + 64);
      }
    softmax(0, L, Dv);
  }

  // dV/dK fragments of step 0 of the first iteration (block 0)
  bf16x8 fc[4];
  fc[0] = tfrag(slot(0), 1, 0, 0);
  fc[1] = tfrag(slot(0), 1, 1, 0);
  fc[2] = tfrag(slot(0), 0, 0, 0);
  fc[3] = tfrag(slot(0), 0, 1, 0);
  for (int i = 0; i + 1 < T; ++i) {
    wait_vmcnt<QCOPIES>();  // block i+1 has landed (block i+2 may not)
    __syncthreads();        // ... for every wave; no wave reads block i-1's slot any more
    f32x4 L[2][4], Dv[2][4];
    dkv_step(slot(i), slot(i + 1), slot(i + 3), roff, toff, loff, kf, vf, pf, dsf, s, dp, dvt,
             dkt, fc, L, Dv, [&](lds_u8* dst) { issue(i + 3, dst); });
    softmax(i + 1, L, Dv);
  }
  // phase C of the last block (its slot was completed by the last iteration's barrier)
  {
    const lds_u8* cs = slot(T - 1);
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
#pragma unroll
      for (int db = 0; db < D / 32; ++db) {
        dvt[db] = mfma32(tfrag(cs, 1, db, kc), pf[kc], dvt[db]);
        dkt[db] = mfma32(tfrag(cs, 0, db, kc), dsf[kc], dkt[db]);
      }
  }
  __builtin_amdgcn_s_waitcnt(0);  // the repeated copies past the last block
  __syncthreads();
  const int64_t orow = ((int64_t)b * S + kvw) * kstride + (int64_t)hk * D;
  store_rows_t(dkt, scale, lds + wave * (32 * 272), dk + orow, kstride, lane);
  store_rows_t(dvt, 1.f, lds + (4 + wave) * (32 * 272), dv + orow, kstride, lane);
}

}  // namespace attn
}  // namespace plz

using namespace plz;
using namespace plz::attn;

namespace {

// shared argument checks of the forward and backward: PLZ_OK, an error status, or kEmpty
// (valid, nothing to do)
constexpr int kEmpty = -1;
int check_shape(const char* what, int batch, int seq, int heads, int kv_heads, int head_dim,
                float scale) {
  PLZ_REQUIRE(batch >= 0 && seq >= 0 && heads > 0 && kv_heads > 0 && heads % kv_heads == 0,
              "%s: need heads a positive multiple of kv_heads", what);
  if (head_dim != D) {
    set_error("%s: head_dim %d is not supported (128 only)", what, head_dim);
    return PLZ_EUNSUPPORTED;
  }
  PLZ_REQUIRE(seq % BM == 0, "%s: seq (%d) must be a multiple of %d", what, seq, BM);
  PLZ_REQUIRE(scale > 0.f, "%s: scale must be positive", what);
  PLZ_REQUIRE((int64_t)seq * heads * D * 2 < ((int64_t)1 << 31),
              "%s: one sequence of q must span < 2 GiB", what);
  return batch == 0 || seq == 0 ? kEmpty : PLZ_OK;
}

bool aligned16(std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if ((uintptr_t)p & 15) return false;
  return true;
}

}  // namespace

extern "C" {

int plz_attn_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, float* lse,
                 int batch, int seq, int heads, int kv_heads, int head_dim, float scale,
                 void* stream) {
  const int rc = check_shape("plz_attn_fwd", batch, seq, heads, kv_heads, head_dim, scale);
  if (rc != PLZ_OK) return rc == kEmpty ? PLZ_OK : rc;
  PLZ_REQUIRE(q && k && v && o && lse, "plz_attn_fwd: null pointer");
  PLZ_REQUIRE(aligned16({q, k, v, o}), "plz_attn_fwd: q, k, v, o must be 16-byte aligned");
  static uint64_t lds_done = 0;
  const int lr = reserve_lds((const void*)attn_fwd_kernel, kLds, lds_done, "plz_attn_fwd");
  if (lr != PLZ_OK) return lr;
  const float scale_log2 = scale * kLog2e;
  hipLaunchKernelGGL(attn_fwd_kernel, dim3((unsigned)(seq / BM) * heads * batch), dim3(NT), kLds, (hipStream_t)stream, q, k, v, o, lse, batch, seq, heads,
                     kv_heads, scale_log2);
  return check_launch("plz_attn_fwd");
}

size_t plz_attn_bwd_workspace(int batch, int seq, int heads) {
  if (batch <= 0 || seq <= 0 || heads <= 0) return 0;
  return 2 * (size_t)batch * (size_t)heads * (size_t)seq * sizeof(float);
}

int plz_attn_bwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* o,
                 const uint16_t* grad_o, const float* lse, uint16_t* grad_q, uint16_t* grad_k,
                 uint16_t* grad_v, void* workspace, size_t workspace_bytes, int batch, int seq,
                 int heads, int kv_heads, int head_dim, float scale, void* stream) {
  const int rc = check_shape("plz_attn_bwd", batch, seq, heads, kv_heads, head_dim, scale);
  if (rc != PLZ_OK) return rc == kEmpty ? PLZ_OK : rc;
  PLZ_REQUIRE(q && k && v && o && grad_o && lse && grad_q && grad_k && grad_v,
              "plz_attn_bwd: null pointer");
  PLZ_REQUIRE(aligned16({q, k, v, o, grad_o, lse, grad_q, grad_k, grad_v}),
              "plz_attn_bwd: every tensor must be 16-byte aligned");
  if (!workspace || workspace_bytes < plz_attn_bwd_workspace(batch, seq, heads) ||
      ((uintptr_t)workspace & 15)) {
    set_error("plz_attn_bwd: workspace of %zu bytes (16-byte aligned) required",
              plz_attn_bwd_workspace(batch, seq, heads));
    return PLZ_EWORKSPACE;
  }
  static uint64_t lds_dq = 0, lds_dkv = 0;
  int lr = reserve_lds((const void*)attn_bwd_dq_kernel, kLds, lds_dq, "plz_attn_bwd");
  if (lr == PLZ_OK)
    lr = reserve_lds((const void*)attn_bwd_dkv_kernel, kLdsDkv, lds_dkv, "plz_attn_bwd");
  if (lr != PLZ_OK) return lr;
  const float scale_log2 = scale * kLog2e;
  float* dsum = (float*)workspace;  // rowsum(grad_o * o), then -lse log2 e
  float* nlse = dsum + (size_t)batch * heads * seq;
  hipLaunchKernelGGL(attn_bwd_dq_kernel, dim3((unsigned)(seq / BM) * heads * batch), dim3(NT), kLds,
                     (hipStream_t)stream, q, k, v, o, grad_o, lse, grad_q, dsum, nlse, batch, seq,
                     heads, kv_heads, scale_log2, scale);
  int r = check_launch("plz_attn_bwd (dq)");
  if (r != PLZ_OK) return r;
  hipLaunchKernelGGL(attn_bwd_dkv_kernel, dim3((unsigned)(seq / BKV) * kv_heads * batch), dim3(NT),
                     kLdsDkv, (hipStream_t)stream, q, k, v, grad_o, nlse, dsum, grad_k, grad_v,
                     batch, seq, heads, kv_heads, scale_log2, scale);
  return check_launch("plz_attn_bwd (dk, dv)");
}

}  // extern "C"
