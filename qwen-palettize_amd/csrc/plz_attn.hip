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
// query live in the two lanes that hold it (l and l^32). O^T is transposed through LDS so that
// the bf16 output is written with 16-byte stores.
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

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__global__ __launch_bounds__(NT) void attn_fwd_kernel(const uint16_t* __restrict__ q,
                                                      const uint16_t* __restrict__ k,
                                                      const uint16_t* __restrict__ v,
                                                      uint16_t* __restrict__ o,
                                                      float* __restrict__ lse, int B, int S,
                                                      int Hq, int Hkv, float scale_log2) {
  extern __shared__ uint4 smem[];
  lds_u8* lds = (lds_u8*)smem;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h2 = lane >> 5, ql = lane & 31;
  const int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
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
    // scale, causal mask, online softmax (log2 domain)
    float mx = -INFINITY;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int kv = kv0 + 32 * nb + 8 * (e >> 2) + 4 * h2 + (e & 3);
        const float s = kv <= qrow ? st[nb][e] * scale_log2 : -INFINITY;
        st[nb][e] = s;
        mx = fmaxf(mx, s);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mnew = fmaxf(mrun, mx);  // finite: block 0 always holds kv 0 <= qrow
    const float alpha = exp2f(mrun - mnew);
    float sum = 0.f;
    bf16x8 pf[4];  // P^T fragments for the 4 k-steps of 16 kv
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      float p[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        p[e] = exp2f(st[nb][e] - mnew);
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
    lrun = lrun * alpha + sum;
    mrun = mnew;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) ot[db][e] *= alpha;
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
    for (int e = 0; e < 16; ++e) {
      const int d = 32 * db + 8 * (e >> 2) + 4 * h2 + (e & 3);
      *reinterpret_cast<__attribute__((address_space(3))) uint16_t*>(st_ + ql * 272 + d * 2) =
          (uint16_t)f2bf(ot[db][e] * inv);
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

}  // namespace attn
}  // namespace plz

using namespace plz;
using namespace plz::attn;

extern "C" {

int plz_attn_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, float* lse,
                 int batch, int seq, int heads, int kv_heads, int head_dim, float scale,
                 void* stream) {
  PLZ_REQUIRE(batch >= 0 && seq >= 0 && heads > 0 && kv_heads > 0 && heads % kv_heads == 0,
              "plz_attn_fwd: need heads a positive multiple of kv_heads");
  if (head_dim != D) {
    set_error("plz_attn_fwd: head_dim %d is not supported (128 only)", head_dim);
    return PLZ_EUNSUPPORTED;
  }
  PLZ_REQUIRE(seq % BM == 0, "plz_attn_fwd: seq (%d) must be a multiple of %d", seq, BM);
  PLZ_REQUIRE(scale > 0.f, "plz_attn_fwd: scale must be positive");
  if (batch == 0 || seq == 0) return PLZ_OK;
  PLZ_REQUIRE(q && k && v && o && lse, "plz_attn_fwd: null pointer");
  PLZ_REQUIRE((((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)o) & 15) == 0,
              "plz_attn_fwd: q, k, v, o must be 16-byte aligned");
  PLZ_REQUIRE((int64_t)seq * kv_heads * D * 2 < ((int64_t)1 << 31),
              "plz_attn_fwd: one sequence of k or v must span < 2 GiB");
  static bool attr = false;
  if (!attr) {
    const hipError_t e = hipFuncSetAttribute((const void*)attn_fwd_kernel,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLds);
    if (e != hipSuccess) {
      set_error("plz_attn_fwd: cannot reserve %zu bytes of LDS: %s", kLds, hipGetErrorString(e));
      return PLZ_EHIP;
    }
    attr = true;
  }
  const float scale_log2 = scale * 1.4426950408889634f;
  hipLaunchKernelGGL(attn_fwd_kernel, dim3((unsigned)(seq / BM), (unsigned)heads, (unsigned)batch),
                     dim3(NT), kLds, (hipStream_t)stream, q, k, v, o, lse, batch, seq, heads,
                     kv_heads, scale_log2);
  return check_launch("plz_attn_fwd");
}

}  // extern "C"
