// Shared device/host helpers for the palettize HIP library (gfx950 / CDNA4 only).
//
// Conventions used by every kernel in this library:
//   * bf16 values travel as raw uint16_t bit patterns; conversion fp32->bf16 is
//     round-to-nearest-even (the rounding torch's .to(torch.bfloat16) uses).
//   * A palettized weight W[N,K] is stored as 2-bit indices packed 16 per int32
//     along K, LSB first (index k of a 16-run sits at bits 2*(k%16)), which has the
//     same bytes as the reference's .idx2 packing on little-endian hosts
//     (palettize_core.py:31-42), plus fp32 palettes [N, K/256, 4]: one 4-entry
//     palette per output row and per 256-wide chunk of K.
//   * W[n,k] = bf16(palette[n, k/256, idx[n,k]]) -- the flat gather of
//     qwen_model.py:97-102,185-186 with group_id = n*(K/256) + k/256.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include "palettize_hip.h"

namespace plz {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kPalGroup = 256;   // K-extent of one palette group
constexpr int kIdxPerWord = 16;  // 2-bit indices per int32

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// fp32 -> bf16 bits, round to nearest even; NaN stays a NaN. On the device this is the
// gfx950 conversion instruction (v_cvt_pk_bf16_f32, round to nearest even); the host
// restates it in integer arithmetic (NaN -> quiet NaN with the top payload bits).
__host__ __device__ __forceinline__ uint32_t f2bf(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(uint16_t, (__bf16)f);
#else
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
#endif
}
// Two fp32 -> one dword of bf16 {lo, hi} with a single conversion instruction.
__device__ __forceinline__ uint32_t f2bf2(float lo, float hi) {
  const bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__host__ __device__ __forceinline__ float bf2f(uint32_t b) {
  return __builtin_bit_cast(float, (uint32_t)(b << 16));
}
// fp32 -> fp16 bits (round to nearest even) through the hardware conversion.
__device__ __forceinline__ uint32_t f2h(float f) {
  _Float16 h = (_Float16)f;
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float h2f(uint32_t b) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

// Raw buffer loads: a resource covering [p, p + bytes); a lane whose offset is out of range
// reads zeros (the hardware range check), which replaces per-lane branches.
typedef __amdgpu_buffer_rsrc_t BufRsrc;
constexpr uint32_t kBufOob = 0x80000000u;  // an offset past any buffer this library builds
__device__ __forceinline__ BufRsrc make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ uint4 buf_load16(BufRsrc r, uint32_t off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Byte permute: result byte i = byte sel.byte[i] of the 8-byte value {hi:lo}.
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// A 4-entry palette prepared for byte-permute lookup: `lo` holds the low bytes of
// the four bf16 entries, `hi` their high bytes (entry c in byte c).
struct PalLut {
  uint32_t lo, hi;
};
__device__ __forceinline__ PalLut make_lut(float p0, float p1, float p2, float p3) {
  uint32_t b01 = f2bf2(p0, p1);
  uint32_t b23 = f2bf2(p2, p3);
  PalLut t;
  t.lo = perm(b23, b01, 0x06040200u);
  t.hi = perm(b23, b01, 0x07050301u);
  return t;
}

// Dequantise one packed word (16 indices, natural k order) into 8 dwords of bf16
// pairs: out[j] = {w[2j] (low half), w[2j+1] (high half)}.
__device__ __forceinline__ void dequant16(uint32_t q, PalLut t, uint32_t out[8]) {
  uint32_t u0 = q & 0x03030303u;          // idx 0,4,8,12
  uint32_t u1 = (q >> 2) & 0x03030303u;   // idx 1,5,9,13
  uint32_t u2 = (q >> 4) & 0x03030303u;   // idx 2,6,10,14
  uint32_t u3 = (q >> 6) & 0x03030303u;   // idx 3,7,11,15
  uint32_t l0 = perm(0, t.lo, u0), h0 = perm(0, t.hi, u0);
  uint32_t l1 = perm(0, t.lo, u1), h1 = perm(0, t.hi, u1);
  uint32_t l2 = perm(0, t.lo, u2), h2 = perm(0, t.hi, u2);
  uint32_t l3 = perm(0, t.lo, u3), h3 = perm(0, t.hi, u3);
  // {w_j, w_j+4} and {w_j+8, w_j+12}
  uint32_t a0 = perm(h0, l0, 0x05010400u), b0 = perm(h0, l0, 0x07030602u);
  uint32_t a1 = perm(h1, l1, 0x05010400u), b1 = perm(h1, l1, 0x07030602u);
  uint32_t a2 = perm(h2, l2, 0x05010400u), b2 = perm(h2, l2, 0x07030602u);
  uint32_t a3 = perm(h3, l3, 0x05010400u), b3 = perm(h3, l3, 0x07030602u);
  out[0] = perm(a1, a0, 0x05040100u);  // w0 w1
  out[1] = perm(a3, a2, 0x05040100u);  // w2 w3
  out[2] = perm(a1, a0, 0x07060302u);  // w4 w5
  out[3] = perm(a3, a2, 0x07060302u);  // w6 w7
  out[4] = perm(b1, b0, 0x05040100u);  // w8 w9
  out[5] = perm(b3, b2, 0x05040100u);  // w10 w11
  out[6] = perm(b1, b0, 0x07060302u);  // w12 w13
  out[7] = perm(b3, b2, 0x07060302u);  // w14 w15
}

// Dequantise the same 16 k positions of two rows (n, n+1) into 16 dwords
// out[k] = {w[n][k] (low half), w[n+1][k] (high half)}: the layout a tile whose
// reduction dimension is n wants.
__device__ __forceinline__ void dequant16_pair(uint32_t qa, PalLut ta, uint32_t qb, PalLut tb,
                                               uint32_t out[16]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t ua = (qa >> (2 * j)) & 0x03030303u;  // row n:   idx j, j+4, j+8, j+12
    uint32_t ub = (qb >> (2 * j)) & 0x03030303u;  // row n+1
    uint32_t la = perm(0, ta.lo, ua), ha = perm(0, ta.hi, ua);
    uint32_t lb = perm(0, tb.lo, ub), hb = perm(0, tb.hi, ub);
    uint32_t ll0 = perm(lb, la, 0x05010400u), hh0 = perm(hb, ha, 0x05010400u);  // k=j, j+4
    uint32_t ll1 = perm(lb, la, 0x07030602u), hh1 = perm(hb, ha, 0x07030602u);  // k=j+8, j+12
    out[j] = perm(hh0, ll0, 0x05010400u);
    out[j + 4] = perm(hh0, ll0, 0x07030602u);
    out[j + 8] = perm(hh1, ll1, 0x05010400u);
    out[j + 12] = perm(hh1, ll1, 0x07030602u);
  }
}

// ---- Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11) ---------------------------------
struct U4 {
  uint32_t x, y, z, w;
};
__host__ __device__ __forceinline__ U4 philox4x32_10(U4 c, uint32_t k0, uint32_t k1) {
  const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    const uint64_t p0 = (uint64_t)M0 * c.x, p1 = (uint64_t)M1 * c.z;
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    c = U4{hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0};
    k0 += W0;
    k1 += W1;
  }
  return c;
}

// Natural log of a positive, normal, finite x: log2 from v_log_f32, times ln 2 carried in two
// parts (ln2_hi + ln2_lo, with the rounding error of r * ln2_hi recovered by an fma). This is
// the arithmetic logf performs for such x; logf adds a rescaling of subnormal inputs and a
// pass-through of infinities around it, which these callers never need.
__device__ __forceinline__ float log_normal(float x) {
  const float ln2_hi = 0x1.62e42ep-1f, ln2_lo = 0x1.efa39ep-25f;  // ln2_lo = ln 2 - ln2_hi
  const float r = __builtin_amdgcn_logf(x);
  const float p = r * ln2_hi;
  return __builtin_fmaf(r, ln2_hi, __builtin_fmaf(r, ln2_lo, __builtin_fmaf(r, ln2_hi, -p)));
}

// u = (top 23 bits + 0.5) / 2^23 lies in [2^-24, 1 - 2^-24]: every value is exact in fp32,
// so u never rounds to 1 (which would make the noise +inf). Both logs see normal inputs:
// u >= 2^-24 and -log(u) >= -log(1 - 2^-24) ~ 5.96e-8.
__device__ __forceinline__ float gumbel_from_bits(uint32_t b) {
  const float u = ((float)(b >> 9) + 0.5f) * (1.0f / 8388608.0f);
  return -log_normal(-log_normal(u));
}

// The Gumbel noise of element (n, k, c) of an [N, K, 4] tensor drawn by Philox at counter
// offset + n*K + k: one 128-bit draw gives the 4 classes of one weight.
__device__ __forceinline__ void philox_gumbel4(uint64_t seed, uint64_t ctr, float (&z)[4]) {
  const U4 r = philox4x32_10(U4{(uint32_t)ctr, (uint32_t)(ctr >> 32), 0u, 0u}, (uint32_t)seed,
                             (uint32_t)(seed >> 32));
  z[0] = gumbel_from_bits(r.x);
  z[1] = gumbel_from_bits(r.y);
  z[2] = gumbel_from_bits(r.z);
  z[3] = gumbel_from_bits(r.w);
}

// The soft forward weight of two consecutive weights of a row (fused_lut_kernel.cu:1974-2003;
// triton_soft_forward.py:160-176 for PLZ_W_HARD_PLAIN) from their 8 logits (lw: bf16 or fp16
// bits, weight-major, classes in order), their 8 noise values and the row's palette group pc:
//   P_c = softmax_c((logit_c + noise_c) / tau)   (one reciprocal of the sum)
//   W_soft = sum_c P_c pal_c,   W_hard = pal[argmax P] (first maximum wins), or over the plain
//   logits with PLZ_W_HARD_PLAIN
// wo = bf16 W of the mode, so = bf16 W_soft, po = P as fp16 (the reference's P_aos element
// type; weight-major, classes in order, two per word). The build-W kernels and the optimizer
// step that builds the next forward's W call this one function, so their outputs agree bit for
// bit.
__device__ __forceinline__ void build_w_two(const uint32_t (&lw)[4], int f16, const float (&nz)[8],
                                            const float (&pc)[4], float inv_tau, int mode,
                                            uint32_t (&wo)[2], uint32_t (&so)[2],
                                            uint32_t (&po)[4]) {
#pragma unroll
  for (int el = 0; el < 2; ++el) {
    float l[4], a[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t bits = (lw[2 * el + c / 2] >> (16 * (c & 1))) & 0xffffu;
      l[c] = f16 ? h2f(bits) : bf2f(bits);
      a[c] = (l[c] + nz[4 * el + c]) * inv_tau;
    }
    const float m = fmaxf(fmaxf(a[0], a[1]), fmaxf(a[2], a[3]));
    float e[4], s = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      e[c] = __expf(a[c] - m);
      s += e[c];
    }
    // one reciprocal, as the soft backward's epilogue computes P: both passes see the same P
    const float rs = 1.f / s;
    float P[4], ws = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      P[c] = e[c] * rs;
      ws += P[c] * pc[c];
    }
    // argmax, first maximum wins (strict >), over P (noisy) or over the plain logits
    const float* v = mode == PLZ_W_HARD_PLAIN ? l : P;
    int am = 0;
    float best = v[0];
#pragma unroll
    for (int c = 1; c < 4; ++c)
      if (v[c] > best) { best = v[c]; am = c; }
    const float wh = am == 0 ? pc[0] : am == 1 ? pc[1] : am == 2 ? pc[2] : pc[3];
    wo[el] = f2bf(mode == PLZ_W_SOFT ? ws : wh);
    so[el] = f2bf(ws);
    po[2 * el] = f2h(P[0]) | (f2h(P[1]) << 16);
    po[2 * el + 1] = f2h(P[2]) | (f2h(P[3]) << 16);
  }
}

// SwiGLU of one element as the HF Qwen3 MLP computes it on bf16 tensors: h = bf16(silu(g)) * u
// for bf16 values g, u (the caller rounds h to bf16). Shared by the elementwise kernel and the
// GEMM epilogue, so the fused and unfused paths agree bit for bit on the same g, u.
__device__ __forceinline__ float swiglu_elem(float g, float u) {
  return bf2f(f2bf(g / (1.f + __expf(-g)))) * u;
}

// 8 bf16 values <-> fp32
__device__ __forceinline__ void unpack8(uint4 v, float f[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf2f(w[i] & 0xffffu);
    f[2 * i + 1] = bf2f(w[i] >> 16);
  }
}
__device__ __forceinline__ uint4 pack8(const float f[8]) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = f2bf(f[2 * i]) | (f2bf(f[2 * i + 1]) << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// The SwiGLU's gradients for 8 consecutive elements from bf16 gate, up and grad_h, shared by
// the elementwise backward and the grad_x GEMM epilogue that fuses it (bit for bit the same)
__device__ __forceinline__ void swiglu_bwd8(uint4 gate, uint4 up, uint4 gh, uint4& gg, uint4& gu) {
  float g[8], u[8], d[8], og[8], ou[8];
  unpack8(gate, g);
  unpack8(up, u);
  unpack8(gh, d);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float sg = 1.f / (1.f + __expf(-g[j]));
    const float s = g[j] * sg;
    ou[j] = d[j] * s;
    og[j] = d[j] * u[j] * sg * (1.f + g[j] * (1.f - sg));
  }
  gg = pack8(og);
  gu = pack8(ou);
}

// ---- error reporting shared by every entry point -------------------------------
void set_error(const char* fmt, ...);
int check_launch(const char* what);
void zero_async(void* p, size_t bytes, hipStream_t stream);  // kernel fill, capture-safe
// Raises a kernel's dynamic-LDS limit to `bytes` on the current device, once per device (the
// attribute is per device); `done` is the calling site's bit mask of devices already set up.
int reserve_lds(const void* fn, size_t bytes, uint64_t& done, const char* what);

}  // namespace plz

#define PLZ_REQUIRE(cond, ...)        \
  do {                                \
    if (!(cond)) {                    \
      plz::set_error(__VA_ARGS__);    \
      return PLZ_EINVAL;              \
    }                                 \
  } while (0)
