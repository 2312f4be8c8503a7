/* CPU oracle, C part -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker; no product code path calls it.
 *
 * Bit-level restatements of the reference's algorithms for the LUT-linear path:
 *   orc_pack / orc_unpack   2-bit LSB-first packing, 4 indices per byte
 *                           (palettize_core.py:31-42 pack_idx2, :159-164 unpack_idx2),
 *                           viewed as 16 indices per little-endian int32 along a row
 *   orc_dequant             W[n,k] = bf16_rne(palette[n, k/256, idx[n,k]])
 *                           (the flat gather of qwen_model.py:97-102,185-186)
 *   orc_gumbel_lcg          the reference's LCG hash sampler, element (n,k,c) drawn with
 *                           idx = (k*N + n)*4 + c, stored [N, K, 4]: the CUDA hash in uint32
 *                           (fused_lut_kernel.cu:1245-1256) or the Triton one in int32 with
 *                           arithmetic shifts (triton_soft_forward.py:51-66)
 *   orc_philox / orc_gumbel_philox
 *                           Philox4x32-10 (Salmon et al., SC'11) and the supplied-noise
 *                           generator of this build (no reference counterpart; pinned by
 *                           the Random123 known-answer vectors in the tests)
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

uint16_t orc_f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* idx: rows*cols uint8 in 0..3 (cols % 16 == 0) -> packed rows*(cols/16) int32 */
void orc_pack(const uint8_t* idx, int32_t* packed, int64_t n_words) {
  for (int64_t w = 0; w < n_words; ++w) {
    uint8_t bytes[4];
    for (int b = 0; b < 4; ++b) {
      uint8_t v = 0;
      for (int j = 0; j < 4; ++j) v |= (uint8_t)((idx[w * 16 + 4 * b + j] & 3u) << (2 * j));
      bytes[b] = v;
    }
    uint32_t q = (uint32_t)bytes[0] | ((uint32_t)bytes[1] << 8) | ((uint32_t)bytes[2] << 16) |
                 ((uint32_t)bytes[3] << 24);
    packed[w] = (int32_t)q;
  }
}

void orc_unpack(const int32_t* packed, uint8_t* idx, int64_t n_words) {
  for (int64_t w = 0; w < n_words; ++w) {
    uint32_t q = (uint32_t)packed[w];
    for (int i = 0; i < 16; ++i) idx[w * 16 + i] = (uint8_t)((q >> (2 * i)) & 3u);
  }
}

void orc_dequant(const int32_t* packed, const float* pal, uint16_t* w, int64_t N, int64_t K) {
  const int64_t G = K / 256, wpr = K / 16;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k) {
      uint32_t q = (uint32_t)packed[n * wpr + k / 16];
      uint32_t c = (q >> (2 * (k % 16))) & 3u;
      w[n * K + k] = orc_f2bf(pal[(n * G + k / 256) * 4 + c]);
    }
}

/* x >> s on an int32 as an arithmetic shift, written out on the uint32 bit pattern */
static uint32_t sra32(uint32_t x, int s) {
  return (x >> s) | ((x & 0x80000000u) ? ~(0xFFFFFFFFu >> s) : 0u);
}

/* 24-bit integer of the hash; arith != 0 shifts as the Triton sampler's int32 does
 * (triton_soft_forward.py:58-62), else logically as the CUDA one (fused_lut_kernel.cu:1247-1251).
 * Wrapping multiplies and adds are the same bits in both. */
static uint32_t lcg24(uint32_t seed, uint32_t idx, int arith) {
  uint32_t x = seed ^ (idx * 0x9E3779B9u);
  x ^= arith ? sra32(x, 13) : x >> 13;
  x = x * 1103515245u + 12345u;
  x ^= arith ? sra32(x, 17) : x >> 17;
  x = x * 1103515245u + 12345u;
  return x & 0xFFFFFFu;
}

static float lcg_gumbel(uint32_t seed, uint32_t idx, int arith) {
  float u = (float)lcg24(seed, idx, arith) * (1.0f / 16777216.0f);
  if (u < 1e-7f) u = 1e-7f;
  return -logf(-logf(u));
}

/* raw 24-bit uniform integers of the hash (bit-exact check target) */
void orc_lcg_bits(uint32_t* out, uint32_t seed, const uint32_t* idx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = lcg24(seed, idx[i], 0);
}

void orc_lcg_bits_i32(uint32_t* out, uint32_t seed, const uint32_t* idx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = lcg24(seed, idx[i], 1);
}

void orc_gumbel_lcg(float* out, uint32_t seed, int64_t N, int64_t K, int arith) {
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k) {
      uint32_t base = ((uint32_t)k * (uint32_t)N + (uint32_t)n) * 4u;
      for (int c = 0; c < 4; ++c)
        out[(n * K + k) * 4 + c] = lcg_gumbel(seed, base + (uint32_t)c, arith);
    }
}

void orc_philox(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
  uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
  uint32_t k0 = key_in[0], k1 = key_in[1];
  for (int i = 0; i < 10; ++i) {
    uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
    uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    uint32_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

void orc_gumbel_philox(float* out, int64_t n, uint64_t seed, uint64_t offset) {
  const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  for (int64_t t = 0; t < n / 4; ++t) {
    uint64_t ctr = offset + (uint64_t)t;
    uint32_t c[4] = {(uint32_t)ctr, (uint32_t)(ctr >> 32), 0u, 0u}, r[4];
    orc_philox(c, key, r);
    for (int j = 0; j < 4; ++j) {
      float u = ((float)(r[j] >> 9) + 0.5f) * (1.0f / 8388608.0f);
      out[4 * t + j] = -logf(-logf(u));
    }
  }
}
