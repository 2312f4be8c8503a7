// Decode GEMV for 1 <= M <= 16 tokens: y[M,N] = x[M,K] W^T, one pass over packed W.
//
// The reference has no decode path; at M = 1 it would run the 64-row-tile forward kernel
// (fused_lut_kernel.cu:309-518). Here the work is bandwidth-bound: 2 bits of index plus
// 0.5 bit of fp32 palette per weight are streamed once.
//
// Layout of the work. A workgroup (4 wave64s) owns RB blocks of 16 rows; its 4 waves
// split K by palette groups (wave w takes groups w, w+4, ...) and the partial sums are
// added in LDS at the end in a fixed order. Inside a wave, v_mfma_f32_16x16x32_bf16 computes
// C[n][m] with A = 16 weight rows and B = x^T (columns m >= M are zero). Lane (n = l%16,
// g = l/16) streams 16 bytes of indices = 64 consecutive k of row n per palette group, so
// its 8 MFMA k-slots for a step come from one packed word. The dequantisation of a word
// yields pairs {w_j, w_j+4} and {w_j+8, w_j+12} (the cheapest byte-permute order); the x
// fragment is permuted into the same slot order in registers, which leaves the dot
// product unchanged.
#include "plz_common.h"

namespace plz {

// Dequantise one word into MFMA slot order: s0 = k {0,4,1,5,2,6,3,7}, s1 = k {8,12,...,15}.
__device__ __forceinline__ void dequant16_slots(uint32_t q, PalLut t, u32x4& s0, u32x4& s1) {
  uint32_t a[4], b[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t u = (q >> (2 * j)) & 0x03030303u;
    const uint32_t l = perm(0, t.lo, u), h = perm(0, t.hi, u);
    a[j] = perm(h, l, 0x05010400u);  // {w_j, w_j+4}
    b[j] = perm(h, l, 0x07030602u);  // {w_j+8, w_j+12}
  }
  s0 = u32x4{a[0], a[1], a[2], a[3]};
  s1 = u32x4{b[0], b[1], b[2], b[3]};
}

// x values of one 16-k word (natural order, two uint4) into the same slot order.
__device__ __forceinline__ void xslots(uint4 x0, uint4 x1, u32x4& s0, u32x4& s1) {
  s0 = u32x4{perm(x0.z, x0.x, 0x05040100u), perm(x0.z, x0.x, 0x07060302u),
             perm(x0.w, x0.y, 0x05040100u), perm(x0.w, x0.y, 0x07060302u)};
  s1 = u32x4{perm(x1.z, x1.x, 0x05040100u), perm(x1.z, x1.x, 0x07060302u),
             perm(x1.w, x1.y, 0x05040100u), perm(x1.w, x1.y, 0x07060302u)};
}

template <int RB, bool GROUPED>
__global__ __launch_bounds__(256) void gemv_kernel(const plz_gemv_desc* __restrict__ descs,
                                                   int n_desc, plz_gemv_desc single, int M) {
  __shared__ f32x4 red[4][RB][64];
  const int64_t blk = blockIdx.x;
  plz_gemv_desc d;
  if (GROUPED) {
    int lo = 0, hi = n_desc - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (descs[mid].block_begin <= blk) lo = mid; else hi = mid - 1;
    }
    d = descs[lo];
  } else {
    d = single;
  }
  const int64_t N = d.N, K = d.K;
  const int64_t n0 = (blk - d.block_begin) * (RB * 16);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int64_t wpr = K / kIdxPerWord, gpr = K / kPalGroup;
  const bool xl = nl < M;

  f32x4 acc[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int64_t kg = wave; kg < gpr; kg += 4) {
    // x[m = nl][kg*256 + 64g .. +64) -> 8 slot fragments (steps s = 0..7)
    u32x4 xs[8];
    {
      const uint4* xp = reinterpret_cast<const uint4*>(d.x + (int64_t)nl * K + kg * kPalGroup + 64 * g);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        uint4 x0 = make_uint4(0, 0, 0, 0), x1 = x0;
        if (xl) { x0 = xp[2 * w]; x1 = xp[2 * w + 1]; }
        xslots(x0, x1, xs[2 * w], xs[2 * w + 1]);
      }
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const int64_t n = n0 + 16 * r + nl;
      uint4 q = make_uint4(0, 0, 0, 0);
      float4 p = make_float4(0.f, 0.f, 0.f, 0.f);
      if (n < N) {
        q = *reinterpret_cast<const uint4*>(d.packed + n * wpr + kg * 16 + 4 * g);
        p = *reinterpret_cast<const float4*>(d.palette + (n * gpr + kg) * 4);
      }
      const PalLut t = make_lut(p.x, p.y, p.z, p.w);
      const uint32_t qs[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        u32x4 a0, a1;
        dequant16_slots(qs[w], t, a0, a1);
        acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a0),
                                                         __builtin_bit_cast(bf16x8, xs[2 * w]),
                                                         acc[r], 0, 0, 0);
        acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a1),
                                                         __builtin_bit_cast(bf16x8, xs[2 * w + 1]),
                                                         acc[r], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RB; ++r) red[wave][r][lane] = acc[r];
  __syncthreads();
  if (wave == 0) {
    // acc lane l: C[n = 4*(l/16) + e][m = l%16]
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const f32x4 s = red[0][r][lane] + red[1][r][lane] + red[2][r][lane] + red[3][r][lane];
      const int m = lane & 15;
      if (m < M) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t n = n0 + 16 * r + 4 * (lane >> 4) + e;
          if (n < N) d.y[(int64_t)m * N + n] = (uint16_t)f2bf(s[e]);
        }
      }
    }
  }
}

constexpr int kRbGrouped = 4;
constexpr int kRbSingle = 1;

static int check_desc(const plz_gemv_desc& d, int i) {
  PLZ_REQUIRE(d.N >= 0 && d.K >= 0, "plz_gemv: descriptor %d has a negative shape", i);
  PLZ_REQUIRE(d.K % 256 == 0, "plz_gemv: descriptor %d: K (%lld) must be a multiple of 256", i,
              (long long)d.K);
  PLZ_REQUIRE(d.N == 0 || d.K == 0 || (d.x && d.packed && d.palette && d.y),
              "plz_gemv: descriptor %d has a null pointer", i);
  PLZ_REQUIRE((((uintptr_t)d.x | (uintptr_t)d.packed | (uintptr_t)d.palette) & 15) == 0,
              "plz_gemv: descriptor %d: x, packed and palette must be 16-byte aligned", i);
  return PLZ_OK;
}

}  // namespace plz

using namespace plz;

extern "C" {

int plz_lut_gemv(const uint16_t* x, const int32_t* packed, const float* palette, uint16_t* y,
                 int64_t M, int64_t N, int64_t K, void* stream) {
  PLZ_REQUIRE(M >= 1 && M <= 16, "plz_lut_gemv: M (%lld) must be in [1, 16]", (long long)M);
  plz_gemv_desc d = {x, packed, palette, y, N, K, 0};
  int rc = check_desc(d, 0);
  if (rc) return rc;
  if (N == 0) return PLZ_OK;
  if (K == 0) {
    hipMemsetAsync(y, 0, (size_t)M * N * 2, (hipStream_t)stream);
    return check_launch("plz_lut_gemv");
  }
  const int64_t blocks = (N + 16 * kRbSingle - 1) / (16 * kRbSingle);
  hipLaunchKernelGGL((gemv_kernel<kRbSingle, false>), dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, nullptr, 0, d, (int)M);
  return check_launch("plz_lut_gemv");
}

int64_t plz_gemv_plan(plz_gemv_desc* descs, int n, int M) {
  if (n < 0 || !descs || M < 1 || M > 16) {
    set_error("plz_gemv_plan: need n >= 0, non-null descriptors and M in [1, 16]");
    return -PLZ_EINVAL;
  }
  int64_t total = 0;
  for (int i = 0; i < n; ++i) {
    int rc = check_desc(descs[i], i);
    if (rc) return -rc;
    descs[i].block_begin = total;
    if (descs[i].K > 0) total += (descs[i].N + 16 * kRbGrouped - 1) / (16 * kRbGrouped);
  }
  return total;
}

int plz_lut_gemv_grouped(const plz_gemv_desc* descs_device, int n, int64_t total_blocks, int M,
                         void* stream) {
  PLZ_REQUIRE(M >= 1 && M <= 16, "plz_lut_gemv_grouped: M (%d) must be in [1, 16]", M);
  PLZ_REQUIRE(n >= 0 && total_blocks >= 0, "plz_lut_gemv_grouped: negative count");
  if (n == 0 || total_blocks == 0) return PLZ_OK;
  PLZ_REQUIRE(descs_device, "plz_lut_gemv_grouped: null descriptor table");
  plz_gemv_desc dummy = {};
  hipLaunchKernelGGL((gemv_kernel<kRbGrouped, true>), dim3((unsigned)total_blocks), dim3(256), 0,
                     (hipStream_t)stream, descs_device, n, dummy, M);
  return check_launch("plz_lut_gemv_grouped");
}

}  // extern "C"
