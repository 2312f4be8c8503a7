// Decode GEMV for 1 <= M <= 16 tokens: y[M,N] = x[M,K] W^T, one pass over packed W.
//
// The reference has no decode path; at M = 1 it would run the 64-row-tile forward kernel
// (fused_lut_kernel.cu:309-518). Here the work is bandwidth-bound: 2 bits of index plus
// 0.5 bit of fp32 palette per weight are streamed once.
//
// Layout of the work. A workgroup (4 wave64s) owns 64*RB rows and streams the whole of K
// in iterations of 4 palette groups (1024 k). Wave w owns RB blocks of 16 rows. Lane
// (n = l%16, q = l/16) works on row n and palette group 4*it + q: it reads that group's 64
// bytes of indices (4 x 16 B, contiguous) and its 16-byte palette, so the four lanes of a
// row read 256 contiguous bytes of indices and 64 contiguous bytes of palettes per
// iteration. These loads are issued one iteration ahead of their use.
// x is shared by every wave: each iteration's x chunk is loaded once per workgroup,
// permuted into MFMA fragment order and kept in LDS (2 KB per token, double buffered, one
// barrier per iteration); waves read their fragments with one 16-byte LDS read each. A
// GEMV that loads x per wave is limited by the vector-memory data-return path, not HBM.
// Inside a wave, v_mfma_f32_16x16x32_bf16 computes C[n][m] with A = 16 weight rows and
// B = x^T. Fragment lanes of tokens m >= M repeat token M-1: they only feed output columns
// m >= M, which are never stored. The four lane quarters feed different palette groups
// into the same MFMA, which is fine because the product sums over every k. A packed word
// dequantises into the slots {w_j, w_j+4} and {w_j+8, w_j+12} (the cheapest byte-permute
// order); the x fragments are permuted into the same slot order, which leaves the dot
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

// Workgroup barrier without the memory fence of __syncthreads(), which would also wait for
// the weight loads in flight: this wave's LDS operations complete, then s_barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xF | (3 << 14) | (7 << 4));  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// LDS x fragments of one iteration: [sub-step 4][fragment 8][quarter 4][token m < M] x 16 B
// = 2 KB per token, double buffered (dynamic LDS: 4 KB x M per workgroup).
constexpr int kXFragBytesPerToken = 4 * 8 * 4 * 16;
constexpr int kGemvRb = 2;                 // row blocks of 16 per wave
constexpr int kGemvRows = 64 * kGemvRb;   // rows per workgroup

template <int RB, bool GROUPED>
__global__ __launch_bounds__(256) void gemv_kernel(const plz_gemv_desc* __restrict__ descs,
                                                   int n_desc, plz_gemv_desc single, int M) {
  extern __shared__ u32x4 xlds[];  // [2][4*8*4*M]
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
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row0 = (blk - d.block_begin) * (64 * RB) + wave * (16 * RB);
  const bool has_rows = row0 < N;  // waves without rows still take part in the barriers
  const int nl = lane & 15, qg = lane >> 4;
  const int gpr = (int)(K / kPalGroup);
  const int iters = (gpr + 3) / 4;
  // sizes were checked on the host to fit the 32-bit buffer range
  const BufRsrc rq = make_rsrc(d.packed, (uint32_t)(N * K / 4));
  const BufRsrc rp = make_rsrc(d.palette, (uint32_t)(N * gpr * 16));
  const BufRsrc rx = make_rsrc(d.x, (uint32_t)(M * K * 2));
  uint32_t oq[RB], op[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const int64_t n = row0 + 16 * r + nl;
    oq[r] = n < N ? (uint32_t)(n * (K / 4) + 64 * qg) : kBufOob;
    op[r] = n < N ? (uint32_t)((n * gpr + qg) * 16) : kBufOob;
  }

  // x staging: item i < 64*M of an iteration is (m = i/64, q, sub-step st, word w); it
  // covers x[m][k0 .. k0+16) with k0 = 256*(4*it + q) + 64*st + 16*w, and produces the two
  // fragments 2w, 2w+1 of sub-step st for fragment lane m + 16*q.
  const int n_items = 64 * M;
  const int xbuf = 4 * 8 * 4 * M;  // u32x4 per buffer
  // fragment lanes of tokens m >= M read token M-1 (a broadcast); their columns are dropped
  const int xl = qg * M + (nl < M ? nl : M - 1);
  auto stage_load = [&](int it, int i, uint4& a, uint4& b) {
    const int m = i >> 6, q = (i >> 4) & 3, st = (i >> 2) & 3, w = i & 3;
    const bool v = 4 * it + q < gpr;
    const uint32_t o = v ? (uint32_t)((m * K + 256 * (4 * it + q) + 64 * st + 16 * w) * 2) : kBufOob;
    a = buf_load16(rx, o);
    b = buf_load16(rx, o + 16u);
  };
  auto stage_store = [&](int buf, int i, uint4 a, uint4 b) {
    const int m = i >> 6, q = (i >> 4) & 3, st = (i >> 2) & 3, w = i & 3;
    u32x4 s0, s1;
    xslots(a, b, s0, s1);
    u32x4* xb = xlds + buf * xbuf;
    xb[((st * 8 + 2 * w) * 4 + q) * M + m] = s0;
    xb[((st * 8 + 2 * w + 1) * 4 + q) * M + m] = s1;
  };
  // M <= 16, so a thread handles at most 4 items per iteration
  constexpr int kMaxItems = 4;
  uint4 xa[kMaxItems], xb[kMaxItems];
  auto stage_issue = [&](int it) {
#pragma unroll
    for (int j = 0; j < kMaxItems; ++j)
      if (tid + 256 * j < n_items) stage_load(it, tid + 256 * j, xa[j], xb[j]);
  };
  auto stage_commit = [&](int buf) {
#pragma unroll
    for (int j = 0; j < kMaxItems; ++j)
      if (tid + 256 * j < n_items) stage_store(buf, tid + 256 * j, xa[j], xb[j]);
  };

  uint4 q[RB][4], p[RB];
  auto load_w = [&](int it, uint4 (&qq)[RB][4], uint4 (&pp)[RB]) {
    const bool v = 4 * it + qg < gpr;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const uint32_t o = v ? oq[r] + 256u * it : kBufOob;
#pragma unroll
      for (int j = 0; j < 4; ++j) qq[r][j] = buf_load16(rq, o + 16u * j);
      pp[r] = buf_load16(rp, v ? op[r] + 64u * it : kBufOob);
    }
  };

  f32x4 acc[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};

  stage_issue(0);
  if (has_rows) load_w(0, q, p);
  stage_commit(0);
  lds_barrier();
  for (int it = 0; it < iters; ++it) {
    const int buf = it & 1;
    const bool more = it + 1 < iters;
    uint4 qn[RB][4], pn[RB];
    if (more) {
      stage_issue(it + 1);
      if (has_rows) load_w(it + 1, qn, pn);
    }
    if (has_rows) {
      PalLut t[RB];
#pragma unroll
      for (int r = 0; r < RB; ++r)
        t[r] = make_lut(__uint_as_float(p[r].x), __uint_as_float(p[r].y),
                        __uint_as_float(p[r].z), __uint_as_float(p[r].w));
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        u32x4 xs[8];
#pragma unroll
        for (int f = 0; f < 8; ++f) xs[f] = xlds[buf * xbuf + (st * 8 + f) * 4 * M + xl];
#pragma unroll
        for (int r = 0; r < RB; ++r) {
          const uint32_t qs[4] = {q[r][st].x, q[r][st].y, q[r][st].z, q[r][st].w};
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            u32x4 a0, a1;
            dequant16_slots(qs[w], t[r], a0, a1);
            acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8, a0), __builtin_bit_cast(bf16x8, xs[2 * w]), acc[r],
                0, 0, 0);
            acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8, a1), __builtin_bit_cast(bf16x8, xs[2 * w + 1]),
                acc[r], 0, 0, 0);
          }
        }
      }
    }
    if (more) {
      stage_commit(buf ^ 1);
#pragma unroll
      for (int r = 0; r < RB; ++r) {
#pragma unroll
        for (int j = 0; j < 4; ++j) q[r][j] = qn[r][j];
        p[r] = pn[r];
      }
    }
    lds_barrier();
  }
  if (!has_rows) return;
  // acc lane l: C[n = 4*(l/16) + e][m = l%16]
  const int m = lane & 15;
  if (m < M) {
#pragma unroll
    for (int r = 0; r < RB; ++r) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t n = row0 + 16 * r + 4 * (lane >> 4) + e;
        if (n < N) d.y[(int64_t)m * N + n] = (uint16_t)f2bf(acc[r][e]);
      }
    }
  }
}

template <bool GROUPED>
static void launch_gemv(int M, dim3 grid, hipStream_t st, const plz_gemv_desc* descs, int n,
                        plz_gemv_desc single) {
  hipLaunchKernelGGL((gemv_kernel<kGemvRb, GROUPED>), grid, dim3(256),
                     2 * kXFragBytesPerToken * M, st, descs, n, single, M);
}

static int check_desc(const plz_gemv_desc& d, int i) {
  PLZ_REQUIRE(d.N >= 0 && d.K >= 0, "plz_gemv: descriptor %d has a negative shape", i);
  PLZ_REQUIRE(d.K % 256 == 0, "plz_gemv: descriptor %d: K (%lld) must be a multiple of 256", i,
              (long long)d.K);
  PLZ_REQUIRE(d.N == 0 || d.K == 0 || (d.x && d.packed && d.palette && d.y),
              "plz_gemv: descriptor %d has a null pointer", i);
  PLZ_REQUIRE(d.N * d.K / 4 < (int64_t)kBufOob && d.N * (d.K / 256) * 16 < (int64_t)kBufOob &&
                  16 * d.K * 2 < (int64_t)kBufOob,
              "plz_gemv: descriptor %d is too large (packed or palette above 2 GiB)", i);
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
  const int64_t blocks = (N + kGemvRows - 1) / kGemvRows;
  launch_gemv<false>((int)M, dim3((unsigned)blocks), (hipStream_t)stream, nullptr, 0, d);
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
    if (descs[i].K > 0) total += (descs[i].N + kGemvRows - 1) / kGemvRows;
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
  launch_gemv<true>(M, dim3((unsigned)total_blocks), (hipStream_t)stream, descs_device, n, dummy);
  return check_launch("plz_lut_gemv_grouped");
}

}  // extern "C"
