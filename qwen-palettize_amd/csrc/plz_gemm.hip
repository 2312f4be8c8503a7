// MFMA GEMM kernels of the LUT-linear path and their C entry points.
//
//   plz_lut_linear_fwd        y = x W^T (+ bias) (+ t B^T)            fused_lut_kernel.cu:309-518
//   plz_lut_linear_bwd_x      grad_x = grad_y W (+ gt A)              fused_lut_kernel.cu:551-720
//   plz_lut_linear_bwd_palette  grad_pal[n,g,c] = sum_{k in g, idx=c} (grad_y^T x)[n,k]
//                                                                     fused_lut_kernel.cu:902-1123
//   plz_soft_bwd              grad_logits / grad_palette of the Gumbel-softmax path, fused in
//                             the epilogue of the dW = grad_y^T x GEMM
//                             (fused_lut_kernel.cu:1877-1924, triton_soft_backward.py:227-325)
//   plz_linear_fwd_dense / plz_linear_bwd_x_dense   the same GEMMs on a materialised bf16 W
//   plz_lora_*                rank-r adapter products of QwenLoRA (qwen_model.py:291-304)
#include "plz_gemm.cuh"
#include "palettize_hip.h"

namespace plz {

struct NoLoad {
  static constexpr int kRegs = 1;
  __device__ static void load(const GemmArgs&, int64_t, int64_t, uint4*) {}
  __device__ static void store(uint4*, const uint4*) {}
};

template <int BI, int BJ, int WI, int WJ>
__device__ __forceinline__ void mma_stage(const uint4* __restrict__ sA, const uint4* __restrict__ sB,
                                          f32x4 (&acc)[WI / 16][WJ / 16], int wi, int wj,
                                          int lane) {
  constexpr int TI = WI / 16, TJ = WJ / 16;
#pragma unroll
  for (int kk = 0; kk < BK / 32; ++kk) {
    bf16x8 a[TI], b[TJ];
    const int ch = kk * 4 + lane / 16;
#pragma unroll
    for (int i = 0; i < TI; ++i)
      a[i] = __builtin_bit_cast(bf16x8, sA[swz(wi * WI + 16 * i + lane % 16, ch)]);
#pragma unroll
    for (int j = 0; j < TJ; ++j)
      b[j] = __builtin_bit_cast(bf16x8, sB[swz(wj * WJ + 16 * j + lane % 16, ch)]);
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
  }
}

// ---------------------------------------------------------------------------------
// Epilogues
// ---------------------------------------------------------------------------------
template <int BI, int BJ, int WI, int WJ>
struct EpiBF16 {  // C (bf16) = alpha * acc + bias[j]
  __device__ static void apply(const GemmArgs& g, f32x4 (&acc)[WI / 16][WJ / 16], int64_t i0,
                               int64_t j0, int wi, int wj, int lane, float*) {
    uint16_t* C = reinterpret_cast<uint16_t*>(g.c);
#pragma unroll
    for (int tj = 0; tj < WJ / 16; ++tj) {
      const int64_t j = j0 + wj * WJ + 16 * tj + lane % 16;
      if (j >= g.J) continue;
      const float bj = g.bias ? bf2f(g.bias[j]) : 0.f;
#pragma unroll
      for (int ti = 0; ti < WI / 16; ++ti)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t i = i0 + wi * WI + 16 * ti + 4 * (lane / 16) + e;
          if (i < g.I) C[i * g.ldc + j] = (uint16_t)f2bf(g.alpha * acc[ti][tj][e] + bj);
        }
    }
  }
};

template <int BI, int BJ, int WI, int WJ>
struct EpiF32 {  // partial[z][i][j] = alpha * acc
  __device__ static void apply(const GemmArgs& g, f32x4 (&acc)[WI / 16][WJ / 16], int64_t i0,
                               int64_t j0, int wi, int wj, int lane, float*) {
    float* P = g.partial + (int64_t)blockIdx.z * g.I * g.J;
#pragma unroll
    for (int tj = 0; tj < WJ / 16; ++tj) {
      const int64_t j = j0 + wj * WJ + 16 * tj + lane % 16;
      if (j >= g.J) continue;
#pragma unroll
      for (int ti = 0; ti < WI / 16; ++ti)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t i = i0 + wi * WI + 16 * ti + 4 * (lane / 16) + e;
          if (i < g.I) P[i * g.J + j] = g.alpha * acc[ti][tj][e];
        }
    }
  }
};

// Stage the 128x128 fp32 accumulator tile in LDS: row-major, 16-byte chunks XOR-swizzled
// by (row & 31) so that both the per-lane writes and the row reads spread over banks.
__device__ __forceinline__ int ctile(int row, int col) {
  return row * 128 + ((((col >> 2) ^ (row & 31))) << 2) + (col & 3);
}

template <int WI, int WJ>
__device__ __forceinline__ void stage_acc128(float* sC, f32x4 (&acc)[WI / 16][WJ / 16], int wi,
                                             int wj, int lane) {
#pragma unroll
  for (int ti = 0; ti < WI / 16; ++ti)
#pragma unroll
    for (int tj = 0; tj < WJ / 16; ++tj)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = wi * WI + 16 * ti + 4 * (lane / 16) + e;
        const int col = wj * WJ + 16 * tj + lane % 16;
        sC[ctile(row, col)] = acc[ti][tj][e];
      }
}

// Hard palette gradient: the tile is dW[n, k] (i = n, j = k). Each 128-wide k segment of
// a row is reduced by index class into partial[z][n][k/128][4] (deterministic order).
template <int BI, int BJ, int WI, int WJ>
struct EpiHardPal {
  static_assert(BI == 128 && BJ == 128, "palette epilogue expects a 128x128 tile");
  __device__ static void apply(const GemmArgs& g, f32x4 (&acc)[WI / 16][WJ / 16], int64_t i0,
                               int64_t j0, int wi, int wj, int lane, float* sC) {
    stage_acc128<WI, WJ>(sC, acc, wi, wj, lane);
    __syncthreads();
    const int row = threadIdx.x >> 1, h = threadIdx.x & 1;
    const int64_t n = i0 + row;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    if (n < g.I) {
      const int64_t wpr = g.Kw / kIdxPerWord;
      const uint4 q4 = *reinterpret_cast<const uint4*>(g.packed + n * wpr + (j0 + 64 * h) / 16);
      const uint32_t qs[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
          const int col = 64 * h + 16 * w + 4 * cc;
          const float4 v = *reinterpret_cast<const float4*>(&sC[ctile(row, col)]);
          const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t c = (qs[w] >> (2 * (4 * cc + e))) & 3u;
            s0 += c == 0 ? vv[e] : 0.f;
            s1 += c == 1 ? vv[e] : 0.f;
            s2 += c == 2 ? vv[e] : 0.f;
            s3 += c == 3 ? vv[e] : 0.f;
          }
        }
      }
    }
    s0 += __shfl_xor(s0, 1);
    s1 += __shfl_xor(s1, 1);
    s2 += __shfl_xor(s2, 1);
    s3 += __shfl_xor(s3, 1);
    if (h == 0 && n < g.I) {
      const int64_t segs = g.J / 128;
      float* dst = g.partial + (((int64_t)blockIdx.z * g.I + n) * segs + j0 / 128) * 4;
      *reinterpret_cast<float4*>(dst) = make_float4(s0, s1, s2, s3);
    }
  }
};

// Soft (Gumbel-softmax) gradient epilogue on the tile gW = dW[n, k]:
//   P_c        = softmax_c((logit_c + noise_c) * inv_tau)
//   W_soft     = sum_c P_c * pal_c
//   grad_logit_c = glog_scale * gW * P_c * (pal_c - W_soft)        (glog_scale = 1 is the
//                  reference formula without 1/tau, fused_lut_kernel.cu:1914-1917)
//   grad_pal_c  += gW * P_c    (reduced over the 128-wide k segment into partial[n][k/128][c])
template <int BI, int BJ, int WI, int WJ>
struct EpiSoft {
  static_assert(BI == 128 && BJ == 128, "soft epilogue expects a 128x128 tile");
  __device__ static void apply(const GemmArgs& g, f32x4 (&acc)[WI / 16][WJ / 16], int64_t i0,
                               int64_t j0, int wi, int wj, int lane, float* sC) {
    stage_acc128<WI, WJ>(sC, acc, wi, wj, lane);
    __syncthreads();
    const int wave = threadIdx.x >> 6;
    const int64_t K = g.J, gpr = g.J / kPalGroup, segs = g.J / 128;
    for (int it = 0; it < 32; ++it) {
      const int row = wave + 4 * it;
      const int64_t n = i0 + row;
      if (n >= g.I) break;
      const int col = 2 * lane;
      const int64_t k = j0 + col;
      const float2 gw = *reinterpret_cast<const float2*>(&sC[ctile(row, col)]);
      const float4 pal = *reinterpret_cast<const float4*>(g.pal + (n * gpr + k / kPalGroup) * 4);
      const float pc[4] = {pal.x, pal.y, pal.z, pal.w};
      const int64_t e0 = (n * K + k) * 4;
      const uint4 lg = *reinterpret_cast<const uint4*>(g.logits + e0);
      const float4 nz0 = *reinterpret_cast<const float4*>(g.noise + e0);
      const float4 nz1 = *reinterpret_cast<const float4*>(g.noise + e0 + 4);
      const uint32_t lw[4] = {lg.x, lg.y, lg.z, lg.w};
      const float nz[8] = {nz0.x, nz0.y, nz0.z, nz0.w, nz1.x, nz1.y, nz1.z, nz1.w};
      float sp[4] = {0.f, 0.f, 0.f, 0.f};
      uint32_t out[4];
#pragma unroll
      for (int el = 0; el < 2; ++el) {
        float a[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint32_t bits = (lw[2 * el + c / 2] >> (16 * (c & 1))) & 0xffffu;
          const float l = g.logits_f16 ? h2f(bits) : bf2f(bits);
          a[c] = (l + nz[4 * el + c]) * g.inv_tau;
        }
        const float m = fmaxf(fmaxf(a[0], a[1]), fmaxf(a[2], a[3]));
        float e[4], s = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          e[c] = __expf(a[c] - m);
          s += e[c];
        }
        const float rs = 1.f / s;
        float P[4], ws = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          P[c] = e[c] * rs;
          ws += P[c] * pc[c];
        }
        const float gv = el == 0 ? gw.x : gw.y;
        uint32_t o16[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float gp = gv * P[c];
          sp[c] += gp;
          const float gl = g.glog_scale * gp * (pc[c] - ws);
          o16[c] = g.logits_f16 ? f2h(gl) : f2bf(gl);
        }
        out[2 * el] = o16[0] | (o16[1] << 16);
        out[2 * el + 1] = o16[2] | (o16[3] << 16);
      }
      *reinterpret_cast<uint4*>(g.grad_logits + e0) = make_uint4(out[0], out[1], out[2], out[3]);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) sp[c] += __shfl_xor(sp[c], off);
      }
      if (lane == 0) {
        float* dst = g.partial + (n * segs + j0 / 128) * 4;
        *reinterpret_cast<float4*>(dst) = make_float4(sp[0], sp[1], sp[2], sp[3]);
      }
    }
  }
};

// ---------------------------------------------------------------------------------
// The kernel
// ---------------------------------------------------------------------------------
template <int BI, int BJ, int WI, int WJ, class LA, class LB, class LA2, class LB2,
          template <int, int, int, int> class EPI>
__global__ __launch_bounds__(256) void gemm_kernel(const GemmArgs g) {
  extern __shared__ uint4 smem[];
  constexpr int TI = WI / 16, TJ = WJ / 16;
  uint4* sA0 = smem;
  uint4* sB0 = smem + BI * CH;
  uint4* sA1 = smem + (BI + BJ) * CH;
  uint4* sB1 = sA1 + BI * CH;

  // Tile order: consecutive workgroups land on different XCDs (round-robin dispatch), so
  // first give each XCD a contiguous slice of the tile space, then walk it in groups of
  // 8 tile-rows so that neighbouring workgroups share A (and B) panels in that XCD's L2.
  int bid = blockIdx.x;
  const int T = g.tiles_i * g.tiles_j;
  if (T % 8 == 0) bid = (bid % 8) * (T / 8) + bid / 8;
  const int GROUP = 8;
  const int per_group = GROUP * g.tiles_j;
  const int first_i = (bid / per_group) * GROUP;
  const int gsz = min(g.tiles_i - first_i, GROUP);
  const int tile_i = first_i + (bid % per_group) % gsz;
  const int tile_j = (bid % per_group) / gsz;
  const int64_t i0 = (int64_t)tile_i * BI, j0 = (int64_t)tile_j * BJ;

  const int64_t rbeg = (int64_t)blockIdx.z * g.r_split;
  const int64_t rend = min(g.R, rbeg + g.r_split);
  const int nk = rend > rbeg ? (int)((rend - rbeg + BK - 1) / BK) : 0;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wi = wave / (BJ / WJ), wj = wave % (BJ / WJ);

  f32x4 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  uint4 ra[LA::kRegs], rb[LB::kRegs];
  if (nk > 0) {
    LA::load(g, i0, rbeg, ra);
    LB::load(g, j0, rbeg, rb);
    LA::store(sA0, ra);
    LB::store(sB0, rb);
  }
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const bool odd = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      LA::load(g, i0, rbeg + (int64_t)(kt + 1) * BK, ra);
      LB::load(g, j0, rbeg + (int64_t)(kt + 1) * BK, rb);
    }
    mma_stage<BI, BJ, WI, WJ>(odd ? sA1 : sA0, odd ? sB1 : sB0, acc, wi, wj, lane);
    if (more) {
      LA::store(odd ? sA0 : sA1, ra);
      LB::store(odd ? sB0 : sB1, rb);
    }
    __syncthreads();
  }
  if constexpr (!__is_same(LA2, NoLoad)) {
    if (g.R2 > 0 && blockIdx.z == 0) {
      uint4 ra2[LA2::kRegs], rb2[LB2::kRegs];
      LA2::load(g, i0, 0, ra2);
      LB2::load(g, j0, 0, rb2);
      LA2::store(sA0, ra2);
      LB2::store(sB0, rb2);
      __syncthreads();
      mma_stage<BI, BJ, WI, WJ>(sA0, sB0, acc, wi, wj, lane);
      __syncthreads();
    }
  }
  EPI<BI, BJ, WI, WJ>::apply(g, acc, i0, j0, wi, wj, lane, reinterpret_cast<float*>(smem));
}

template <int BI, int BJ, int WI, int WJ, class LA, class LB, class LA2, class LB2,
          template <int, int, int, int> class EPI>
static int launch_gemm(GemmArgs g, int splits, hipStream_t stream, const char* what) {
  g.tiles_i = (int)((g.I + BI - 1) / BI);
  g.tiles_j = (int)((g.J + BJ - 1) / BJ);
  if (g.r_split <= 0) g.r_split = g.R;
  size_t lds = (size_t)2 * (BI + BJ) * CH * 16;
  if (__is_same(EPI<BI, BJ, WI, WJ>, EpiHardPal<BI, BJ, WI, WJ>) ||
      __is_same(EPI<BI, BJ, WI, WJ>, EpiSoft<BI, BJ, WI, WJ>))
    lds = lds > 128 * 128 * 4 ? lds : 128 * 128 * 4;
  auto kern = gemm_kernel<BI, BJ, WI, WJ, LA, LB, LA2, LB2, EPI>;
  static bool attr_done = false;
  if (!attr_done) {
    hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    attr_done = true;
  }
  const int64_t tiles = (int64_t)g.tiles_i * g.tiles_j;
  if (tiles == 0 || splits == 0) return PLZ_OK;
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles, 1, (unsigned)splits), dim3(256), lds, stream, g);
  return check_launch(what);
}

// ---------------------------------------------------------------------------------
// Reductions of split partial sums
// ---------------------------------------------------------------------------------
// out[n][g][c] = sum_z sum_{s<2} partial[z][n][2g+s][c]   (128-wide segments -> 256 groups)
__global__ void reduce_pal_kernel(const float* __restrict__ partial, float* __restrict__ out,
                                  int64_t N, int64_t G, int Z) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N * G) return;
  const int64_t n = t / G, gg = t % G;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int z = 0; z < Z; ++z) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float4 v = *reinterpret_cast<const float4*>(partial + (((int64_t)z * N + n) * 2 * G + 2 * gg + h) * 4);
      s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
    }
  }
  *reinterpret_cast<float4*>(out + t * 4) = s;
}

// out = sum_z partial[z][i][j], written as bf16 or fp32, optionally transposed (out[j][i]).
__global__ void reduce_f32_kernel(const float* __restrict__ partial, void* __restrict__ out,
                                  int64_t I, int64_t J, int Z, int out_bf16, int transpose) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= I * J) return;
  float s = 0.f;
  for (int z = 0; z < Z; ++z) s += partial[(int64_t)z * I * J + t];
  const int64_t i = t / J, j = t % J;
  const int64_t o = transpose ? j * I + i : t;
  if (out_bf16)
    reinterpret_cast<uint16_t*>(out)[o] = (uint16_t)f2bf(s);
  else
    reinterpret_cast<float*>(out)[o] = s;
}

// Number of reduction splits for a tile grid of `tiles` workgroups over reduction R:
// enough workgroups to cover the 256 CUs about twice, each split at least 16 stages deep.
static int pick_splits(int64_t tiles, int64_t R) {
  int64_t z = (512 + tiles - 1) / tiles;
  int64_t zmax = R / (16 * BK);
  if (z > zmax) z = zmax;
  if (z < 1) z = 1;
  if (z > 64) z = 64;
  return (int)z;
}
static int64_t split_len(int64_t R, int z) {
  int64_t per = (R + z - 1) / z;
  return (per + BK - 1) / BK * BK;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Main tile configuration: 128x128 workgroup tile, 64x64 per wave.
#define CFG_MAIN 128, 128, 64, 64
// Skinny configuration for rank-r outputs: 128 x 32 tile, 32x32 per wave.
#define CFG_SKINNY 128, 32, 32, 32

}  // namespace plz

using namespace plz;

extern "C" {

int plz_lut_linear_fwd(const uint16_t* x, const int32_t* packed, const float* palette,
                       const uint16_t* bias, const uint16_t* lora_t, const uint16_t* lora_b,
                       int rank, uint16_t* y, int64_t M, int64_t N, int64_t K, void* stream) {
  PLZ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "plz_lut_linear_fwd: negative shape");
  PLZ_REQUIRE(K % 256 == 0, "plz_lut_linear_fwd: K (%lld) must be a multiple of 256", (long long)K);
  PLZ_REQUIRE(N % 8 == 0, "plz_lut_linear_fwd: N (%lld) must be a multiple of 8", (long long)N);
  PLZ_REQUIRE(rank >= 0 && rank <= BK && rank % 8 == 0,
              "plz_lut_linear_fwd: rank (%d) must be a multiple of 8 in [0, 64]", rank);
  if (M == 0 || N == 0) return PLZ_OK;
  PLZ_REQUIRE(x && packed && palette && y, "plz_lut_linear_fwd: null pointer");
  PLZ_REQUIRE(aligned16(x) && aligned16(palette) && aligned16(packed),
              "plz_lut_linear_fwd: x, packed and palette must be 16-byte aligned");
  PLZ_REQUIRE(rank == 0 || (lora_t && lora_b && aligned16(lora_t) && aligned16(lora_b)),
              "plz_lut_linear_fwd: rank > 0 needs 16-byte aligned lora_t and lora_b");
  GemmArgs g = {};
  g.a = x; g.lda = K;
  g.packed = packed; g.pal = palette; g.Nw = N; g.Kw = K;
  g.I = M; g.J = N; g.R = K;
  g.a2 = lora_t; g.lda2 = rank; g.b2 = lora_b; g.ldb2 = rank; g.R2 = rank;
  g.c = y; g.ldc = N; g.bias = bias; g.alpha = 1.f;
  return launch_gemm<CFG_MAIN, LoadRC<128, 0>, LoadLutRC<128>, LoadRC<128, 2>, LoadRC<128, 3>,
                     EpiBF16>(g, 1, (hipStream_t)stream, "plz_lut_linear_fwd");
}

int plz_lut_linear_bwd_x(const uint16_t* grad_y, const int32_t* packed, const float* palette,
                         const uint16_t* lora_gt, const uint16_t* lora_a, int rank,
                         uint16_t* grad_x, int64_t M, int64_t N, int64_t K, void* stream) {
  PLZ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "plz_lut_linear_bwd_x: negative shape");
  PLZ_REQUIRE(K % 256 == 0, "plz_lut_linear_bwd_x: K (%lld) must be a multiple of 256",
              (long long)K);
  PLZ_REQUIRE(N % 8 == 0, "plz_lut_linear_bwd_x: N (%lld) must be a multiple of 8", (long long)N);
  PLZ_REQUIRE(rank >= 0 && rank <= BK && rank % 8 == 0,
              "plz_lut_linear_bwd_x: rank (%d) must be a multiple of 8 in [0, 64]", rank);
  if (M == 0 || K == 0) return PLZ_OK;
  PLZ_REQUIRE(grad_y && packed && palette && grad_x, "plz_lut_linear_bwd_x: null pointer");
  PLZ_REQUIRE(aligned16(grad_y) && aligned16(palette),
              "plz_lut_linear_bwd_x: grad_y and palette must be 16-byte aligned");
  PLZ_REQUIRE(rank == 0 || (lora_gt && lora_a && aligned16(lora_gt) && aligned16(lora_a)),
              "plz_lut_linear_bwd_x: rank > 0 needs 16-byte aligned lora_gt and lora_a");
  GemmArgs g = {};
  g.a = grad_y; g.lda = N;
  g.packed = packed; g.pal = palette; g.Nw = N; g.Kw = K;
  g.I = M; g.J = K; g.R = N;
  g.a2 = lora_gt; g.lda2 = rank; g.b2 = lora_a; g.ldb2 = K; g.R2 = rank;
  g.c = grad_x; g.ldc = K; g.alpha = 1.f;
  return launch_gemm<CFG_MAIN, LoadRC<128, 0>, LoadLutNN<128>, LoadRC<128, 2>, LoadMNC<128, 3>,
                     EpiBF16>(g, 1, (hipStream_t)stream, "plz_lut_linear_bwd_x");
}

static int palette_splits(int64_t M, int64_t N, int64_t K) {
  return pick_splits(((N + 127) / 128) * (K / 128), M);
}

size_t plz_lut_linear_bwd_palette_workspace(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const int z = palette_splits(M, N, K);
  return (size_t)z * N * (K / 128) * 4 * sizeof(float);
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
    hipMemsetAsync(grad_palette, 0, (size_t)N * (K / 256) * 16, (hipStream_t)stream);
    return check_launch("plz_lut_linear_bwd_palette");
  }
  PLZ_REQUIRE(x && grad_y && aligned16(x) && aligned16(grad_y) && aligned16(packed),
              "plz_lut_linear_bwd_palette: x, grad_y and packed must be non-null, 16-byte aligned");
  const size_t need = plz_lut_linear_bwd_palette_workspace(M, N, K);
  if (!workspace || workspace_bytes < need) {
    set_error("plz_lut_linear_bwd_palette: workspace of %zu bytes needed, %zu given", need,
              workspace_bytes);
    return PLZ_EWORKSPACE;
  }
  const int z = palette_splits(M, N, K);
  GemmArgs g = {};
  g.a = grad_y; g.lda = N;   // A(i=n, r=m) = grad_y[m, n]
  g.b = x; g.ldb = K;        // B(j=k, r=m) = x[m, k]
  g.packed = packed; g.Nw = N; g.Kw = K;
  g.I = N; g.J = K; g.R = M; g.r_split = split_len(M, z);
  g.partial = reinterpret_cast<float*>(workspace);
  int rc = launch_gemm<CFG_MAIN, LoadMNC<128, 0>, LoadMNC<128, 1>, NoLoad, NoLoad, EpiHardPal>(
      g, z, (hipStream_t)stream, "plz_lut_linear_bwd_palette");
  if (rc != PLZ_OK) return rc;
  const int64_t G = K / 256, n_out = N * G;
  hipLaunchKernelGGL(reduce_pal_kernel, dim3((unsigned)((n_out + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, g.partial, grad_palette, N, G, z);
  return check_launch("plz_lut_linear_bwd_palette/reduce");
}

int plz_linear_fwd_dense(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                         const uint16_t* lora_t, const uint16_t* lora_b, int rank, uint16_t* y,
                         int64_t M, int64_t N, int64_t K, void* stream) {
  PLZ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "plz_linear_fwd_dense: negative shape");
  PLZ_REQUIRE(K % 8 == 0 && N % 8 == 0, "plz_linear_fwd_dense: K and N must be multiples of 8");
  PLZ_REQUIRE(rank >= 0 && rank <= BK && rank % 8 == 0,
              "plz_linear_fwd_dense: rank (%d) must be a multiple of 8 in [0, 64]", rank);
  if (M == 0 || N == 0) return PLZ_OK;
  PLZ_REQUIRE(x && w && y && aligned16(x) && aligned16(w),
              "plz_linear_fwd_dense: x, w, y must be non-null; x, w 16-byte aligned");
  PLZ_REQUIRE(rank == 0 || (lora_t && lora_b && aligned16(lora_t) && aligned16(lora_b)),
              "plz_linear_fwd_dense: rank > 0 needs 16-byte aligned lora_t and lora_b");
  GemmArgs g = {};
  g.a = x; g.lda = K; g.b = w; g.ldb = K;
  g.I = M; g.J = N; g.R = K;
  g.a2 = lora_t; g.lda2 = rank; g.b2 = lora_b; g.ldb2 = rank; g.R2 = rank;
  g.c = y; g.ldc = N; g.bias = bias; g.alpha = 1.f;
  return launch_gemm<CFG_MAIN, LoadRC<128, 0>, LoadRC<128, 1>, LoadRC<128, 2>, LoadRC<128, 3>,
                     EpiBF16>(g, 1, (hipStream_t)stream, "plz_linear_fwd_dense");
}

int plz_linear_bwd_x_dense(const uint16_t* grad_y, const uint16_t* w, const uint16_t* lora_gt,
                           const uint16_t* lora_a, int rank, uint16_t* grad_x, int64_t M,
                           int64_t N, int64_t K, void* stream) {
  PLZ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "plz_linear_bwd_x_dense: negative shape");
  PLZ_REQUIRE(K % 8 == 0 && N % 8 == 0, "plz_linear_bwd_x_dense: K and N must be multiples of 8");
  PLZ_REQUIRE(rank >= 0 && rank <= BK && rank % 8 == 0,
              "plz_linear_bwd_x_dense: rank (%d) must be a multiple of 8 in [0, 64]", rank);
  if (M == 0 || K == 0) return PLZ_OK;
  PLZ_REQUIRE(grad_y && w && grad_x && aligned16(grad_y) && aligned16(w),
              "plz_linear_bwd_x_dense: grad_y, w, grad_x must be non-null; grad_y, w aligned");
  PLZ_REQUIRE(rank == 0 || (lora_gt && lora_a && aligned16(lora_gt) && aligned16(lora_a)),
              "plz_linear_bwd_x_dense: rank > 0 needs 16-byte aligned lora_gt and lora_a");
  GemmArgs g = {};
  g.a = grad_y; g.lda = N;
  g.b = w; g.ldb = K;  // B(j=k, r=n) = w[n, k]
  g.I = M; g.J = K; g.R = N;
  g.a2 = lora_gt; g.lda2 = rank; g.b2 = lora_a; g.ldb2 = K; g.R2 = rank;
  g.c = grad_x; g.ldc = K; g.alpha = 1.f;
  return launch_gemm<CFG_MAIN, LoadRC<128, 0>, LoadMNC<128, 1>, LoadRC<128, 2>, LoadMNC<128, 3>,
                     EpiBF16>(g, 1, (hipStream_t)stream, "plz_linear_bwd_x_dense");
}

size_t plz_soft_bwd_workspace(int64_t M, int64_t N, int64_t K) {
  (void)M;
  if (N <= 0 || K <= 0) return 0;
  return (size_t)N * (K / 128) * 4 * sizeof(float);
}

int plz_soft_bwd(const uint16_t* x, const uint16_t* grad_y, const uint16_t* logits,
                 int logits_dtype, const float* noise, const float* palette, float tau,
                 int scale_grad_by_inv_tau, uint16_t* grad_logits, float* grad_palette,
                 void* workspace, size_t workspace_bytes, int64_t M, int64_t N, int64_t K,
                 void* stream) {
  PLZ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "plz_soft_bwd: negative shape");
  PLZ_REQUIRE(K % 256 == 0, "plz_soft_bwd: K (%lld) must be a multiple of 256", (long long)K);
  PLZ_REQUIRE(N % 8 == 0, "plz_soft_bwd: N (%lld) must be a multiple of 8", (long long)N);
  PLZ_REQUIRE(logits_dtype == PLZ_DT_BF16 || logits_dtype == PLZ_DT_FP16,
              "plz_soft_bwd: logits dtype must be bf16 or fp16");
  PLZ_REQUIRE(tau > 0.f, "plz_soft_bwd: tau must be positive");
  if (N == 0 || K == 0) return PLZ_OK;
  PLZ_REQUIRE(x && grad_y && logits && noise && palette && grad_logits && grad_palette,
              "plz_soft_bwd: null pointer");
  PLZ_REQUIRE(aligned16(x) && aligned16(grad_y) && aligned16(logits) && aligned16(noise) &&
                  aligned16(palette) && aligned16(grad_logits),
              "plz_soft_bwd: operands must be 16-byte aligned");
  const size_t need = plz_soft_bwd_workspace(M, N, K);
  if (!workspace || workspace_bytes < need) {
    set_error("plz_soft_bwd: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
    return PLZ_EWORKSPACE;
  }
  GemmArgs g = {};
  g.a = grad_y; g.lda = N;
  g.b = x; g.ldb = K;
  g.pal = palette; g.Nw = N; g.Kw = K;
  g.I = N; g.J = K; g.R = M; g.r_split = M > 0 ? M : 1;
  g.partial = reinterpret_cast<float*>(workspace);
  g.logits = logits; g.noise = noise; g.inv_tau = 1.f / tau;
  g.glog_scale = scale_grad_by_inv_tau ? 1.f / tau : 1.f;
  g.grad_logits = grad_logits; g.logits_f16 = logits_dtype == PLZ_DT_FP16;
  int rc = launch_gemm<CFG_MAIN, LoadMNC<128, 0>, LoadMNC<128, 1>, NoLoad, NoLoad, EpiSoft>(
      g, 1, (hipStream_t)stream, "plz_soft_bwd");
  if (rc != PLZ_OK) return rc;
  const int64_t G = K / 256, n_out = N * G;
  hipLaunchKernelGGL(reduce_pal_kernel, dim3((unsigned)((n_out + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, g.partial, grad_palette, N, G, 1);
  return check_launch("plz_soft_bwd/reduce");
}

int plz_lora_project(const uint16_t* x, const uint16_t* lora_a, float scale, uint16_t* t,
                     int64_t M, int64_t K, int rank, void* stream) {
  PLZ_REQUIRE(M >= 0 && K >= 0 && rank > 0 && rank <= 32 && rank % 8 == 0,
              "plz_lora_project: need M, K >= 0 and rank a multiple of 8 in [8, 32]");
  PLZ_REQUIRE(K % 8 == 0, "plz_lora_project: K must be a multiple of 8");
  if (M == 0) return PLZ_OK;
  PLZ_REQUIRE(x && lora_a && t && aligned16(x) && aligned16(lora_a),
              "plz_lora_project: null or misaligned pointer");
  GemmArgs g = {};
  g.a = x; g.lda = K; g.b = lora_a; g.ldb = K;
  g.I = M; g.J = rank; g.R = K;
  g.c = t; g.ldc = rank; g.alpha = scale;
  return launch_gemm<CFG_SKINNY, LoadRC<128, 0>, LoadRC<32, 1>, NoLoad, NoLoad, EpiBF16>(
      g, 1, (hipStream_t)stream, "plz_lora_project");
}

int plz_lora_grad_t(const uint16_t* grad_y, const uint16_t* lora_b, float scale, uint16_t* gt,
                    int64_t M, int64_t N, int rank, void* stream) {
  PLZ_REQUIRE(M >= 0 && N >= 0 && rank > 0 && rank <= 32 && rank % 8 == 0,
              "plz_lora_grad_t: need M, N >= 0 and rank a multiple of 8 in [8, 32]");
  PLZ_REQUIRE(N % 8 == 0, "plz_lora_grad_t: N must be a multiple of 8");
  if (M == 0) return PLZ_OK;
  PLZ_REQUIRE(grad_y && lora_b && gt && aligned16(grad_y) && aligned16(lora_b),
              "plz_lora_grad_t: null or misaligned pointer");
  GemmArgs g = {};
  g.a = grad_y; g.lda = N;
  g.b = lora_b; g.ldb = rank;  // B(j, r=n) = lora_b[n, j]
  g.I = M; g.J = rank; g.R = N;
  g.c = gt; g.ldc = rank; g.alpha = scale;
  return launch_gemm<CFG_SKINNY, LoadRC<128, 0>, LoadMNC<32, 1>, NoLoad, NoLoad, EpiBF16>(
      g, 1, (hipStream_t)stream, "plz_lora_grad_t");
}

static int lora_splits(int64_t rows, int64_t M) { return pick_splits((rows + 127) / 128, M); }

size_t plz_lora_weight_grads_workspace(int64_t M, int64_t N, int64_t K, int rank) {
  if (M <= 0 || rank <= 0) return 0;
  size_t zb = (size_t)lora_splits(N, M) * N * rank;
  size_t za = (size_t)lora_splits(K, M) * K * rank;
  return (zb > za ? zb : za) * sizeof(float);
}

int plz_lora_weight_grads(const uint16_t* x, const uint16_t* grad_y, const uint16_t* t,
                          const uint16_t* gt, float scale, void* grad_a, void* grad_b,
                          int out_dtype, void* workspace, size_t workspace_bytes, int64_t M,
                          int64_t N, int64_t K, int rank, void* stream) {
  PLZ_REQUIRE(M >= 0 && N >= 0 && K >= 0 && rank > 0 && rank <= 32 && rank % 8 == 0,
              "plz_lora_weight_grads: bad shape");
  PLZ_REQUIRE(N % 8 == 0 && K % 8 == 0, "plz_lora_weight_grads: N and K must be multiples of 8");
  PLZ_REQUIRE(out_dtype == PLZ_DT_BF16 || out_dtype == PLZ_DT_FP32,
              "plz_lora_weight_grads: out dtype must be bf16 or fp32");
  PLZ_REQUIRE(x && grad_y && t && gt && grad_a && grad_b, "plz_lora_weight_grads: null pointer");
  PLZ_REQUIRE(aligned16(x) && aligned16(grad_y) && aligned16(t) && aligned16(gt),
              "plz_lora_weight_grads: inputs must be 16-byte aligned");
  const size_t need = plz_lora_weight_grads_workspace(M, N, K, rank);
  if (M > 0 && (!workspace || workspace_bytes < need)) {
    set_error("plz_lora_weight_grads: workspace of %zu bytes needed, %zu given", need,
              workspace_bytes);
    return PLZ_EWORKSPACE;
  }
  hipStream_t s = (hipStream_t)stream;
  const int bf = out_dtype == PLZ_DT_BF16;
  if (M == 0) {
    hipMemsetAsync(grad_b, 0, (size_t)N * rank * (bf ? 2 : 4), s);
    hipMemsetAsync(grad_a, 0, (size_t)K * rank * (bf ? 2 : 4), s);
    return check_launch("plz_lora_weight_grads");
  }
  float* ws = reinterpret_cast<float*>(workspace);
  // grad_B[n, j] = scale * sum_m grad_y[m, n] t[m, j]
  {
    const int z = lora_splits(N, M);
    GemmArgs g = {};
    g.a = grad_y; g.lda = N; g.b = t; g.ldb = rank;
    g.I = N; g.J = rank; g.R = M; g.r_split = split_len(M, z);
    g.partial = ws; g.alpha = scale;
    int rc = launch_gemm<CFG_SKINNY, LoadMNC<128, 0>, LoadMNC<32, 1>, NoLoad, NoLoad, EpiF32>(
        g, z, s, "plz_lora_weight_grads/B");
    if (rc) return rc;
    hipLaunchKernelGGL(reduce_f32_kernel, dim3((unsigned)((N * rank + 255) / 256)), dim3(256), 0,
                       s, ws, grad_b, N, (int64_t)rank, z, bf, 0);
    if ((rc = check_launch("plz_lora_weight_grads/B reduce"))) return rc;
  }
  // grad_A[j, k] = sum_m gt[m, j] x[m, k]  (computed as its transpose [k, j])
  {
    const int z = lora_splits(K, M);
    GemmArgs g = {};
    g.a = x; g.lda = K; g.b = gt; g.ldb = rank;
    g.I = K; g.J = rank; g.R = M; g.r_split = split_len(M, z);
    g.partial = ws; g.alpha = 1.f;
    int rc = launch_gemm<CFG_SKINNY, LoadMNC<128, 0>, LoadMNC<32, 1>, NoLoad, NoLoad, EpiF32>(
        g, z, s, "plz_lora_weight_grads/A");
    if (rc) return rc;
    hipLaunchKernelGGL(reduce_f32_kernel, dim3((unsigned)((K * rank + 255) / 256)), dim3(256), 0,
                       s, ws, grad_a, K, (int64_t)rank, z, bf, 1);
    return check_launch("plz_lora_weight_grads/A reduce");
  }
}

}  // extern "C"
