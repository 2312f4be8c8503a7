// Skinny MFMA GEMMs (128x32 tiles) for the rank-r adapter products of QwenLoRA
// (qwen_model.py:291-304): t = s x A^T, gt = s grad_y B, grad_A = gt^T x, grad_B = s grad_y^T t.
// The large training GEMMs live in plz_gemm2.hip.
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

// Skinny configuration for rank-r outputs: 128 x 32 tile, 32x32 per wave.
#define CFG_SKINNY 128, 32, 32, 32

}  // namespace plz

using namespace plz;

extern "C" {

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
