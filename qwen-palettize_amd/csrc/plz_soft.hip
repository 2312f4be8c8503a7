// Soft (Gumbel-softmax) forward: noise generation and the build-W kernel.
//
//   P_c = softmax_c((logit_c + noise_c) / tau)           fused_lut_kernel.cu:1974-1983
//   W_soft = sum_c P_c pal_c                              fused_lut_kernel.cu:1995
//   W_hard = pal[argmax_c P_c]   (first max wins)         fused_lut_kernel.cu:1998-2003
//   W_hard = pal[argmax_c logit_c] (first max wins)       triton_soft_forward.py:160-176
// The forward weight W = W_hard is the straight-through estimator's value
// (fused_lut_linear_cuda.py:906-910); W_soft is what the backward differentiates.
#include "plz_common.h"
#include "palettize_hip.h"

namespace plz {

__global__ void philox_gumbel_kernel(float* __restrict__ out, int64_t n4, uint64_t seed,
                                     uint64_t offset) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n4) return;
  const uint64_t ctr = offset + (uint64_t)t;
  const U4 r = philox4x32_10(U4{(uint32_t)ctr, (uint32_t)(ctr >> 32), 0u, 0u}, (uint32_t)seed,
                             (uint32_t)(seed >> 32));
  *reinterpret_cast<float4*>(out + 4 * t) =
      make_float4(gumbel_from_bits(r.x), gumbel_from_bits(r.y), gumbel_from_bits(r.z),
                  gumbel_from_bits(r.w));
}

// The reference's LCG hash samplers. ARITH = false: the CUDA one (fused_lut_kernel.cu:1245-1256),
// uint32 throughout. ARITH = true: the Triton one (triton_soft_forward.py:51-66), the same
// statements in int32, where >> is an arithmetic shift; multiplies and adds wrap to the same
// bits either way, so only the two shifts differ (when the shifted value has bit 31 set).
template <bool ARITH>
__device__ __forceinline__ uint32_t lcg_shr(uint32_t x, int s) {
  return ARITH ? (uint32_t)((int32_t)x >> s) : x >> s;
}
template <bool ARITH>
__device__ __forceinline__ float lcg_gumbel(uint32_t seed, uint32_t idx) {
  uint32_t x = seed ^ (idx * 0x9E3779B9u);
  x ^= lcg_shr<ARITH>(x, 13);
  x = x * 1103515245u + 12345u;
  x ^= lcg_shr<ARITH>(x, 17);
  x = x * 1103515245u + 12345u;
  float u = (float)(x & 0xFFFFFFu) * (1.0f / 16777216.0f);
  u = fmaxf(u, 1e-7f);
  return -logf(-logf(u));
}

// Element (n, k, c) drawn with idx = (k*N + n)*4 + c in uint32 arithmetic, stored at [n, k, c].
template <bool ARITH>
__global__ void lcg_gumbel_kernel(float* __restrict__ out, uint32_t seed, int64_t N, int64_t K) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // element (n, k)
  if (t >= N * K) return;
  const int64_t n = t / K, k = t % K;
  const uint32_t base = ((uint32_t)k * (uint32_t)N + (uint32_t)n) * 4u;
  *reinterpret_cast<float4*>(out + 4 * t) =
      make_float4(lcg_gumbel<ARITH>(seed, base), lcg_gumbel<ARITH>(seed, base + 1),
                  lcg_gumbel<ARITH>(seed, base + 2), lcg_gumbel<ARITH>(seed, base + 3));
}

// ---- reference-layout batched P / W --------------------------------------------------
// fused_compute_P_W_batched (fused_lut_kernel.cu:2097-2158) in the reference's own layouts:
// logits (4, K, N) fp16 planes, palette (G, 4) bf16 with row o in group o / group_size,
// P_aos (K, N, 4) fp16 and W (K, N) bf16 = sum_c P_c pal_c (the soft weight; this build does
// not take an argmax). Element e = j*N + o draws class c at idx e*4 + c from the CUDA hash
// keyed by step_seed ^ (seed_offset * 0x9E3779B9) (fused_lut_kernel.cu:2129). Each thread
// takes 4 consecutive elements of the flat (K, N) index: with vec, as one 8-byte load per
// logit plane, two 16-byte P stores and one 8-byte W store.
constexpr int kPwBlock = 256;
__global__ void pw_ref_batched_kernel(const plz_pw_ref_desc* __restrict__ descs, int n_desc,
                                      int64_t group_size, float inv_tau, uint32_t step_seed) {
  const int64_t b = blockIdx.x;
  int lo = 0, hi = n_desc - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (descs[mid].block_begin <= b) lo = mid; else hi = mid - 1;
  }
  const plz_pw_ref_desc d = descs[lo];
  const int64_t KN = d.K * d.N;
  const int64_t e0 = ((b - d.block_begin) * kPwBlock + threadIdx.x) * 4;
  if (e0 >= KN) return;
  const int cnt = KN - e0 < 4 ? (int)(KN - e0) : 4;
  const uint32_t seed = step_seed ^ (d.seed_offset * 0x9E3779B9u);
  float l[4][4];  // [element][class]
  if (d.vec) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint2 v = *reinterpret_cast<const uint2*>(d.logits + c * KN + e0);
      l[0][c] = h2f(v.x & 0xffffu); l[1][c] = h2f(v.x >> 16);
      l[2][c] = h2f(v.y & 0xffffu); l[3][c] = h2f(v.y >> 16);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int c = 0; c < 4; ++c) l[i][c] = i < cnt ? h2f(d.logits[c * KN + e0 + i]) : 0.f;
  }
  int64_t o = e0 % d.N;
  uint32_t pbits[4][2], wbits[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t idx = (uint32_t)(e0 + i) * 4u;
    float a[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) a[c] = (l[i][c] + lcg_gumbel<false>(seed, idx + c)) * inv_tau;
    const float m = fmaxf(fmaxf(a[0], a[1]), fmaxf(a[2], a[3]));
    float ex[4], s = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      ex[c] = expf(a[c] - m);
      s += ex[c];
    }
    const uint2 pv = *reinterpret_cast<const uint2*>(d.palette + (o / group_size) * 4);
    const float pal[4] = {bf2f(pv.x & 0xffffu), bf2f(pv.x >> 16), bf2f(pv.y & 0xffffu),
                          bf2f(pv.y >> 16)};
    float P[4], w = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      P[c] = ex[c] / s;
      w += P[c] * pal[c];
    }
    pbits[i][0] = f2h(P[0]) | (f2h(P[1]) << 16);
    pbits[i][1] = f2h(P[2]) | (f2h(P[3]) << 16);
    wbits[i] = f2bf(w);
    if (++o == d.N) o = 0;
  }
  if (d.vec) {
    uint4* pp = reinterpret_cast<uint4*>(d.p_aos + e0 * 4);
    pp[0] = make_uint4(pbits[0][0], pbits[0][1], pbits[1][0], pbits[1][1]);
    pp[1] = make_uint4(pbits[2][0], pbits[2][1], pbits[3][0], pbits[3][1]);
    *reinterpret_cast<uint2*>(d.w + e0) =
        make_uint2(wbits[0] | (wbits[1] << 16), wbits[2] | (wbits[3] << 16));
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (i < cnt) {
        uint32_t* pp = reinterpret_cast<uint32_t*>(d.p_aos + (e0 + i) * 4);
        pp[0] = pbits[i][0];
        pp[1] = pbits[i][1];
        d.w[e0 + i] = (uint16_t)wbits[i];
      }
  }
}

// ---- build W -------------------------------------------------------------------------
// One thread per 2 consecutive k of one row: 16 B of logits, 32 B of noise in; 4 B out.
// GEN: the noise is drawn here (Philox at counter offset + n*K + k, the values
// plz_gumbel_philox would have stored) instead of read.
template <bool GEN>
__device__ __forceinline__ void build_w_pair(const uint16_t* __restrict__ logits, int f16,
                                             const float* __restrict__ noise, uint64_t seed,
                                             uint64_t offset, const float* __restrict__ pal,
                                             float inv_tau, int mode, uint16_t* __restrict__ w,
                                             uint16_t* __restrict__ w_soft, int64_t K, int64_t t,
                                             uint16_t* __restrict__ p_out = nullptr) {
  const int64_t half = K / 2;
  const int64_t n = t / half, k = 2 * (t % half);
  const float4 p = *reinterpret_cast<const float4*>(pal + (n * (K / kPalGroup) + k / kPalGroup) * 4);
  const float pc[4] = {p.x, p.y, p.z, p.w};
  const int64_t e0 = (n * K + k) * 4;
  const uint4 lg = *reinterpret_cast<const uint4*>(logits + e0);
  const uint32_t lw[4] = {lg.x, lg.y, lg.z, lg.w};
  float nz[8];
  if constexpr (GEN) {
    float z[4];
    philox_gumbel4(seed, offset + (uint64_t)(n * K + k), z);
    nz[0] = z[0]; nz[1] = z[1]; nz[2] = z[2]; nz[3] = z[3];
    philox_gumbel4(seed, offset + (uint64_t)(n * K + k + 1), z);
    nz[4] = z[0]; nz[5] = z[1]; nz[6] = z[2]; nz[7] = z[3];
  } else {
    const float4 z0 = *reinterpret_cast<const float4*>(noise + e0);
    const float4 z1 = *reinterpret_cast<const float4*>(noise + e0 + 4);
    nz[0] = z0.x; nz[1] = z0.y; nz[2] = z0.z; nz[3] = z0.w;
    nz[4] = z1.x; nz[5] = z1.y; nz[6] = z1.z; nz[7] = z1.w;
  }
  uint32_t wo[2], so[2], po[4];
  build_w_two(lw, f16, nz, pc, inv_tau, mode, wo, so, po);
  if (p_out) *reinterpret_cast<uint4*>(p_out + e0) = make_uint4(po[0], po[1], po[2], po[3]);
  const int64_t o = n * K + k;
  *reinterpret_cast<uint32_t*>(w + o) = wo[0] | (wo[1] << 16);
  if (w_soft) *reinterpret_cast<uint32_t*>(w_soft + o) = so[0] | (so[1] << 16);
}

template <bool GEN>
__global__ void build_w_kernel(const uint16_t* __restrict__ logits, int f16,
                               const float* __restrict__ noise, uint64_t seed, uint64_t offset,
                               const float* __restrict__ pal, float inv_tau, int mode,
                               uint16_t* __restrict__ w, uint16_t* __restrict__ w_soft,
                               uint16_t* __restrict__ p_out, int64_t N, int64_t K) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N * (K / 2)) return;
  build_w_pair<GEN>(logits, f16, noise, seed, offset, pal, inv_tau, mode, w, w_soft, K, t, p_out);
}

// Many linears in one launch (fused_lut_kernel.cu:2071-2211 batches the per-layer build the
// same way): block b belongs to the descriptor whose block_begin is the last one <= b.
constexpr int kBuildWBlock = 256;
__global__ void build_w_batched_kernel(const plz_build_w_desc* __restrict__ descs, int n_desc,
                                       uint64_t offset, float inv_tau, int mode) {
  const int64_t b = blockIdx.x;
  int lo = 0, hi = n_desc - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (descs[mid].block_begin <= b) lo = mid; else hi = mid - 1;
  }
  const plz_build_w_desc d = descs[lo];
  const int64_t t = (b - d.block_begin) * kBuildWBlock + threadIdx.x;
  if (t >= d.N * (d.K / 2)) return;
  if (d.noise)
    build_w_pair<false>(d.logits, d.logits_dtype == PLZ_DT_FP16, d.noise, 0, 0, d.palette,
                        inv_tau, mode, d.w, d.w_soft, d.K, t, d.p_out);
  else  // the descriptor's own Philox key (uniform per block)
    build_w_pair<true>(d.logits, d.logits_dtype == PLZ_DT_FP16, nullptr, d.noise_seed,
                       offset + d.noise_counter, d.palette, inv_tau, mode, d.w, d.w_soft, d.K, t,
                       d.p_out);
}

}  // namespace plz

using namespace plz;

extern "C" {

int plz_gumbel_philox(float* noise, int64_t n, uint64_t seed, uint64_t offset, void* stream) {
  PLZ_REQUIRE(n >= 0 && n % 4 == 0, "plz_gumbel_philox: n (%lld) must be a multiple of 4",
              (long long)n);
  if (n == 0) return PLZ_OK;
  PLZ_REQUIRE(noise && ((uintptr_t)noise & 15) == 0,
              "plz_gumbel_philox: noise must be non-null and 16-byte aligned");
  const int64_t n4 = n / 4;
  hipLaunchKernelGGL(philox_gumbel_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, noise, n4, seed, offset);
  return check_launch("plz_gumbel_philox");
}

static int gumbel_lcg(float* noise, uint32_t seed, int64_t N, int64_t K, bool arith,
                      void* stream, const char* what) {
  PLZ_REQUIRE(N >= 0 && K >= 0, "%s: negative shape", what);
  if (N == 0 || K == 0) return PLZ_OK;
  PLZ_REQUIRE(noise && ((uintptr_t)noise & 15) == 0,
              "%s: noise must be non-null and 16-byte aligned", what);
  const int64_t n = N * K;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (arith)
    hipLaunchKernelGGL(lcg_gumbel_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, noise,
                       seed, N, K);
  else
    hipLaunchKernelGGL(lcg_gumbel_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, noise,
                       seed, N, K);
  return check_launch(what);
}

int plz_gumbel_lcg(float* noise, uint32_t seed, int64_t N, int64_t K, void* stream) {
  return gumbel_lcg(noise, seed, N, K, false, stream, "plz_gumbel_lcg");
}

int plz_gumbel_lcg_triton(float* noise, uint32_t seed, int64_t N, int64_t K, void* stream) {
  return gumbel_lcg(noise, seed, N, K, true, stream, "plz_gumbel_lcg_triton");
}

int64_t plz_pw_ref_plan(plz_pw_ref_desc* descs, int n, int64_t group_size) {
  if (n < 0 || (n > 0 && !descs) || group_size <= 0) {
    set_error("plz_pw_ref_plan: need n >= 0, non-null descriptors and group_size > 0");
    return -PLZ_EINVAL;
  }
  int64_t total = 0;
  for (int i = 0; i < n; ++i) {
    plz_pw_ref_desc& d = descs[i];
    if (d.K < 0 || d.N < 0 || d.N % group_size != 0 || d.K * d.N * 4 > 0xFFFFFFFFll) {
      set_error("plz_pw_ref_plan: descriptor %d: N (%lld) must be a multiple of group_size "
                "(%lld) and 4*K*N must fit 32 bits", i, (long long)d.N, (long long)group_size);
      return -PLZ_EINVAL;
    }
    const int64_t kn = d.K * d.N;
    if (kn > 0 && (!d.logits || !d.palette || !d.p_aos || !d.w ||
                   (((uintptr_t)d.logits | (uintptr_t)d.p_aos | (uintptr_t)d.w) & 1) ||
                   ((uintptr_t)d.palette & 7))) {
      set_error("plz_pw_ref_plan: descriptor %d: null or misaligned pointer", i);
      return -PLZ_EINVAL;
    }
    d.vec = (kn % 4 == 0 && ((uintptr_t)d.logits & 7) == 0 && ((uintptr_t)d.p_aos & 15) == 0 &&
             ((uintptr_t)d.w & 7) == 0) ? 1 : 0;
    d.block_begin = total;
    total += (kn + 4 * kPwBlock - 1) / (4 * kPwBlock);
  }
  return total;
}

int plz_soft_pw_ref_batched(const plz_pw_ref_desc* descs_device, int n, int64_t total_blocks,
                            int64_t group_size, float tau, uint32_t step_seed, void* stream) {
  PLZ_REQUIRE(n >= 0 && total_blocks >= 0, "plz_soft_pw_ref_batched: negative count");
  PLZ_REQUIRE(group_size > 0, "plz_soft_pw_ref_batched: group_size must be positive");
  PLZ_REQUIRE(tau > 0.f, "plz_soft_pw_ref_batched: tau must be positive");
  if (n == 0 || total_blocks == 0) return PLZ_OK;
  PLZ_REQUIRE(descs_device, "plz_soft_pw_ref_batched: null descriptor table");
  hipLaunchKernelGGL(pw_ref_batched_kernel, dim3((unsigned)total_blocks), dim3(kPwBlock), 0,
                     (hipStream_t)stream, descs_device, n, group_size, 1.f / tau, step_seed);
  return check_launch("plz_soft_pw_ref_batched");
}

static int build_w(const uint16_t* logits, int logits_dtype, bool gen, const float* noise,
                   uint64_t seed, uint64_t offset, const float* palette, float tau, int mode,
                   uint16_t* w, uint16_t* w_soft, uint16_t* p_out, int64_t N, int64_t K,
                   void* stream, const char* what) {
  PLZ_REQUIRE(N >= 0 && K >= 0, "%s: negative shape", what);
  PLZ_REQUIRE(K % 256 == 0, "%s: K (%lld) must be a multiple of 256", what, (long long)K);
  PLZ_REQUIRE(logits_dtype == PLZ_DT_BF16 || logits_dtype == PLZ_DT_FP16,
              "%s: logits dtype must be bf16 or fp16", what);
  PLZ_REQUIRE(mode == PLZ_W_SOFT || mode == PLZ_W_HARD_NOISY || mode == PLZ_W_HARD_PLAIN,
              "%s: unknown mode %d", what, mode);
  PLZ_REQUIRE(tau > 0.f, "%s: tau must be positive", what);
  if (N == 0 || K == 0) return PLZ_OK;
  PLZ_REQUIRE(logits && palette && w && (gen || noise), "%s: null pointer", what);
  PLZ_REQUIRE((((uintptr_t)logits | (uintptr_t)noise | (uintptr_t)palette) & 15) == 0 &&
                  (((uintptr_t)w | (uintptr_t)w_soft) & 3) == 0 && ((uintptr_t)p_out & 15) == 0,
              "%s: misaligned pointer", what);
  const int64_t n = N * K / 2;
  const dim3 grid((unsigned)((n + 255) / 256));
  const int f16 = logits_dtype == PLZ_DT_FP16 ? 1 : 0;
  if (gen)
    hipLaunchKernelGGL(build_w_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, logits, f16,
                       nullptr, seed, offset, palette, 1.f / tau, mode, w, w_soft, p_out, N, K);
  else
    hipLaunchKernelGGL(build_w_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, logits,
                       f16, noise, (uint64_t)0, (uint64_t)0, palette, 1.f / tau, mode, w, w_soft,
                       p_out, N, K);
  return check_launch(what);
}

int plz_soft_build_w(const uint16_t* logits, int logits_dtype, const float* noise,
                     const float* palette, float tau, int mode, uint16_t* w, uint16_t* w_soft,
                     uint16_t* p_out, int64_t N, int64_t K, void* stream) {
  return build_w(logits, logits_dtype, false, noise, 0, 0, palette, tau, mode, w, w_soft, p_out,
                 N, K, stream, "plz_soft_build_w");
}

int plz_soft_build_w_philox(const uint16_t* logits, int logits_dtype, uint64_t seed,
                            uint64_t offset, const float* palette, float tau, int mode,
                            uint16_t* w, uint16_t* w_soft, uint16_t* p_out, int64_t N, int64_t K,
                            void* stream) {
  return build_w(logits, logits_dtype, true, nullptr, seed, offset, palette, tau, mode, w, w_soft,
                 p_out, N, K, stream, "plz_soft_build_w_philox");
}

int64_t plz_build_w_plan(plz_build_w_desc* descs, int n) {
  if (n < 0 || (n > 0 && !descs)) {
    set_error("plz_build_w_plan: need n >= 0 and non-null descriptors");
    return -PLZ_EINVAL;
  }
  int64_t total = 0;
  for (int i = 0; i < n; ++i) {
    const plz_build_w_desc& d = descs[i];
    if (d.N < 0 || d.K < 0 || d.K % 256 != 0 ||
        (d.logits_dtype != PLZ_DT_BF16 && d.logits_dtype != PLZ_DT_FP16)) {
      set_error("plz_build_w_plan: descriptor %d: need K %% 256 == 0 and bf16/fp16 logits", i);
      return -PLZ_EINVAL;
    }
    if (d.N > 0 && d.K > 0 &&
        (!d.logits || !d.palette || !d.w ||
         (((uintptr_t)d.logits | (uintptr_t)d.noise | (uintptr_t)d.palette |
           (uintptr_t)d.p_out) & 15) ||
         (((uintptr_t)d.w | (uintptr_t)d.w_soft) & 3))) {
      set_error("plz_build_w_plan: descriptor %d: null or misaligned pointer", i);
      return -PLZ_EINVAL;
    }
    descs[i].block_begin = total;
    total += (d.N * (d.K / 2) + kBuildWBlock - 1) / kBuildWBlock;
  }
  return total;
}

int plz_soft_build_w_batched_philox(const plz_build_w_desc* descs_device, int n,
                                    int64_t total_blocks, uint64_t noise_offset, float tau,
                                    int mode, void* stream) {
  PLZ_REQUIRE(n >= 0 && total_blocks >= 0, "plz_soft_build_w_batched: negative count");
  PLZ_REQUIRE(mode == PLZ_W_SOFT || mode == PLZ_W_HARD_NOISY || mode == PLZ_W_HARD_PLAIN,
              "plz_soft_build_w_batched: unknown mode %d", mode);
  PLZ_REQUIRE(tau > 0.f, "plz_soft_build_w_batched: tau must be positive");
  if (n == 0 || total_blocks == 0) return PLZ_OK;
  PLZ_REQUIRE(descs_device, "plz_soft_build_w_batched: null descriptor table");
  hipLaunchKernelGGL(build_w_batched_kernel, dim3((unsigned)total_blocks), dim3(kBuildWBlock), 0,
                     (hipStream_t)stream, descs_device, n, noise_offset, 1.f / tau, mode);
  return check_launch("plz_soft_build_w_batched");
}

int plz_soft_build_w_batched(const plz_build_w_desc* descs_device, int n, int64_t total_blocks,
                             float tau, int mode, void* stream) {
  return plz_soft_build_w_batched_philox(descs_device, n, total_blocks, 0, tau, mode, stream);
}

}  // extern "C"
