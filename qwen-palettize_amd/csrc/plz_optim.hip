// Fused optimizer step of the layer training (train_qwen.py:154-221 FP32MasterOptimizer,
// :1303-1319 two-tier gradient clipping, :1343-1348 logits clamp to +-5 tau):
//
//   per clip group G:  coef_G = min(1, max_norm_G / (||grad over G||_2 + 1e-6))
//                      (torch.nn.utils.clip_grad_norm_)
//   per element:       g = grad * coef_G
//                      p = p * (1 - lr * wd)
//                      m = m + (1 - b1) (g - m)                 (torch lerp form)
//                      v = b2 v + (1 - b2) g^2
//                      p = p - (lr / bc1) m / (sqrt(v) / sqrt(bc2) + eps)
//                      p = clamp(p, lo, hi)
//                      param = bf16(p) (bf16 parameters keep an fp32 master p)
// which is torch.optim.AdamW's multi-tensor step (betas, eps, weight decay as given) on fp32
// masters. Two kernels stream every parameter once each: the squared-norm partials, then the
// update (the norms are finished on the device in between; no host synchronisation). HBM-bound:
// a bf16 parameter with master moves 30 bytes per element (grad read twice, m/v/master read and
// written, param written), in 16-byte accesses of 8 consecutive elements per thread.
#include <cmath>

#include "plz_common.h"
#include "palettize_hip.h"

namespace plz {
namespace opt {

constexpr int kThreads = 256;
constexpr int kVec = 8;                                  // contiguous elements per chunk
constexpr int kChunks = 4;                               // chunks per thread
constexpr int kBlockElems = kThreads * kVec * kChunks;   // elements per block: 8192

__device__ __forceinline__ int find_desc(const plz_adamw_desc* d, int n, int64_t b) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (d[mid].block_begin <= b) lo = mid; else hi = mid - 1;
  }
  return lo;
}
__device__ __forceinline__ float grad_at(const plz_adamw_desc& d, int64_t i) {
  return d.dtype == PLZ_DT_BF16 ? bf2f(reinterpret_cast<const uint16_t*>(d.grad)[i])
                                : reinterpret_cast<const float*>(d.grad)[i];
}
// 8 consecutive gradients starting at i (16-byte aligned: the whole chunk is in range)
__device__ __forceinline__ void grad8(const plz_adamw_desc& d, int64_t i, float (&g)[kVec]) {
  if (d.dtype == PLZ_DT_BF16) {
    const uint4 v = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(d.grad) + i);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      g[2 * j] = bf2f(w[j] & 0xffffu);
      g[2 * j + 1] = bf2f(w[j] >> 16);
    }
  } else {
    const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(d.grad) + i);
    const float4 a = p[0], b = p[1];
    g[0] = a.x; g[1] = a.y; g[2] = a.z; g[3] = a.w; g[4] = b.x; g[5] = b.y; g[6] = b.z; g[7] = b.w;
  }
}
__device__ __forceinline__ void load8(const float* p, float (&v)[kVec]) {
  const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
__device__ __forceinline__ void store8(float* p, const float (&v)[kVec]) {
  reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
  reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
}

template <int NT = kThreads>
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float s = 0.f;
  if (threadIdx.x == 0)
    for (int w = 0; w < NT / 64; ++w) s += red[w];
  return s;  // valid in thread 0
}

// partial[b] = sum of squared (unclipped) gradients of block b; group[b] = its clip group
__global__ __launch_bounds__(kThreads) void sumsq_kernel(const plz_adamw_desc* __restrict__ descs,
                                                         int n_desc, float* __restrict__ partial,
                                                         int* __restrict__ group) {
  __shared__ float red[kThreads / 64];
  const int64_t b = blockIdx.x;
  const plz_adamw_desc d = descs[find_desc(descs, n_desc, b)];
  const int64_t base = (b - d.block_begin) * kBlockElems;
  float s = 0.f;
  if (d.grad_sq) {  // the producer's sums of 512 elements: 16 per full block
    const int64_t i = base / 512 + threadIdx.x;
    if (threadIdx.x < kBlockElems / 512 && i < d.n / 512) s = d.grad_sq[i];
  } else {
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const int64_t i0 = base + ((int64_t)c * kThreads + threadIdx.x) * kVec;
      if (i0 + kVec <= d.n) {
        float g[kVec];
        grad8(d, i0, g);
#pragma unroll
        for (int j = 0; j < kVec; ++j) s += g[j] * g[j];
      } else {
        for (int64_t i = i0; i < d.n; ++i) {
          const float g = grad_at(d, i);
          s += g * g;
        }
      }
    }
  }
  s = block_sum(s, red);
  if (threadIdx.x == 0) {
    partial[b] = s;
    group[b] = d.clip_group;
  }
}

// coef[G] = min(1, max_norm[G] / (sqrt(sum of group G's partials) + 1e-6)); coef[2 + G] = norm
// (a fixed assignment of partials to threads and a fixed reduction tree: deterministic)
// One workgroup per clip group reads every partial: 1024 threads with 16 independent loads of
// each array in flight per thread, so the walk over the partials is a few memory round trips.
constexpr int kCoefThreads = 1024;
constexpr int kCoefUnroll = 16;
__global__ __launch_bounds__(kCoefThreads) void clip_coef_kernel(const float* __restrict__ partial,
                                                                 const int* __restrict__ group,
                                                                 int64_t nblocks, float max0,
                                                                 float max1,
                                                                 float* __restrict__ coef) {
  __shared__ float red[kCoefThreads / 64];
  const int G = blockIdx.x;
  float acc[kCoefUnroll];
#pragma unroll
  for (int u = 0; u < kCoefUnroll; ++u) acc[u] = 0.f;
  int64_t i = threadIdx.x;
  for (; i + (kCoefUnroll - 1) * kCoefThreads < nblocks; i += kCoefUnroll * kCoefThreads) {
    int gr[kCoefUnroll];
    float pv[kCoefUnroll];
#pragma unroll
    for (int u = 0; u < kCoefUnroll; ++u) {
      gr[u] = group[i + u * kCoefThreads];
      pv[u] = partial[i + u * kCoefThreads];
    }
#pragma unroll
    for (int u = 0; u < kCoefUnroll; ++u) acc[u] += gr[u] == G ? pv[u] : 0.f;
  }
  for (; i < nblocks; i += kCoefThreads) acc[0] += group[i] == G ? partial[i] : 0.f;
#pragma unroll
  for (int w = kCoefUnroll / 2; w > 0; w >>= 1)
#pragma unroll
    for (int u = 0; u < w; ++u) acc[u] += acc[u + w];
  const float s = block_sum<kCoefThreads>(acc[0], red);
  if (threadIdx.x == 0) {
    const float mx = G == 0 ? max0 : max1;
    const float c = mx / (sqrtf(s) + 1e-6f);
    coef[G] = mx > 0.f ? fminf(c, 1.f) : 1.f;  // max_norm <= 0: no clipping
    coef[2 + G] = sqrtf(s);
  }
}

struct Hyper {
  float beta1, beta2, eps, weight_decay, bc1, bc2_sqrt;
};
__device__ __forceinline__ float adamw_one(float g, float& p, float& m, float& v, float step_size,
                                           float decay, const Hyper& h, float lo, float hi) {
  if (h.weight_decay != 0.f) p *= decay;
  m = m + (1.f - h.beta1) * (g - m);
  v = v * h.beta2;
  v = v + (1.f - h.beta2) * g * g;
  const float denom = sqrtf(v) / h.bc2_sqrt + h.eps;
  p = p - step_size * (m / denom);
  p = fminf(fmaxf(p, lo), hi);
  return p;
}

// The next forward's weight of the two weights whose 8 logits (elements i0 .. i0+7 of a
// [N, K, 4] parameter, K even) were just updated, from their new bf16 bits lw: exactly what
// build_w_batched_kernel computes from the stored logits (same helper, same noise counters).
__device__ __forceinline__ void build_chunk(const plz_build_w_desc& bd, int64_t i0,
                                            const uint32_t (&lw)[4], uint64_t offset,
                                            float inv_tau, int mode) {
  const uint32_t w0 = (uint32_t)(i0 >> 2);  // N*K < 2^31 (checked by the plan)
  const uint32_t K = (uint32_t)bd.K;
  const uint32_t n = w0 / K, k = w0 - n * K;
  const float4 p = *reinterpret_cast<const float4*>(
      bd.palette + ((size_t)n * (K / kPalGroup) + k / kPalGroup) * 4);
  const float pc[4] = {p.x, p.y, p.z, p.w};
  float nz[8];
  if (bd.noise) {
    const float4 z0 = *reinterpret_cast<const float4*>(bd.noise + i0);
    const float4 z1 = *reinterpret_cast<const float4*>(bd.noise + i0 + 4);
    nz[0] = z0.x; nz[1] = z0.y; nz[2] = z0.z; nz[3] = z0.w;
    nz[4] = z1.x; nz[5] = z1.y; nz[6] = z1.z; nz[7] = z1.w;
  } else {
    float z[4];
    const uint64_t ctr = offset + bd.noise_counter + w0;
    philox_gumbel4(bd.noise_seed, ctr, z);
    nz[0] = z[0]; nz[1] = z[1]; nz[2] = z[2]; nz[3] = z[3];
    philox_gumbel4(bd.noise_seed, ctr + 1, z);
    nz[4] = z[0]; nz[5] = z[1]; nz[6] = z[2]; nz[7] = z[3];
  }
  uint32_t wo[2], so[2], po[4];
  build_w_two(lw, 0, nz, pc, inv_tau, mode, wo, so, po);
  *reinterpret_cast<uint32_t*>(bd.w + w0) = wo[0] | (wo[1] << 16);
  if (bd.w_soft) *reinterpret_cast<uint32_t*>(bd.w_soft + w0) = so[0] | (so[1] << 16);
  if (bd.p_out) *reinterpret_cast<uint4*>(bd.p_out + i0) = make_uint4(po[0], po[1], po[2], po[3]);
}

struct BuildArgs {
  const plz_build_w_desc* descs;  // entry i belongs to update descriptor i
  uint64_t offset;
  float inv_tau;
  int mode;
};

// The update of blocks block0 .. block0 + gridDim.x - 1. BUILD: every descriptor of these blocks
// has a build entry (the plan puts them after all others), whose weight is rebuilt from the
// updated logits.
template <bool BUILD>
__global__ __launch_bounds__(kThreads) void adamw_kernel(const plz_adamw_desc* __restrict__ descs,
                                                         int n_desc, const float* __restrict__ coef,
                                                         const Hyper h, int64_t block0,
                                                         const BuildArgs ba) {
  const int64_t b = blockIdx.x + block0;
  const int di = find_desc(descs, n_desc, b);
  const plz_adamw_desc d = descs[di];
  const int64_t base = (b - d.block_begin) * kBlockElems;
  const float c = coef[d.clip_group];
  const float step_size = d.lr / h.bc1;
  const float decay = 1.f - d.lr * h.weight_decay;
  float* p32 = d.master ? d.master : reinterpret_cast<float*>(d.param);
  if (base + kBlockElems <= d.n) {
    // whole block in range: every chunk's loads are issued before any chunk is updated (the
    // state arrays may alias for all the compiler knows, so it would not hoist them itself)
    float g[kChunks][kVec], p[kChunks][kVec], m[kChunks][kVec], v[kChunks][kVec];
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch) {
      const int64_t i0 = base + ((int64_t)ch * kThreads + threadIdx.x) * kVec;
      grad8(d, i0, g[ch]);
      load8(p32 + i0, p[ch]);
      load8(d.exp_avg + i0, m[ch]);
      load8(d.exp_avg_sq + i0, v[ch]);
    }
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch) {
      const int64_t i0 = base + ((int64_t)ch * kThreads + threadIdx.x) * kVec;
#pragma unroll
      for (int j = 0; j < kVec; ++j)
        adamw_one(g[ch][j] * c, p[ch][j], m[ch][j], v[ch][j], step_size, decay, h, d.clamp_lo,
                  d.clamp_hi);
      store8(d.exp_avg + i0, m[ch]);
      store8(d.exp_avg_sq + i0, v[ch]);
      store8(p32 + i0, p[ch]);
      if (d.master && d.dtype == PLZ_DT_BF16) {
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = f2bf2(p[ch][2 * j], p[ch][2 * j + 1]);
        *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(d.param) + i0) =
            make_uint4(w[0], w[1], w[2], w[3]);
        if (BUILD) build_chunk(ba.descs[di], i0, w, ba.offset, ba.inv_tau, ba.mode);
      } else if (d.master) {
        store8(reinterpret_cast<float*>(d.param) + i0, p[ch]);
      }
    }
    return;
  }
#pragma unroll
  for (int ch = 0; ch < kChunks; ++ch) {
    const int64_t i0 = base + ((int64_t)ch * kThreads + threadIdx.x) * kVec;
    if (i0 + kVec <= d.n) {
      float g[kVec], p[kVec], m[kVec], v[kVec];
      grad8(d, i0, g);
      load8(p32 + i0, p);
      load8(d.exp_avg + i0, m);
      load8(d.exp_avg_sq + i0, v);
#pragma unroll
      for (int j = 0; j < kVec; ++j)
        adamw_one(g[j] * c, p[j], m[j], v[j], step_size, decay, h, d.clamp_lo, d.clamp_hi);
      store8(d.exp_avg + i0, m);
      store8(d.exp_avg_sq + i0, v);
      store8(p32 + i0, p);
      if (d.master && d.dtype == PLZ_DT_BF16) {
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = f2bf2(p[2 * j], p[2 * j + 1]);
        *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(d.param) + i0) =
            make_uint4(w[0], w[1], w[2], w[3]);
        if (BUILD) build_chunk(ba.descs[di], i0, w, ba.offset, ba.inv_tau, ba.mode);
      } else if (d.master) {
        store8(reinterpret_cast<float*>(d.param) + i0, p);
      }
    } else {
      for (int64_t i = i0; i < d.n; ++i) {
        float p = p32[i], m = d.exp_avg[i], v = d.exp_avg_sq[i];
        adamw_one(grad_at(d, i) * c, p, m, v, step_size, decay, h, d.clamp_lo, d.clamp_hi);
        d.exp_avg[i] = m;
        d.exp_avg_sq[i] = v;
        p32[i] = p;
        if (d.master && d.dtype == PLZ_DT_BF16)
          reinterpret_cast<uint16_t*>(d.param)[i] = (uint16_t)f2bf(p);
        else if (d.master)
          reinterpret_cast<float*>(d.param)[i] = p;
      }
    }
  }
}

static unsigned grid_of(int64_t n) { return (unsigned)n; }

}  // namespace opt
}  // namespace plz

using namespace plz;
using namespace plz::opt;

extern "C" {

int64_t plz_adamw_plan(plz_adamw_desc* descs, int n) {
  if (n < 0 || (n > 0 && !descs)) {
    set_error("plz_adamw_plan: need n >= 0 and non-null descriptors");
    return -PLZ_EINVAL;
  }
  int64_t total = 0;
  for (int i = 0; i < n; ++i) {
    const plz_adamw_desc& d = descs[i];
    if (d.n < 0 || (d.dtype != PLZ_DT_BF16 && d.dtype != PLZ_DT_FP32) ||
        (d.clip_group != 0 && d.clip_group != 1) || !(d.clamp_lo <= d.clamp_hi)) {
      set_error("plz_adamw_plan: descriptor %d: bad size, dtype, clip group or clamp range", i);
      return -PLZ_EINVAL;
    }
    if (d.n > 0 && (!d.param || !d.grad || !d.exp_avg || !d.exp_avg_sq ||
                    (d.dtype == PLZ_DT_BF16 && !d.master))) {
      set_error("plz_adamw_plan: descriptor %d: null pointer (bf16 parameters need a master)", i);
      return -PLZ_EINVAL;
    }
    if ((((uintptr_t)d.param | (uintptr_t)d.grad | (uintptr_t)d.master | (uintptr_t)d.exp_avg |
          (uintptr_t)d.exp_avg_sq) & 15) != 0) {
      set_error("plz_adamw_plan: descriptor %d: pointers must be 16-byte aligned", i);
      return -PLZ_EINVAL;
    }
    if (d.grad_sq && (d.n % 512 != 0 || ((uintptr_t)d.grad_sq & 3) != 0)) {
      set_error("plz_adamw_plan: descriptor %d: grad_sq needs n %% 512 == 0 (one sum per 512 "
                "elements) and 4-byte alignment", i);
      return -PLZ_EINVAL;
    }
    descs[i].block_begin = total;
    total += (d.n + kBlockElems - 1) / kBlockElems;
  }
  return total;
}

size_t plz_adamw_workspace(int64_t total_blocks) {
  if (total_blocks <= 0) return 64;
  return ((size_t)total_blocks * 8 + 63) / 64 * 64 + 64;
}

// The step of plz_adamw_step / plz_adamw_step_build: norms, clip coefficients, then the update
// of blocks [0, split) and, with builds, of blocks [split, total) with their weights rebuilt.
static int adamw_step_impl(const plz_adamw_desc* descs_device, const BuildArgs* ba, int n,
                           int64_t total_blocks, int64_t split, float max_norm0, float max_norm1,
                           double beta1, double beta2, float eps, float weight_decay,
                           int64_t step, float* norms_out, void* workspace,
                           size_t workspace_bytes, hipStream_t s, const char* what) {
  PLZ_REQUIRE(n >= 0 && total_blocks >= 0 && step >= 1, "%s: bad count or step", what);
  PLZ_REQUIRE(beta1 >= 0.f && beta1 < 1.f && beta2 >= 0.f && beta2 < 1.f && eps > 0.f,
              "%s: need 0 <= betas < 1 and eps > 0", what);
  if (n == 0 || total_blocks == 0) return PLZ_OK;
  PLZ_REQUIRE(descs_device, "%s: null descriptor table", what);
  PLZ_REQUIRE(total_blocks < (1ll << 31), "%s: too many elements", what);
  PLZ_REQUIRE(split >= 0 && split <= total_blocks, "%s: split block out of range", what);
  const size_t need = plz_adamw_workspace(total_blocks);
  if (!workspace || workspace_bytes < need) {
    set_error("%s: workspace of %zu bytes needed, %zu given", what, need, workspace_bytes);
    return PLZ_EWORKSPACE;
  }
  float* partial = reinterpret_cast<float*>(workspace);
  int* group = reinterpret_cast<int*>(partial + total_blocks);
  float* coef = reinterpret_cast<float*>((char*)workspace + need - 64);
  hipLaunchKernelGGL(sumsq_kernel, dim3(grid_of(total_blocks)), dim3(kThreads), 0, s, descs_device,
                     n, partial, group);
  int rc = check_launch(what);
  if (rc) return rc;
  hipLaunchKernelGGL(clip_coef_kernel, dim3(2), dim3(kCoefThreads), 0, s, partial, group,
                     total_blocks, max_norm0, max_norm1, coef);
  if ((rc = check_launch(what))) return rc;
  // bias corrections in double on the host, as torch computes its Python-float scalars
  const float bc1 = (float)(1.0 - std::pow(beta1, (double)step));
  const float bc2_sqrt = (float)std::sqrt(1.0 - std::pow(beta2, (double)step));
  const Hyper h{(float)beta1, (float)beta2, eps, weight_decay, bc1, bc2_sqrt};
  const BuildArgs none{nullptr, 0, 1.f, 0};
  if (split > 0) {
    hipLaunchKernelGGL(adamw_kernel<false>, dim3(grid_of(split)), dim3(kThreads), 0, s,
                       descs_device, n, coef, h, (int64_t)0, none);
    if ((rc = check_launch(what))) return rc;
  }
  if (split < total_blocks) {
    // the builds read palettes that blocks [0, split) update: a second launch on the same
    // stream starts after all of them have finished
    if (ba)
      hipLaunchKernelGGL(adamw_kernel<true>, dim3(grid_of(total_blocks - split)), dim3(kThreads),
                         0, s, descs_device, n, coef, h, split, *ba);
    else
      hipLaunchKernelGGL(adamw_kernel<false>, dim3(grid_of(total_blocks - split)), dim3(kThreads),
                         0, s, descs_device, n, coef, h, split, none);
    if ((rc = check_launch(what))) return rc;
  }
  if (norms_out) {
    hipMemcpyAsync(norms_out, coef + 2, 2 * sizeof(float), hipMemcpyDeviceToDevice, s);
    return check_launch(what);
  }
  return PLZ_OK;
}

int plz_adamw_step(const plz_adamw_desc* descs_device, int n, int64_t total_blocks,
                   float max_norm0, float max_norm1, double beta1, double beta2, float eps,
                   float weight_decay, int64_t step, float* norms_out, void* workspace,
                   size_t workspace_bytes, void* stream) {
  return adamw_step_impl(descs_device, nullptr, n, total_blocks, total_blocks, max_norm0,
                         max_norm1, beta1, beta2, eps, weight_decay, step, norms_out, workspace,
                         workspace_bytes, (hipStream_t)stream, "plz_adamw_step");
}

int64_t plz_adamw_plan_build(plz_adamw_desc* descs, const plz_build_w_desc* builds, int n,
                             int64_t* split_block) {
  const int64_t total = plz_adamw_plan(descs, n);
  if (total < 0) return total;
  if (!split_block || (n > 0 && !builds)) {
    set_error("plz_adamw_plan_build: need the build table and split_block");
    return -PLZ_EINVAL;
  }
  int first = n;
  for (int i = 0; i < n; ++i) {
    const plz_build_w_desc& b = builds[i];
    if (!b.w) {
      if (first < n) {
        set_error("plz_adamw_plan_build: descriptor %d has no build but follows descriptor %d, "
                  "which has one: descriptors with a build must come last", i, first);
        return -PLZ_EINVAL;
      }
      continue;
    }
    if (first == n) first = i;
    const plz_adamw_desc& d = descs[i];
    plz_build_w_desc probe = b;
    if (d.dtype != PLZ_DT_BF16 || !d.master || b.logits != d.param ||
        b.logits_dtype != PLZ_DT_BF16 || b.N <= 0 || b.K <= 0 || b.N * b.K * 4 != d.n ||
        b.N * b.K >= (1ll << 31) || plz_build_w_plan(&probe, 1) < 0) {
      set_error("plz_adamw_plan_build: build %d must rebuild its own bf16 [N, K, 4] parameter "
                "(logits == param, N*K*4 == n, N*K < 2^31, K %% 256 == 0, aligned palette and w)", i);
      return -PLZ_EINVAL;
    }
  }
  *split_block = first < n ? descs[first].block_begin : total;
  return total;
}

int plz_adamw_step_build(const plz_adamw_desc* descs_device, const plz_build_w_desc* builds_device,
                         int n, int64_t total_blocks, int64_t split_block, uint64_t noise_offset,
                         float tau, int mode, float max_norm0, float max_norm1, double beta1,
                         double beta2, float eps, float weight_decay, int64_t step,
                         float* norms_out, void* workspace, size_t workspace_bytes,
                         void* stream) {
  const char* what = "plz_adamw_step_build";
  PLZ_REQUIRE(mode == PLZ_W_SOFT || mode == PLZ_W_HARD_NOISY || mode == PLZ_W_HARD_PLAIN,
              "%s: unknown mode %d", what, mode);
  PLZ_REQUIRE(tau > 0.f, "%s: tau must be positive", what);
  PLZ_REQUIRE(builds_device || split_block >= total_blocks, "%s: null build table", what);
  const BuildArgs ba{builds_device, noise_offset, 1.f / tau, mode};
  return adamw_step_impl(descs_device, &ba, n, total_blocks, split_block, max_norm0, max_norm1,
                         beta1, beta2, eps, weight_decay, step, norms_out, workspace,
                         workspace_bytes, (hipStream_t)stream, what);
}

}  // extern "C"
