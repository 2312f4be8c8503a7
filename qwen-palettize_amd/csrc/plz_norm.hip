// Fused RMSNorm and SwiGLU of the Qwen3 decoder layer, plus the bias-gradient reduction.
//
// RMSNorm follows HF Qwen3RMSNorm (transformers models/qwen3/modeling_qwen3.py:50-64):
//   h = x.float() * rsqrt(mean(x.float()^2) + eps);  y = weight * h.to(bf16)
// where the final product is a bf16 x bf16 multiply (fp32 compute, one rounding).
// SwiGLU follows Qwen3MLP (modeling_qwen3.py:70-83): h = act(gate) * up with act = silu on
// bf16 tensors: silu rounded to bf16, then the bf16 product rounded again.
// There is no counterpart kernel in the reference (it calls the HF modules).
#include "plz_common.h"

namespace plz {

constexpr int kNormMaxChunks = 8;  // cols <= 8 * 512 = 4096

// Row shapes: LPR lanes per row (RPW = 64 / LPR rows per wave) and up to MAXC 8-column chunks
// per lane. Per-head norms (128 columns) put 4 rows in a wave, so no lane idles; hidden-size
// rows (2560) take a whole wave with 5 chunks per lane.
template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
#pragma unroll
  for (int off = LPR / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// bf16 a + b as torch adds two bf16 tensors (fp32 sum, one rounding), 8 lanes at a time
__device__ __forceinline__ uint4 add8(uint4 a, uint4 b) {
  float fa[8], fb[8];
  unpack8(a, fa);
  unpack8(b, fb);
#pragma unroll
  for (int j = 0; j < 8; ++j) fa[j] = fa[j] + fb[j];
  return pack8(fa);
}

// ADD: the row is first the bf16 sum x + res (a residual add, written to sum), then normalised.
template <int LPR, int MAXC, bool ADD = false>
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ wt,
                                                          uint16_t* __restrict__ y,
                                                          float* __restrict__ rstd, int64_t rows,
                                                          int64_t cols, float eps,
                                                          const uint16_t* __restrict__ res = nullptr,
                                                          uint16_t* __restrict__ sum = nullptr) {
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63, sub = lane / LPR, l = lane % LPR;
  const int64_t row = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + sub;
  const bool valid = row < rows;  // lanes of a missing row compute on zeros (shuffles stay whole)
  const int nch = (int)(cols / 8);
  const uint4* xr = reinterpret_cast<const uint4*>(x + (valid ? row : 0) * cols);
  uint4 xv[MAXC];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = l + LPR * i;
    xv[i] = make_uint4(0, 0, 0, 0);
    if (valid && c < nch) {
      xv[i] = xr[c];
      if (ADD) {
        xv[i] = add8(xv[i], reinterpret_cast<const uint4*>(res + row * cols)[c]);
        reinterpret_cast<uint4*>(sum + row * cols)[c] = xv[i];
      }
      float f[8];
      unpack8(xv[i], f);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += f[j] * f[j];
    }
  }
  ss = row_sum<LPR>(ss);
  if (!valid) return;
  const float r = rsqrtf(ss / (float)cols + eps);
  if (l == 0 && rstd) rstd[row] = r;
  uint4* yr = reinterpret_cast<uint4*>(y + row * cols);
  const uint4* wr = reinterpret_cast<const uint4*>(wt);
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = l + LPR * i;
    if (c < nch) {
      float f[8], w[8], o[8];
      unpack8(xv[i], f);
      unpack8(wr[c], w);
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = w[j] * bf2f(f2bf(f[j] * r));
      yr[c] = pack8(o);
    }
  }
}

// Pieces of the norm backward for one 8-column chunk, each product and sum rounded on its own
// (no contraction), so that every kernel that forms them (this one and the fused per-head norm +
// RoPE below) produces the same bits: dot += (g w) (x r), and r ((g w) - (x r) dot).
__device__ __forceinline__ float norm_bwd_dot(const float f[8], const float g[8], const float w[8],
                                              float r, float dot) {
#pragma clang fp contract(off)
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float h = f[j] * r, t = g[j] * w[j];
    dot = dot + t * h;
  }
  return dot;
}
__device__ __forceinline__ void norm_bwd_out(const float f[8], const float g[8], const float w[8],
                                             float r, float dot, float o[8]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float h = f[j] * r, t = g[j] * w[j];
    o[j] = r * (t - h * dot);
  }
}

// Backward. With h = x r, g = grad_y * w (fp32):
//   grad_x = r * (g - h * mean(g * h)),  grad_w = sum_rows grad_y * bf16(h)
// Each workgroup takes a strided set of row groups, U groups per iteration (their loads are
// all issued before any is used, so short rows do not pay the memory latency per row);
// per-lane column partials of grad_w are summed over the workgroup's rows in LDS (fixed order)
// and written to partial[block][cols]; a second kernel adds the blocks in a fixed order.
// WG = false: no weight gradient (frozen weights: no partials, no LDS, no second kernel).
// ADD: grad_x = bf16(norm backward) + add, as autograd sums the two gradients of a residual
// stream that also feeds this norm (bf16 + bf16, one rounding).
template <int LPR, int MAXC, int U, bool WG = true, bool ADD = false>
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wt, const float* __restrict__ rstd,
    const uint16_t* __restrict__ gy, uint16_t* __restrict__ gx, float* __restrict__ partial,
    int64_t rows, int64_t cols, const uint16_t* __restrict__ add = nullptr) {
  constexpr int RPW = 64 / LPR;
  __shared__ float red[WG ? 4 * RPW : 1][MAXC][LPR][8];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, sub = lane / LPR, l = lane % LPR;
  const int nch = (int)(cols / 8);
  const uint4* wr = reinterpret_cast<const uint4*>(wt);
  float gw[MAXC][8];
#pragma unroll
  for (int i = 0; i < MAXC; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) gw[i][j] = 0.f;
  const int64_t step = (int64_t)gridDim.x * 4 * RPW;  // rows between a wave's row groups
  for (int64_t r0 = ((int64_t)blockIdx.x * 4 + wave) * RPW; r0 < rows; r0 += step * U) {
    uint4 xv[U][MAXC], gv[U][MAXC];
    float rs[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t row = r0 + step * u + sub;
      const bool valid = row < rows;
      rs[u] = valid ? rstd[row] : 0.f;
#pragma unroll
      for (int i = 0; i < MAXC; ++i) {
        const int c = l + LPR * i;
        xv[u][i] = make_uint4(0, 0, 0, 0);
        gv[u][i] = xv[u][i];
        if (valid && c < nch) {
          xv[u][i] = reinterpret_cast<const uint4*>(x + row * cols)[c];
          gv[u][i] = reinterpret_cast<const uint4*>(gy + row * cols)[c];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t row = r0 + step * u + sub;
      const float r = rs[u];
      float dot = 0.f;
#pragma unroll
      for (int i = 0; i < MAXC; ++i) {
        const int c = l + LPR * i;
        if (c < nch) {
          float f[8], g[8], w[8];
          unpack8(xv[u][i], f);
          unpack8(gv[u][i], g);
          unpack8(wr[c], w);
          dot = norm_bwd_dot(f, g, w, r, dot);
          if (WG)
#pragma unroll
            for (int j = 0; j < 8; ++j)
              gw[i][j] += g[j] * bf2f(f2bf(f[j] * r));  // zero for a missing row (g = 0)
        }
      }
      dot = row_sum<LPR>(dot) / (float)cols;
      if (row < rows) {
        uint4* outr = reinterpret_cast<uint4*>(gx + row * cols);
#pragma unroll
        for (int i = 0; i < MAXC; ++i) {
          const int c = l + LPR * i;
          if (c < nch) {
            float f[8], g[8], w[8], o[8];
            unpack8(xv[u][i], f);
            unpack8(gv[u][i], g);
            unpack8(wr[c], w);
            norm_bwd_out(f, g, w, r, dot, o);
            outr[c] = ADD ? add8(pack8(o), reinterpret_cast<const uint4*>(add + row * cols)[c])
                          : pack8(o);
          }
        }
      }
    }
  }
  if (!WG) return;
#pragma unroll
  for (int i = 0; i < MAXC; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) red[wave * RPW + sub][i][l][j] = gw[i][j];
  __syncthreads();
  // column chunk c = l + LPR*i summed over the workgroup's 4*RPW row slots in order
  for (int idx = threadIdx.x; idx < nch * 8; idx += 256) {
    const int c = idx / 8, j = idx % 8;
    const int i = c / LPR, ll = c % LPR;
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < 4 * RPW; ++w) sum += red[w][i][ll][j];
    partial[(int64_t)blockIdx.x * cols + idx] = sum;
  }
}

// out[c] = sum over the blocks' partials of column c: 64 columns per workgroup, its 16 waves
// take every 16th block (8 loads in flight per lane), then their sums are added in a fixed tree.
constexpr int kSumWaves = 16;
__global__ __launch_bounds__(kSumWaves * 64) void sum_blocks_kernel(
    const float* __restrict__ partial, float* __restrict__ out, int blocks, int64_t cols) {
  __shared__ float red[kSumWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + lane;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (c < cols) {
    int b = wave;
    for (; b + 7 * kSumWaves < blocks; b += 8 * kSumWaves)
#pragma unroll
      for (int u = 0; u < 8; ++u) acc[u] += partial[(int64_t)(b + kSumWaves * u) * cols + c];
    for (; b < blocks; b += kSumWaves) acc[0] += partial[(int64_t)b * cols + c];
  }
  red[wave][lane] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  __syncthreads();
  if (wave == 0 && c < cols) {
    float v[kSumWaves];
#pragma unroll
    for (int w = 0; w < kSumWaves; ++w) v[w] = red[w][lane];
#pragma unroll
    for (int h = kSumWaves / 2; h > 0; h >>= 1)
#pragma unroll
      for (int w = 0; w < h; ++w) v[w] += v[w + h];
    out[c] = v[0];
  }
}

__device__ __forceinline__ float silu(float g) { return g / (1.f + __expf(-g)); }

// 8 consecutive elements: h = bf16(silu(g)) * u, and its gradients
__device__ __forceinline__ uint4 swiglu_fwd8(uint4 gate, uint4 up) {
  float g[8], u[8], o[8];
  unpack8(gate, g);
  unpack8(up, u);
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = swiglu_elem(g[j], u[j]);
  return pack8(o);
}

__global__ void swiglu_fwd_kernel(const uint16_t* __restrict__ gate, const uint16_t* __restrict__ up,
                                  uint16_t* __restrict__ h, int64_t n8) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n8) return;
  reinterpret_cast<uint4*>(h)[t] =
      swiglu_fwd8(reinterpret_cast<const uint4*>(gate)[t], reinterpret_cast<const uint4*>(up)[t]);
}

__global__ void swiglu_bwd_kernel(const uint16_t* __restrict__ gate, const uint16_t* __restrict__ up,
                                  const uint16_t* __restrict__ gh, uint16_t* __restrict__ gg,
                                  uint16_t* __restrict__ gu, int64_t n8) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n8) return;
  swiglu_bwd8(reinterpret_cast<const uint4*>(gate)[t], reinterpret_cast<const uint4*>(up)[t],
              reinterpret_cast<const uint4*>(gh)[t], reinterpret_cast<uint4*>(gg)[t],
              reinterpret_cast<uint4*>(gu)[t]);
}

// The same on rows x F elements whose operands have their own row pitches (elements, multiples
// of 8): gate and up side by side in one [rows, 2F] tensor (a fused gate/up projection), h and
// the gradients wherever the caller keeps them.
__global__ void swiglu_fwd_rows_kernel(const uint16_t* __restrict__ gate,
                                       const uint16_t* __restrict__ up, int64_t ld_in,
                                       uint16_t* __restrict__ h, int64_t ld_h, int64_t rows,
                                       int64_t f8) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= rows * f8) return;
  const int64_t r = t / f8, c = (t % f8) * 8;
  *reinterpret_cast<uint4*>(h + r * ld_h + c) =
      swiglu_fwd8(*reinterpret_cast<const uint4*>(gate + r * ld_in + c),
                  *reinterpret_cast<const uint4*>(up + r * ld_in + c));
}
__global__ void swiglu_bwd_rows_kernel(const uint16_t* __restrict__ gate,
                                       const uint16_t* __restrict__ up, int64_t ld_in,
                                       const uint16_t* __restrict__ gh, int64_t ld_h,
                                       uint16_t* __restrict__ gg, uint16_t* __restrict__ gu,
                                       int64_t ld_g, int64_t rows, int64_t f8) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= rows * f8) return;
  const int64_t r = t / f8, c = (t % f8) * 8;
  swiglu_bwd8(*reinterpret_cast<const uint4*>(gate + r * ld_in + c),
              *reinterpret_cast<const uint4*>(up + r * ld_in + c),
              *reinterpret_cast<const uint4*>(gh + r * ld_h + c),
              *reinterpret_cast<uint4*>(gg + r * ld_g + c), *reinterpret_cast<uint4*>(gu + r * ld_g + c));
}

// grad_bias[n] = sum_m grad_y[m, n]: one thread per column, rows in order.
__global__ void bias_grad_kernel(const uint16_t* __restrict__ gy, float* __restrict__ gb,
                                 int64_t M, int64_t N) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  float s = 0.f;
  for (int64_t m = 0; m < M; ++m) s += bf2f(gy[m * N + n]);
  gb[n] = s;
}

// ---- per-head RMSNorm + RoPE (q_norm / k_norm then apply_rotary_pos_emb) ----------------
// HF Qwen3 attention normalises each head's 128 query / key values (Qwen3RMSNorm) and then
// rotates them (apply_rotary_pos_emb, rotate_half convention). One 16-lane DPP row per (token,
// head): lane l holds columns 8 l .. 8 l + 7, and the rotation partner of column j < 64,
// column j + 64, sits in lane l ^ 8 (row_ror:8). Every value is computed exactly as the
// separate kernels compute it (rmsnorm_fwd_kernel<16, 1> then rope_kernel, and rope_kernel<true>
// then rmsnorm_bwd_kernel<16, 1, U>), so the fused pair is bit-identical to them; the norm's own
// weight gradient is not formed (the layer's per-head norms are frozen).
constexpr int HNR_D = 128;
__device__ __forceinline__ uint32_t dpp_ror8(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false);
}
__device__ __forceinline__ uint4 dpp_ror8(uint4 v) {
  return make_uint4(dpp_ror8(v.x), dpp_ror8(v.y), dpp_ror8(v.z), dpp_ror8(v.w));
}
__device__ __forceinline__ void load8(const float* p, float f[8]) {
  const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
  f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
  f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}

// rows = tokens x heads rows of 128; the position of row t is (t / heads) % S
__global__ __launch_bounds__(256) void head_norm_rope_fwd_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wt, const float* __restrict__ cosv,
    const float* __restrict__ sinv, uint16_t* __restrict__ y, float* __restrict__ rstd,
    int64_t rows, int64_t S, int heads, float eps) {
  const int lane = threadIdx.x & 63, sub = lane >> 4, l = lane & 15;
  const int64_t row = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 4 + sub;
  const bool valid = row < rows;  // a missing row's 16 lanes compute on zeros together
  const uint4 xv = valid ? reinterpret_cast<const uint4*>(x + row * HNR_D)[l] : make_uint4(0, 0, 0, 0);
  float f[8];
  unpack8(xv, f);
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) ss += f[j] * f[j];
  ss = row_sum<16>(ss);
  const float r = rsqrtf(ss / (float)HNR_D + eps);
  float w[8], o[8];
  unpack8(reinterpret_cast<const uint4*>(wt)[l], w);
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = w[j] * bf2f(f2bf(f[j] * r));
  const uint4 nv = pack8(o);            // the norm's bf16 output
  const uint4 pv = dpp_ror8(nv);        // the partner lane's
  if (!valid) return;
  if (l == 0 && rstd) rstd[row] = r;
  const int64_t pos = (row / heads) % S;
  float n[8], pn[8], c[8], sn[8], out[8];
  unpack8(nv, n);
  unpack8(pv, pn);
  load8(cosv + pos * HNR_D + 8 * l, c);
  load8(sinv + pos * HNR_D + 8 * l, sn);
  {
#pragma clang fp contract(off)  // products and sums rounded one by one, as rope_kernel does
    if (l < 8) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float a = n[j] * c[j], b = pn[j] * sn[j];
        out[j] = a - b;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float a = n[j] * c[j], b = pn[j] * sn[j];
        out[j] = a + b;
      }
    }
  }
  reinterpret_cast<uint4*>(y + row * HNR_D)[l] = pack8(out);
}

__global__ __launch_bounds__(256) void head_norm_rope_bwd_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wt, const float* __restrict__ rstd,
    const float* __restrict__ cosv, const float* __restrict__ sinv,
    const uint16_t* __restrict__ gy, uint16_t* __restrict__ gx, int64_t rows, int64_t S,
    int heads) {
  const int lane = threadIdx.x & 63, sub = lane >> 4, l = lane & 15;
  const int64_t row = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 4 + sub;
  const bool valid = row < rows;
  const uint4 zero = make_uint4(0, 0, 0, 0);
  const uint4 gv = valid ? reinterpret_cast<const uint4*>(gy + row * HNR_D)[l] : zero;
  const uint4 xv = valid ? reinterpret_cast<const uint4*>(x + row * HNR_D)[l] : zero;
  const uint4 pg = dpp_ror8(gv);  // the partner lane's output gradient
  const int64_t pos = valid ? (row / heads) % S : 0;
  float g[8], p[8], c[8], sp[8], gn[8];
  unpack8(gv, g);
  unpack8(pg, p);
  load8(cosv + pos * HNR_D + 8 * l, c);
  load8(sinv + pos * HNR_D + 8 * (l ^ 8), sp);  // sin at the partner's columns
  {
#pragma clang fp contract(off)  // the transposed rotation, as rope_kernel<true>
    if (l < 8) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float a = g[j] * c[j], b = p[j] * sp[j];
        gn[j] = a + b;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float a = g[j] * c[j], b = p[j] * sp[j];
        gn[j] = a - b;
      }
    }
  }
  // the norm's backward on the rotation's bf16 gradient
  const uint4 gnv = pack8(gn);
  float f[8], gb[8], w[8];
  unpack8(xv, f);
  unpack8(gnv, gb);
  unpack8(reinterpret_cast<const uint4*>(wt)[l], w);
  const float r = valid ? rstd[row] : 0.f;
  float dot = norm_bwd_dot(f, gb, w, r, 0.f);
  dot = row_sum<16>(dot) / (float)HNR_D;
  if (!valid) return;
  float o[8];
  norm_bwd_out(f, gb, w, r, dot, o);
  reinterpret_cast<uint4*>(gx + row * HNR_D)[l] = pack8(o);
}

// Kernel shape of a row width: lanes per row, chunks per lane, row groups per iteration.
struct NormShape {
  int lpr, maxc, u;
};
static NormShape norm_shape(int64_t cols) {
  if (cols <= 128) return {16, 1, 4};
  if (cols <= 512) return {64, 1, 4};
  return {64, kNormMaxChunks, 1};
}
static int rmsnorm_bwd_blocks(int64_t rows, int64_t cols) {
  const NormShape sh = norm_shape(cols);
  const int64_t per_block = 4LL * (64 / sh.lpr) * sh.u;
  const int64_t b = (rows + per_block - 1) / per_block;
  return (int)(b < 1024 ? b : 1024);
}

static bool a16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace plz

using namespace plz;

extern "C" {

int plz_rmsnorm_fwd(const uint16_t* x, const uint16_t* weight, uint16_t* y, float* rstd,
                    int64_t rows, int64_t cols, float eps, void* stream) {
  PLZ_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && cols <= 64 * 8 * kNormMaxChunks,
              "plz_rmsnorm_fwd: cols (%lld) must be a positive multiple of 8 up to 4096",
              (long long)cols);
  if (rows == 0) return PLZ_OK;
  PLZ_REQUIRE(x && weight && y && a16(x) && a16(weight) && a16(y),
              "plz_rmsnorm_fwd: x, weight, y must be non-null and 16-byte aligned");
  const NormShape sh = norm_shape(cols);
  const int64_t per_block = 4LL * (64 / sh.lpr);
  const dim3 grid((unsigned)((rows + per_block - 1) / per_block));
  if (sh.lpr == 16)
    hipLaunchKernelGGL((rmsnorm_fwd_kernel<16, 1>), grid, dim3(256), 0, (hipStream_t)stream, x,
                       weight, y, rstd, rows, cols, eps);
  else if (sh.maxc == 1)
    hipLaunchKernelGGL((rmsnorm_fwd_kernel<64, 1>), grid, dim3(256), 0, (hipStream_t)stream, x,
                       weight, y, rstd, rows, cols, eps);
  else
    hipLaunchKernelGGL((rmsnorm_fwd_kernel<64, kNormMaxChunks>), grid, dim3(256), 0,
                       (hipStream_t)stream, x, weight, y, rstd, rows, cols, eps);
  return check_launch("plz_rmsnorm_fwd");
}

size_t plz_rmsnorm_bwd_workspace(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return (size_t)rmsnorm_bwd_blocks(rows, cols) * cols * sizeof(float);
}

int plz_rmsnorm_bwd(const uint16_t* x, const uint16_t* weight, const float* rstd,
                    const uint16_t* grad_y, uint16_t* grad_x, float* grad_weight,
                    void* workspace, size_t workspace_bytes, int64_t rows, int64_t cols,
                    void* stream) {
  PLZ_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && cols <= 64 * 8 * kNormMaxChunks,
              "plz_rmsnorm_bwd: cols (%lld) must be a positive multiple of 8 up to 4096",
              (long long)cols);
  PLZ_REQUIRE(grad_weight, "plz_rmsnorm_bwd: null grad_weight");
  if (rows == 0) {
    zero_async(grad_weight, (size_t)cols * 4, (hipStream_t)stream);
    return check_launch("plz_rmsnorm_bwd");
  }
  PLZ_REQUIRE(x && weight && rstd && grad_y && grad_x && a16(x) && a16(weight) && a16(grad_y) &&
                  a16(grad_x),
              "plz_rmsnorm_bwd: operands must be non-null and 16-byte aligned");
  const size_t need = plz_rmsnorm_bwd_workspace(rows, cols);
  if (!workspace || workspace_bytes < need) {
    set_error("plz_rmsnorm_bwd: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
    return PLZ_EWORKSPACE;
  }
  const int blocks = rmsnorm_bwd_blocks(rows, cols);
  float* part = reinterpret_cast<float*>(workspace);
  const NormShape sh = norm_shape(cols);
  if (sh.lpr == 16)
    hipLaunchKernelGGL((rmsnorm_bwd_kernel<16, 1, 4>), dim3(blocks), dim3(256), 0,
                       (hipStream_t)stream, x, weight, rstd, grad_y, grad_x, part, rows, cols);
  else if (sh.maxc == 1)
    hipLaunchKernelGGL((rmsnorm_bwd_kernel<64, 1, 4>), dim3(blocks), dim3(256), 0,
                       (hipStream_t)stream, x, weight, rstd, grad_y, grad_x, part, rows, cols);
  else
    hipLaunchKernelGGL((rmsnorm_bwd_kernel<64, kNormMaxChunks, 1>), dim3(blocks), dim3(256), 0,
                       (hipStream_t)stream, x, weight, rstd, grad_y, grad_x, part, rows, cols);
  int rc = check_launch("plz_rmsnorm_bwd");
  if (rc) return rc;
  hipLaunchKernelGGL(sum_blocks_kernel, dim3((unsigned)((cols + 63) / 64)),
                     dim3(kSumWaves * 64), 0, (hipStream_t)stream, part, grad_weight, blocks, cols);
  return check_launch("plz_rmsnorm_bwd/reduce");
}

int plz_swiglu_fwd(const uint16_t* gate, const uint16_t* up, uint16_t* h, int64_t n,
                   void* stream) {
  PLZ_REQUIRE(n >= 0 && n % 8 == 0, "plz_swiglu_fwd: n (%lld) must be a multiple of 8",
              (long long)n);
  if (n == 0) return PLZ_OK;
  PLZ_REQUIRE(gate && up && h && a16(gate) && a16(up) && a16(h),
              "plz_swiglu_fwd: operands must be non-null and 16-byte aligned");
  const int64_t n8 = n / 8;
  hipLaunchKernelGGL(swiglu_fwd_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, gate, up, h, n8);
  return check_launch("plz_swiglu_fwd");
}

int plz_swiglu_bwd(const uint16_t* gate, const uint16_t* up, const uint16_t* grad_h,
                   uint16_t* grad_gate, uint16_t* grad_up, int64_t n, void* stream) {
  PLZ_REQUIRE(n >= 0 && n % 8 == 0, "plz_swiglu_bwd: n (%lld) must be a multiple of 8",
              (long long)n);
  if (n == 0) return PLZ_OK;
  PLZ_REQUIRE(gate && up && grad_h && grad_gate && grad_up && a16(gate) && a16(up) &&
                  a16(grad_h) && a16(grad_gate) && a16(grad_up),
              "plz_swiglu_bwd: operands must be non-null and 16-byte aligned");
  const int64_t n8 = n / 8;
  hipLaunchKernelGGL(swiglu_bwd_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, gate, up, grad_h, grad_gate, grad_up, n8);
  return check_launch("plz_swiglu_bwd");
}

int plz_swiglu_fwd_rows(const uint16_t* gate, const uint16_t* up, int64_t ld_in, uint16_t* h,
                        int64_t ld_h, int64_t rows, int64_t F, void* stream) {
  PLZ_REQUIRE(rows >= 0 && F >= 0 && F % 8 == 0 && ld_in % 8 == 0 && ld_h % 8 == 0 &&
                  ld_in >= F && ld_h >= F,
              "plz_swiglu_fwd_rows: F and the row pitches must be multiples of 8, pitches >= F");
  if (rows == 0 || F == 0) return PLZ_OK;
  PLZ_REQUIRE(gate && up && h && a16(gate) && a16(up) && a16(h),
              "plz_swiglu_fwd_rows: operands must be non-null and 16-byte aligned");
  const int64_t n = rows * (F / 8);
  hipLaunchKernelGGL(swiglu_fwd_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, gate, up, ld_in, h, ld_h, rows, F / 8);
  return check_launch("plz_swiglu_fwd_rows");
}

int plz_swiglu_bwd_rows(const uint16_t* gate, const uint16_t* up, int64_t ld_in,
                        const uint16_t* grad_h, int64_t ld_h, uint16_t* grad_gate,
                        uint16_t* grad_up, int64_t ld_g, int64_t rows, int64_t F, void* stream) {
  PLZ_REQUIRE(rows >= 0 && F >= 0 && F % 8 == 0 && ld_in % 8 == 0 && ld_h % 8 == 0 &&
                  ld_g % 8 == 0 && ld_in >= F && ld_h >= F && ld_g >= F,
              "plz_swiglu_bwd_rows: F and the row pitches must be multiples of 8, pitches >= F");
  if (rows == 0 || F == 0) return PLZ_OK;
  PLZ_REQUIRE(gate && up && grad_h && grad_gate && grad_up && a16(gate) && a16(up) &&
                  a16(grad_h) && a16(grad_gate) && a16(grad_up),
              "plz_swiglu_bwd_rows: operands must be non-null and 16-byte aligned");
  const int64_t n = rows * (F / 8);
  hipLaunchKernelGGL(swiglu_bwd_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, gate, up, ld_in, grad_h, ld_h, grad_gate, grad_up, ld_g,
                     rows, F / 8);
  return check_launch("plz_swiglu_bwd_rows");
}

int plz_bias_grad(const uint16_t* grad_y, float* grad_bias, int64_t M, int64_t N, void* stream) {
  PLZ_REQUIRE(M >= 0 && N >= 0, "plz_bias_grad: negative shape");
  if (N == 0) return PLZ_OK;
  PLZ_REQUIRE(grad_bias && (M == 0 || grad_y), "plz_bias_grad: null pointer");
  hipLaunchKernelGGL(bias_grad_kernel, dim3((unsigned)((N + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, grad_y, grad_bias, M, N);
  return check_launch("plz_bias_grad");
}


int plz_head_norm_rope_fwd(const uint16_t* x, const uint16_t* weight, const float* cos_table,
                           const float* sin_table, uint16_t* y, float* rstd, int64_t rows,
                           int64_t seq, int heads, int head_dim, float eps, void* stream) {
  PLZ_REQUIRE(head_dim == HNR_D, "plz_head_norm_rope_fwd: head_dim %d is not supported (128 only)",
              head_dim);
  PLZ_REQUIRE(rows >= 0 && seq > 0 && heads > 0, "plz_head_norm_rope_fwd: need rows >= 0, seq > 0, heads > 0");
  if (rows == 0) return PLZ_OK;
  PLZ_REQUIRE(x && weight && cos_table && sin_table && y && a16(x) && a16(weight) &&
                  a16(cos_table) && a16(sin_table) && a16(y),
              "plz_head_norm_rope_fwd: operands must be non-null and 16-byte aligned");
  const int64_t n = rows * heads;
  hipLaunchKernelGGL(head_norm_rope_fwd_kernel, dim3((unsigned)((n + 15) / 16)), dim3(256), 0,
                     (hipStream_t)stream, x, weight, cos_table, sin_table, y, rstd, n, seq, heads,
                     eps);
  return check_launch("plz_head_norm_rope_fwd");
}

int plz_head_norm_rope_bwd(const uint16_t* x, const uint16_t* weight, const float* rstd,
                           const float* cos_table, const float* sin_table, const uint16_t* grad_y,
                           uint16_t* grad_x, int64_t rows, int64_t seq, int heads, int head_dim,
                           void* stream) {
  PLZ_REQUIRE(head_dim == HNR_D, "plz_head_norm_rope_bwd: head_dim %d is not supported (128 only)",
              head_dim);
  PLZ_REQUIRE(rows >= 0 && seq > 0 && heads > 0, "plz_head_norm_rope_bwd: need rows >= 0, seq > 0, heads > 0");
  if (rows == 0) return PLZ_OK;
  PLZ_REQUIRE(x && weight && rstd && cos_table && sin_table && grad_y && grad_x && a16(x) &&
                  a16(weight) && a16(cos_table) && a16(sin_table) && a16(grad_y) && a16(grad_x),
              "plz_head_norm_rope_bwd: operands must be non-null and 16-byte aligned");
  const int64_t n = rows * heads;
  hipLaunchKernelGGL(head_norm_rope_bwd_kernel, dim3((unsigned)((n + 15) / 16)), dim3(256), 0,
                     (hipStream_t)stream, x, weight, rstd, cos_table, sin_table, grad_y, grad_x,
                     n, seq, heads);
  return check_launch("plz_head_norm_rope_bwd");
}


int plz_add_rmsnorm_fwd(const uint16_t* x, const uint16_t* residual, const uint16_t* weight,
                        uint16_t* sum, uint16_t* y, float* rstd, int64_t rows, int64_t cols,
                        float eps, void* stream) {
  PLZ_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && cols <= 64 * 8 * kNormMaxChunks,
              "plz_add_rmsnorm_fwd: cols (%lld) must be a positive multiple of 8 up to 4096",
              (long long)cols);
  if (rows == 0) return PLZ_OK;
  PLZ_REQUIRE(x && residual && weight && sum && y && a16(x) && a16(residual) && a16(weight) &&
                  a16(sum) && a16(y),
              "plz_add_rmsnorm_fwd: operands must be non-null and 16-byte aligned");
  const NormShape sh = norm_shape(cols);
  const int64_t per_block = 4LL * (64 / sh.lpr);
  const dim3 grid((unsigned)((rows + per_block - 1) / per_block));
  const hipStream_t st = (hipStream_t)stream;
  if (sh.lpr == 16)
    hipLaunchKernelGGL((rmsnorm_fwd_kernel<16, 1, true>), grid, dim3(256), 0, st, x, weight, y,
                       rstd, rows, cols, eps, residual, sum);
  else if (sh.maxc == 1)
    hipLaunchKernelGGL((rmsnorm_fwd_kernel<64, 1, true>), grid, dim3(256), 0, st, x, weight, y,
                       rstd, rows, cols, eps, residual, sum);
  else
    hipLaunchKernelGGL((rmsnorm_fwd_kernel<64, kNormMaxChunks, true>), grid, dim3(256), 0, st, x,
                       weight, y, rstd, rows, cols, eps, residual, sum);
  return check_launch("plz_add_rmsnorm_fwd");
}

int plz_rmsnorm_bwd_add(const uint16_t* x, const uint16_t* weight, const float* rstd,
                        const uint16_t* grad_y, const uint16_t* grad_add, uint16_t* grad_x,
                        int64_t rows, int64_t cols, void* stream) {
  PLZ_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && cols <= 64 * 8 * kNormMaxChunks,
              "plz_rmsnorm_bwd_add: cols (%lld) must be a positive multiple of 8 up to 4096",
              (long long)cols);
  if (rows == 0) return PLZ_OK;
  PLZ_REQUIRE(x && weight && rstd && grad_y && grad_add && grad_x && a16(x) && a16(weight) &&
                  a16(grad_y) && a16(grad_add) && a16(grad_x),
              "plz_rmsnorm_bwd_add: operands must be non-null and 16-byte aligned");
  const int blocks = rmsnorm_bwd_blocks(rows, cols);
  const NormShape sh = norm_shape(cols);
  const hipStream_t st = (hipStream_t)stream;
  if (sh.lpr == 16)
    hipLaunchKernelGGL((rmsnorm_bwd_kernel<16, 1, 4, false, true>), dim3(blocks), dim3(256), 0, st,
                       x, weight, rstd, grad_y, grad_x, nullptr, rows, cols, grad_add);
  else if (sh.maxc == 1)
    hipLaunchKernelGGL((rmsnorm_bwd_kernel<64, 1, 4, false, true>), dim3(blocks), dim3(256), 0, st,
                       x, weight, rstd, grad_y, grad_x, nullptr, rows, cols, grad_add);
  else
    hipLaunchKernelGGL((rmsnorm_bwd_kernel<64, kNormMaxChunks, 1, false, true>), dim3(blocks),
                       dim3(256), 0, st, x, weight, rstd, grad_y, grad_x, nullptr, rows, cols,
                       grad_add);
  return check_launch("plz_rmsnorm_bwd_add");
}

}  // extern "C"
