// Layer-step kernels around the palettized linears: rotary position embedding and the
// distillation loss of the decoder-layer training step.
//
// RoPE follows HF Qwen3's apply_rotary_pos_emb with rotate_half (transformers
// models/qwen3/modeling_qwen3.py), computed in fp32 on bf16 tensors:
//   y = (x.float() * cos + rotate_half(x.float()) * sin).to(bf16),
//   rotate_half(x)[j] = -x[j + D/2] (j < D/2),  x[j - D/2] (j >= D/2)
// with cos/sin fp32 [S, D] indexed by the token's position (row % S). The backward is the
// transpose: grad_x[j] = g[j] cos[j] + (j < D/2 ? g[j + D/2] sin[j + D/2]
//                                                : -g[j - D/2] sin[j - D/2]).
// Products and sums are rounded separately (floating-point contraction is off in the kernel, so
// no fused multiply-add), as the elementwise torch expression does: both directions match it
// bit for bit.
//
// The loss is train_qwen.py:229-249 compute_loss ('1-cos+norm_mse', weights normalised):
//   l_cos = mean_rows(1 - cos(s_r, t_r)),  cos = s.t / (max(|s|, eps) max(|t|, eps))
//   l_mse = mean((s - t)^2) / max(mean(t^2), 1e-6),  loss = wc l_cos + wm l_mse
// over the student and teacher outputs s, t bf16 [rows, D], in fp32. loss_rows_kernel makes one
// pass over s and t for the per-row sums, loss_final_kernel reduces them in a fixed order, and
// loss_bwd_kernel writes grad_s (bf16) in a second pass from the same per-row sums.
#include "plz_common.h"

namespace plz {
namespace lyr {

__device__ __forceinline__ void unpack8(uint4 v, float (&f)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ uint4 pack8(const float (&f)[8]) {
  return make_uint4(f2bf(f[0]) | (f2bf(f[1]) << 16), f2bf(f[2]) | (f2bf(f[3]) << 16),
                    f2bf(f[4]) | (f2bf(f[5]) << 16), f2bf(f[6]) | (f2bf(f[7]) << 16));
}
__device__ __forceinline__ void load8f(const float* p, float (&f)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
  f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}

// One thread per (row, head, 8 consecutive j of the first half) and their partners j + D/2.
template <bool BWD>
__global__ void rope_kernel(const uint16_t* __restrict__ x, const float* __restrict__ cosv,
                            const float* __restrict__ sinv, uint16_t* __restrict__ y,
                            int64_t rows, int64_t S, int heads, int D) {
#pragma clang fp contract(off)  // products and sums rounded one by one, as torch does
  const int h = D / 2, cpr = h / 8;  // 8-wide chunks per half
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= rows * heads * cpr) return;
  const int c8 = (int)(t % cpr);
  const int64_t rh = t / cpr;  // row * heads + head
  const int64_t pos = (rh / heads) % S;
  const int64_t base = rh * D + 8 * c8;
  float lo[8], hi[8], cl[8], ch[8], sl[8], sh[8], ol[8], oh[8];
  unpack8(*reinterpret_cast<const uint4*>(x + base), lo);
  unpack8(*reinterpret_cast<const uint4*>(x + base + h), hi);
  const float* cp = cosv + pos * D + 8 * c8;
  const float* sp = sinv + pos * D + 8 * c8;
  load8f(cp, cl);
  load8f(cp + h, ch);
  load8f(sp, sl);
  load8f(sp + h, sh);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    // plain operators under the pragma: helper functions from headers would carry their own
    // contraction flags into the inlined code
    if (!BWD) {
      const float a = lo[j] * cl[j], b = hi[j] * sl[j], c = hi[j] * ch[j], d = lo[j] * sh[j];
      ol[j] = a - b;
      oh[j] = c + d;
    } else {
      const float a = lo[j] * cl[j], b = hi[j] * sh[j], c = hi[j] * ch[j], d = lo[j] * sl[j];
      ol[j] = a + b;
      oh[j] = c - d;
    }
  }
  *reinterpret_cast<uint4*>(y + base) = pack8(ol);
  *reinterpret_cast<uint4*>(y + base + h) = pack8(oh);
}

// ---- distillation loss ------------------------------------------------------------------
// Per-row sums {s.t, s.s, t.t, (s-t).(s-t)}: one wave per row, lanes stride over 8-wide chunks.
__global__ __launch_bounds__(256) void loss_rows_kernel(const uint16_t* __restrict__ s,
                                                        const uint16_t* __restrict__ t,
                                                        float4* __restrict__ stats, int64_t rows,
                                                        int D) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // wave-uniform
  if (row >= rows) return;
  const uint4* sp = reinterpret_cast<const uint4*>(s + row * D);
  const uint4* tp = reinterpret_cast<const uint4*>(t + row * D);
  float st = 0.f, ss = 0.f, tt = 0.f, dd = 0.f;
  for (int c = lane; c < D / 8; c += 64) {
    float a[8], b[8];
    unpack8(sp[c], a);
    unpack8(tp[c], b);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      st += a[j] * b[j];
      ss += a[j] * a[j];
      tt += b[j] * b[j];
      const float d = a[j] - b[j];
      dd += d * d;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    st += __shfl_xor(st, off);
    ss += __shfl_xor(ss, off);
    tt += __shfl_xor(tt, off);
    dd += __shfl_xor(dd, off);
  }
  if (lane == 0) stats[row] = make_float4(st, ss, tt, dd);
}

// One workgroup of 1024 threads: sum over rows of (1 - cos), t.t and (s-t).(s-t) in a fixed
// order (thread-strided partial sums, then a tree in LDS). out = {loss, l_cos, t_var, l_mse}.
__global__ __launch_bounds__(1024) void loss_final_kernel(const float4* __restrict__ stats,
                                                          int64_t rows, int D, float wc, float wm,
                                                          float eps, float* __restrict__ out) {
  __shared__ float red[3][1024];
  float c = 0.f, tt = 0.f, dd = 0.f;
  for (int64_t r = threadIdx.x; r < rows; r += 1024) {
    const float4 v = stats[r];
    c += 1.f - v.x / (fmaxf(sqrtf(v.y), eps) * fmaxf(sqrtf(v.z), eps));
    tt += v.z;
    dd += v.w;
  }
  red[0][threadIdx.x] = c;
  red[1][threadIdx.x] = tt;
  red[2][threadIdx.x] = dd;
  __syncthreads();
  for (int w = 512; w >= 1; w >>= 1) {
    if ((int)threadIdx.x < w) {
#pragma unroll
      for (int k = 0; k < 3; ++k) red[k][threadIdx.x] += red[k][threadIdx.x + w];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const float n = (float)rows * (float)D;
    const float l_cos = red[0][0] / (float)rows;
    const float t_var = fmaxf(red[1][0] / n, 1e-6f);
    const float l_mse = red[2][0] / n / t_var;
    out[0] = wc * l_cos + wm * l_mse;
    out[1] = l_cos;
    out[2] = t_var;
    out[3] = l_mse;
  }
}

// grad_s = go * [ -wc/T * d cos_r/ds  +  wm * 2 (s - t) / (T D t_var) ].
// cos_r = s.t / (max(|s|, eps) max(|t|, eps)), each norm clamped on its own; the clamp passes
// no gradient and the norm's own gradient s / |s| is kept even where the clamp is active (the
// in-place no-grad clamp of torch's cosine_similarity, which train_qwen.py:234 calls):
// d cos_r/ds = t / (ns' nt') - (s.t) s / (ns'^2 nt' |s|), ns' = max(|s|, eps), zero at s = 0.
__global__ __launch_bounds__(256) void loss_bwd_kernel(const uint16_t* __restrict__ s,
                                                       const uint16_t* __restrict__ t,
                                                       const float4* __restrict__ stats,
                                                       const float* __restrict__ scal,
                                                       const float* __restrict__ grad_loss,
                                                       uint16_t* __restrict__ gs, int64_t rows,
                                                       int D, float wc, float wm, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float4 v = stats[row];
  const float go = grad_loss[0], t_var = scal[2];
  const float T = (float)rows;
  const float ns = sqrtf(v.y), nsc = fmaxf(ns, eps), ntc = fmaxf(sqrtf(v.z), eps);
  // d cos/ds = ca * t + cb * s
  const float ca = 1.f / (nsc * ntc);
  const float cb = ns > 0.f ? -v.x / (nsc * nsc * ntc * ns) : 0.f;
  const float kc = -go * wc / T;
  const float km = go * wm * 2.f / (T * (float)D * t_var);
  const float a = kc * ca - km, b = kc * cb + km;  // grad = a t + b s
  const uint4* sp = reinterpret_cast<const uint4*>(s + row * D);
  const uint4* tp = reinterpret_cast<const uint4*>(t + row * D);
  uint4* gp = reinterpret_cast<uint4*>(gs + row * D);
  for (int c = lane; c < D / 8; c += 64) {
    float x[8], y[8], g[8];
    unpack8(sp[c], x);
    unpack8(tp[c], y);
#pragma unroll
    for (int j = 0; j < 8; ++j) g[j] = a * y[j] + b * x[j];
    gp[c] = pack8(g);
  }
}

static bool a16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace lyr
}  // namespace plz

using namespace plz;
using namespace plz::lyr;

extern "C" {

static int rope(bool bwd, const uint16_t* x, const float* cosv, const float* sinv, uint16_t* y,
                int64_t rows, int64_t seq, int heads, int head_dim, void* stream,
                const char* what) {
  PLZ_REQUIRE(rows >= 0 && seq > 0 && heads > 0 && head_dim > 0 && head_dim % 16 == 0,
              "%s: need rows >= 0, seq > 0, heads > 0 and head_dim a multiple of 16", what);
  if (rows == 0) return PLZ_OK;
  PLZ_REQUIRE(x && cosv && sinv && y && a16(x) && a16(cosv) && a16(sinv) && a16(y),
              "%s: operands must be non-null and 16-byte aligned", what);
  const int64_t n = rows * heads * (head_dim / 16);
  const unsigned blocks = (unsigned)((n + 255) / 256);
  if (bwd)
    hipLaunchKernelGGL(rope_kernel<true>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, x,
                       cosv, sinv, y, rows, seq, heads, head_dim);
  else
    hipLaunchKernelGGL(rope_kernel<false>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, x,
                       cosv, sinv, y, rows, seq, heads, head_dim);
  return check_launch(what);
}

int plz_rope_fwd(const uint16_t* x, const float* cos_table, const float* sin_table, uint16_t* y,
                 int64_t rows, int64_t seq, int heads, int head_dim, void* stream) {
  return rope(false, x, cos_table, sin_table, y, rows, seq, heads, head_dim, stream,
              "plz_rope_fwd");
}

int plz_rope_bwd(const uint16_t* grad_y, const float* cos_table, const float* sin_table,
                 uint16_t* grad_x, int64_t rows, int64_t seq, int heads, int head_dim,
                 void* stream) {
  return rope(true, grad_y, cos_table, sin_table, grad_x, rows, seq, heads, head_dim, stream,
              "plz_rope_bwd");
}

size_t plz_distill_loss_workspace(int64_t rows) { return rows > 0 ? (size_t)rows * 16 : 0; }

int plz_distill_loss_fwd(const uint16_t* student, const uint16_t* teacher, float w_cos,
                         float w_mse, float eps, float* out4, void* workspace,
                         size_t workspace_bytes, int64_t rows, int64_t dim, void* stream) {
  PLZ_REQUIRE(rows > 0 && dim > 0 && dim % 8 == 0,
              "plz_distill_loss_fwd: need rows > 0 and dim a positive multiple of 8");
  PLZ_REQUIRE(w_cos + w_mse > 0.f && eps > 0.f,
              "plz_distill_loss_fwd: weights must sum to a positive value and eps be positive");
  PLZ_REQUIRE(student && teacher && out4 && a16(student) && a16(teacher),
              "plz_distill_loss_fwd: operands must be non-null and 16-byte aligned");
  if (!workspace || workspace_bytes < plz_distill_loss_workspace(rows) || !a16(workspace)) {
    set_error("plz_distill_loss_fwd: workspace of %zu bytes (16-byte aligned) needed",
              plz_distill_loss_workspace(rows));
    return PLZ_EWORKSPACE;
  }
  const float tot = w_cos + w_mse;
  float4* stats = reinterpret_cast<float4*>(workspace);
  hipLaunchKernelGGL(loss_rows_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream, student, teacher, stats, rows, (int)dim);
  int rc = check_launch("plz_distill_loss_fwd");
  if (rc) return rc;
  hipLaunchKernelGGL(loss_final_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, stats, rows,
                     (int)dim, w_cos / tot, w_mse / tot, eps, out4);
  return check_launch("plz_distill_loss_fwd/final");
}

int plz_distill_loss_bwd(const uint16_t* student, const uint16_t* teacher, const float* out4,
                         const float* grad_loss, float w_cos, float w_mse, float eps,
                         uint16_t* grad_student, const void* workspace, size_t workspace_bytes,
                         int64_t rows, int64_t dim, void* stream) {
  PLZ_REQUIRE(rows > 0 && dim > 0 && dim % 8 == 0,
              "plz_distill_loss_bwd: need rows > 0 and dim a positive multiple of 8");
  PLZ_REQUIRE(w_cos + w_mse > 0.f && eps > 0.f,
              "plz_distill_loss_bwd: weights must sum to a positive value and eps be positive");
  PLZ_REQUIRE(student && teacher && out4 && grad_loss && grad_student && a16(student) &&
                  a16(teacher) && a16(grad_student),
              "plz_distill_loss_bwd: operands must be non-null and 16-byte aligned");
  if (!workspace || workspace_bytes < plz_distill_loss_workspace(rows) || !a16(workspace)) {
    set_error("plz_distill_loss_bwd: the forward's workspace of %zu bytes is needed",
              plz_distill_loss_workspace(rows));
    return PLZ_EWORKSPACE;
  }
  const float tot = w_cos + w_mse;
  hipLaunchKernelGGL(loss_bwd_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream, student, teacher,
                     reinterpret_cast<const float4*>(workspace), out4, grad_loss, grad_student,
                     rows, (int)dim, w_cos / tot, w_mse / tot, eps);
  return check_launch("plz_distill_loss_bwd");
}

}  // extern "C"
