/* palettize_hip.h -- C ABI of the MI355X (gfx950) LUT-linear library libpalettize_hip.so.
 *
 * Every entry point takes raw device pointers, plain sizes and a hipStream_t passed as
 * void*, returns PLZ_OK (0) or an error code, and never allocates device memory: outputs
 * and workspaces are owned by the caller (workspace sizes come from the *_workspace
 * queries). The last error message of the calling thread is returned by plz_last_error().
 * Work is enqueued on the given stream only; nothing synchronises the host.
 *
 * bf16 tensors travel as uint16_t bit patterns. A palettized weight W[N,K] (output rows
 * n, input columns k) is
 *   packed  int32 [N, K/16]   2-bit indices, 16 per word along K, index of column k at
 *                             bits 2*(k%16) (LSB first; same bytes as the reference's
 *                             .idx2 packing, palettize_core.py:31-42)
 *   palette fp32  [N, K/256, 4]  one 4-entry palette per row and per 256 columns
 * and W[n,k] = bf16(palette[n, k/256, idx[n,k]]) (round to nearest even), the flat
 * gather of qwen_model.py:97-102,185-186. The reference's own layout (palette group =
 * 256 output channels spanning all of K) is the special case
 * palette[n, g, :] = palette_ref[n/256, :] (expanded by the Python wrapper).
 * K must be a multiple of 256 and N a multiple of 8 unless stated otherwise.
 */
#ifndef PALETTIZE_HIP_H
#define PALETTIZE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PLZ_ABI_VERSION 18

/* status codes */
#define PLZ_OK 0
#define PLZ_EINVAL 1       /* bad shape, dtype, alignment or null pointer */
#define PLZ_EHIP 2         /* a HIP launch failed */
#define PLZ_EUNSUPPORTED 3 /* valid request this build does not implement */
#define PLZ_EWORKSPACE 4   /* workspace missing or smaller than the *_workspace query */

/* dtype codes */
#define PLZ_DT_BF16 0
#define PLZ_DT_FP16 1
#define PLZ_DT_FP32 2

/* soft forward weight modes (plz_soft_build_w) */
#define PLZ_W_SOFT 0       /* W = sum_c P_c pal_c                                        */
#define PLZ_W_HARD_NOISY 1 /* W = pal[argmax_c P_c], first max wins (fused_lut_kernel.cu:1998-2003) */
#define PLZ_W_HARD_PLAIN 2 /* W = pal[argmax_c logits_c], first max wins (triton_soft_forward.py:160-176) */

/* ---- errors / version ------------------------------------------------------------ */
const char* plz_last_error(void);
int plz_abi_version(void);

/* ---- index formats and dequantisation --------------------------------------------- */
/* idx uint8 [rows, cols] (values 0..3) <-> packed int32 [rows, cols/16]; cols % 16 == 0.
 * Replaces the reference's pack_idx2/unpack_idx2 (palettize_core.py:31-47,159-172) for the
 * device layout (packing along the row). */
int plz_pack_indices(const uint8_t* idx, int32_t* packed, int64_t rows, int64_t cols,
                     void* stream);
int plz_unpack_indices(const int32_t* packed, uint8_t* idx, int64_t rows, int64_t cols,
                       void* stream);
/* w bf16 [N, K] = dequantised weight. The gather of qwen_model.py:185-186. */
int plz_dequant(const int32_t* packed, const float* palette, uint16_t* w, int64_t N, int64_t K,
                void* stream);

/* ---- hard LUT linear ------------------------------------------------------------- */
/* y[M,N] = x[M,K] W^T (+ bias[N]) (+ lora_t[M,rank] lora_b[N,rank]^T).
 * lora_t already carries the LoRA scaling (see plz_lora_project); rank in {0,8,...,64}.
 * Replaces fused_lut_linear_fwd (fused_lut_linear_cuda.py:74-117) and its kernel
 * fused_lut_linear_fwd_tc_kernel (fused_lut_kernel.cu:309-518), plus the LoRA add of
 * QwenLoRA.forward (qwen_model.py:291-304). */
int plz_lut_linear_fwd(const uint16_t* x, const int32_t* packed, const float* palette,
                       const uint16_t* bias, const uint16_t* lora_t, const uint16_t* lora_b,
                       int rank, uint16_t* y, void* workspace, size_t workspace_bytes, int64_t M,
                       int64_t N, int64_t K, void* stream);
/* Optional workspace of the four one-pass GEMMs (lut fwd / bwd_x, dense fwd / bwd_x): when the
 * output tiles leave a last, partial wave on the GPU, those tiles are split over the
 * reduction and summed by a second kernel (fp32 partials in the workspace). NULL disables the
 * split; a smaller non-NULL workspace than the tail partials need returns PLZ_EWORKSPACE.
 * 0 = no split.
 * The two LUT GEMMs (plz_lut_linear_fwd, plz_lut_linear_bwd_x) have two schedules, chosen by
 * the workspace given: from M = 4096 rows their queries ask for room for a bf16 copy of W
 * (N*K*2 bytes, rounded up to 256) ahead of the tail partials, and with that much workspace
 * the call dequantises W into it and runs the dense GEMM on it (faster at these sizes than
 * rebuilding W tiles inside the GEMM's loop); with less (or NULL) it runs the one-pass LUT
 * GEMM, splitting its last wave when the workspace holds the tail partials
 * (plz_linear_fwd_dense_workspace / plz_linear_bwd_x_dense_workspace give that size). The two
 * schedules differ only in MFMA summation order (bf16 rounding of the output). */
size_t plz_lut_linear_fwd_workspace(int64_t M, int64_t N, int64_t K);

/* grad_x[M,K] = grad_y[M,N] W (+ lora_gt[M,rank] lora_a[rank,K]).
 * Replaces the grad_x half of fused_lut_linear_bwd (fused_lut_linear_cuda.py:119-150) and
 * fused_lut_linear_bwd_grad_x_tc_kernel (fused_lut_kernel.cu:551-720). Workspace and
 * schedules as for plz_lut_linear_fwd. */
int plz_lut_linear_bwd_x(const uint16_t* grad_y, const int32_t* packed, const float* palette,
                         const uint16_t* lora_gt, const uint16_t* lora_a, int rank,
                         uint16_t* grad_x, void* workspace, size_t workspace_bytes, int64_t M,
                         int64_t N, int64_t K, void* stream);
size_t plz_lut_linear_bwd_x_workspace(int64_t M, int64_t N, int64_t K);

/* grad_palette fp32 [N, K/256, 4]: grad_palette[n,g,c] = sum over k in group g with
 * idx[n,k] == c of (grad_y^T x)[n,k]. Deterministic (fixed-order two-stage reduction).
 * Replaces the grad_palette half of fused_lut_linear_bwd (fused_lut_linear_cuda.py:152-170)
 * and fused_lut_linear_bwd_grad_palette_kernel (fused_lut_kernel.cu:902-1123). */
size_t plz_lut_linear_bwd_palette_workspace(int64_t M, int64_t N, int64_t K);
int plz_lut_linear_bwd_palette(const uint16_t* x, const uint16_t* grad_y, const int32_t* packed,
                               float* grad_palette, void* workspace, size_t workspace_bytes,
                               int64_t M, int64_t N, int64_t K, void* stream);

/* grad_palette as plz_lut_linear_bwd_palette (bit for bit), plus both LoRA weight gradients
 * from the same dW tiles: grad_a [rank, K] = scale * lora_b^T dW and grad_b [N, rank] =
 * scale * dW lora_a^T with dW = grad_y^T x, lora_a [rank, K], lora_b [N, rank] bf16, rank a
 * multiple of 8 in [8, 32]; grads_dtype PLZ_DT_BF16 or PLZ_DT_FP32 for grad_a / grad_b.
 * These are the reference's LoRA weight gradients (autograd of QwenLoRA.forward,
 * qwen_model.py:291-304: grad_B = grad_y^T (x A) s, grad_A = x^T (grad_y B) s), computed
 * here in fp32 from dW without a further pass over x and grad_y (the separate route is
 * plz_lora_weight_grads on t and gt). Deterministic (fixed-order sums). The workspace holds
 * the grad_palette partials and the LoRA partials (query below; 16-byte aligned). */
size_t plz_lut_linear_bwd_palette_lora_workspace(int64_t M, int64_t N, int64_t K, int rank);
int plz_lut_linear_bwd_palette_lora(const uint16_t* x, const uint16_t* grad_y,
                                    const int32_t* packed, const uint16_t* lora_a,
                                    const uint16_t* lora_b, int rank, float scale,
                                    float* grad_palette, void* grad_a, void* grad_b,
                                    int grads_dtype, void* workspace, size_t workspace_bytes,
                                    int64_t M, int64_t N, int64_t K, void* stream);

/* No counterpart in the reference: plz_lut_linear_bwd_palette for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). It takes no workspace and allocates nothing: the split-M partials live in a
 * 32 MiB device array inside the library (one per GPU, held until the process ends), so
 * N * K may be at most 268,435,456 (N x K/128 x 16 bytes per split; larger weights get
 * PLZ_EINVAL). The split count is the workspace variant's, lowered where its partials would
 * not fit (then the fp32 sums run in another order). Every call on a GPU shares that GPU's
 * array: calls that overlap on one GPU (other streams, other threads) race and must be
 * serialised by the caller. */
int plz_lut_linear_bwd_palette_noalloc(const uint16_t* x, const uint16_t* grad_y,
                                       const int32_t* packed, float* grad_palette, int64_t M,
                                       int64_t N, int64_t K, void* stream);

/* grad_bias fp32 [N] = sum_m grad_y[m, n]. Replaces fused_lut_linear_bwd_grad_bias_kernel
 * (fused_lut_kernel.cu:1129-1147). Any N. */
int plz_bias_grad(const uint16_t* grad_y, float* grad_bias, int64_t M, int64_t N, void* stream);

/* ---- dense bf16 linear (soft path: W materialised by plz_soft_build_w) ---------------- */
/* y = x w^T (+bias) (+lora); w bf16 [N, K]. Replaces the torch.matmul(x, W) of
 * CUDAFusedLUTLinearSoft.forward (fused_lut_linear_cuda.py:912). K, N multiples of 8. */
int plz_linear_fwd_dense(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                         const uint16_t* lora_t, const uint16_t* lora_b, int rank, uint16_t* y,
                         void* workspace, size_t workspace_bytes, int64_t M, int64_t N, int64_t K,
                         void* stream);
/* plz_linear_fwd_dense with a residual: y = residual + (x w^T (+bias) (+lora)), the GEMM's
 * output rounded to bf16 and the sum rounded again, as the separate bf16 add after it.
 * residual bf16 [M, N] and y 16-byte aligned. Replaces the decoder layer's final residual add
 * `hidden_states = residual + hidden_states` after the MLP's down projection (HF
 * `modeling_qwen3.py` Qwen3DecoderLayer.forward, which the reference's layer runs via
 * qwen_model.py:590) with the down GEMM's epilogue. */
int plz_linear_fwd_dense_residual(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                  const uint16_t* lora_t, const uint16_t* lora_b, int rank,
                                  const uint16_t* residual, uint16_t* y, void* workspace,
                                  size_t workspace_bytes, int64_t M, int64_t N, int64_t K,
                                  void* stream);
size_t plz_linear_fwd_dense_workspace(int64_t M, int64_t N, int64_t K);
/* Gate and up projections with the SwiGLU in the epilogue: h [M, N] = silu(x Wg^T) * (x Wu^T)
 * as the HF Qwen3 MLP computes it in bf16 (transformers modeling_qwen3.py:70-83; the gate and
 * up outputs are rounded to bf16 first, as the unfused path does, and never stored).
 * w_gate_up bf16 [2N, K]: the rows of Wg and Wu interleaved in 128-row blocks (128 gate rows,
 * the 128 matching up rows, ...). N a multiple of 128, K of 8; no bias, no LoRA. No
 * counterpart in the reference, which runs the two nn.Linear and the activation apart. */
int plz_linear_fwd_dense_swiglu(const uint16_t* x, const uint16_t* w_gate_up, uint16_t* h,
                                int64_t M, int64_t N, int64_t K, void* stream);
/* A trained gate/up pair (one soft linear over the concatenated rows) with the SwiGLU in the
 * epilogue: y [M, 2F] = x w^T (+ lora_t lora_b^T), the pre-activations the SwiGLU backward
 * needs (skipped when y is null), and h [M, F] = silu(y[:, :F]) * y[:, F:] from the bf16 y.
 * w bf16 [2F, K] = [Wg; Wu] as stored (no interleaved copy: each output tile reads 128 gate
 * rows and the 128 matching up rows), lora_b [2F, rank]. Bit-equal to plz_linear_fwd_dense
 * without a workspace (no reduction split) followed by plz_swiglu_fwd_rows; this kernel never
 * splits the reduction. F a multiple of 128, K of 8, rank of 8 up to 64. No
 * counterpart in the reference: the HF Qwen3 MLP it trains runs gate_proj, up_proj and
 * act_fn(gate) * up apart (transformers models/qwen3/modeling_qwen3.py). */
int plz_linear_fwd_dense_swiglu_cat(const uint16_t* x, const uint16_t* w, const uint16_t* lora_t,
                                    const uint16_t* lora_b, int rank, uint16_t* y, uint16_t* h,
                                    int64_t M, int64_t F, int64_t K, void* stream);
/* grad_x = grad_y w (+lora). Replaces torch.matmul(grad_y, W.T)
 * (fused_lut_linear_cuda.py:944). */
int plz_linear_bwd_x_dense(const uint16_t* grad_y, const uint16_t* w, const uint16_t* lora_gt,
                           const uint16_t* lora_a, int rank, uint16_t* grad_x, void* workspace,
                           size_t workspace_bytes, int64_t M, int64_t N, int64_t K,
                           void* stream);
/* plz_linear_bwd_x_dense followed by the SwiGLU backward in its epilogue: with gate_up
 * [M, 2K] = [gate | up] the pre-activations of h = silu(gate) * up (K = the SwiGLU's width),
 * grad_h = grad_y w (+ lora) is rounded to bf16 and grad_gate_up [M, 2K] = [grad_gate | grad_up]
 * written from it, bit for bit plz_linear_bwd_x_dense then plz_swiglu_bwd_rows; grad_h itself
 * is not stored. Replaces the down projection's grad_x matmul and the autograd of HF Qwen3MLP's
 * act_fn(gate_proj(x)) * up_proj(x) (modeling_qwen3.py, via qwen_model.py:590) behind it. */
int plz_linear_bwd_x_dense_swiglu(const uint16_t* grad_y, const uint16_t* w,
                                  const uint16_t* lora_gt, const uint16_t* lora_a, int rank,
                                  const uint16_t* gate_up, uint16_t* grad_gate_up, void* workspace,
                                  size_t workspace_bytes, int64_t M, int64_t N, int64_t K,
                                  void* stream);
size_t plz_linear_bwd_x_dense_workspace(int64_t M, int64_t N, int64_t K);

/* ---- soft (Gumbel-softmax) path --------------------------------------------------- */
/* noise fp32 [n] = -log(-log(u)), u from Philox4x32-10 (Salmon et al., SC'11) keyed by
 * seed, counter = offset + element index / 4 (one 128-bit draw per 4 consecutive
 * elements), u = ((bits >> 9) + 0.5) * 2^-23, so 2^-24 <= u <= 1 - 2^-24 exactly in fp32
 * and the noise is always finite. Replaces the in-kernel LCG sampler of
 * fused_lut_kernel.cu:1245-1256 with a supplied-noise tensor. n % 4 == 0. */
int plz_gumbel_philox(float* noise, int64_t n, uint64_t seed, uint64_t offset, void* stream);
/* The reference's own sampler, bit-exact in its integer part: noise[n,k,c] =
 * gumbel_sample(seed, (k*N + n)*4 + c) of fused_lut_kernel.cu:1245-1256 and
 * triton_soft_forward.py:51-66, written in [N, K, 4] layout. */
int plz_gumbel_lcg(float* noise, uint32_t seed, int64_t N, int64_t K, void* stream);
/* The Triton sampler _gumbel_sample (triton_soft_forward.py:51-66), which the reference's
 * preferred soft path (TritonSoftLinear, triton_soft_forward.py:317-411) draws from: the same
 * statements in int32, where >> is an arithmetic shift, so it differs from plz_gumbel_lcg
 * wherever a shifted intermediate has bit 31 set. Same [N, K, 4] layout and index. */
int plz_gumbel_lcg_triton(float* noise, uint32_t seed, int64_t N, int64_t K, void* stream);

/* Batched soft P / W in the reference's own layouts. Replaces fused_compute_P_W_batched
 * (fused_lut_linear_cuda.py:513-607 and :1016-1077, kernel fused_lut_kernel.cu:2097-2158):
 *   logits  (4, K, N) fp16 planes      palette (G, 4) bf16, row o in group o / group_size
 *   p_aos   (K, N, 4) fp16 = softmax_c((logit_c + g_c) / tau)
 *   w       (K, N) bf16    = sum_c P_c pal_c (the soft weight, as the reference returns)
 * with g_c the CUDA LCG draw gumbel_sample(step_seed ^ (seed_offset * 0x9E3779B9),
 * (j*N + o)*4 + c) (fused_lut_kernel.cu:2129); seed_offset is the layer's position. */
typedef struct plz_pw_ref_desc {
  const uint16_t* logits;   /* (4, K, N) fp16 */
  const uint16_t* palette;  /* (G, 4) bf16 */
  uint16_t* p_aos;          /* (K, N, 4) fp16 */
  uint16_t* w;              /* (K, N) bf16 */
  int64_t K, N;
  int64_t block_begin;      /* filled by plz_pw_ref_plan */
  uint32_t seed_offset;     /* the layer's index in the batch */
  int32_t vec;              /* filled by plz_pw_ref_plan */
} plz_pw_ref_desc;
/* Checks n host descriptors (N % group_size == 0, 4*K*N < 2^32, pointers at least 2-byte
 * aligned, the palette 8-byte aligned), fills block_begin and vec, and returns the launch's
 * block count (or a negative status). */
int64_t plz_pw_ref_plan(plz_pw_ref_desc* descs, int n, int64_t group_size);
/* descs_device: a device copy of the planned descriptors. */
int plz_soft_pw_ref_batched(const plz_pw_ref_desc* descs_device, int n, int64_t total_blocks,
                            int64_t group_size, float tau, uint32_t step_seed, void* stream);

/* Builds the forward weight of the soft path from logits [N, K, 4] (bf16 or fp16),
 * noise fp32 [N, K, 4] and palette fp32 [N, K/256, 4]:
 *   P_c = softmax_c((logit_c + noise_c) / tau)
 *   w   bf16 [N, K]  per mode (PLZ_W_SOFT / PLZ_W_HARD_NOISY / PLZ_W_HARD_PLAIN)
 *   w_soft bf16 [N, K] = sum_c P_c pal_c (optional, may be null)
 *   p_out fp16 [N, K, 4] = P (optional, may be null; 16-byte aligned): what the reference's
 *         forward saves as P_aos for its backward (fused_lut_linear_cuda.py:903-905, 919);
 *         plz_soft_bwd_probs reads it
 * Replaces compute_P_W_hard_aos_kernel (fused_lut_kernel.cu:1946-2004) and
 * compute_P_W_ste_kernel (triton_soft_forward.py:83-181). */
int plz_soft_build_w(const uint16_t* logits, int logits_dtype, const float* noise,
                     const float* palette, float tau, int mode, uint16_t* w, uint16_t* w_soft,
                     uint16_t* p_out, int64_t N, int64_t K, void* stream);
/* The same with the noise drawn in the kernel: element (n, k, c) = the value
 * plz_gumbel_philox(seed, offset) stores there (Philox counter offset + n*K + k), so no noise
 * tensor is written or read. Replaces the in-kernel sampling of
 * compute_P_W_hard_aos_kernel (fused_lut_kernel.cu:1946-2004) with this build's Philox. */
int plz_soft_build_w_philox(const uint16_t* logits, int logits_dtype, uint64_t seed,
                            uint64_t offset, const float* palette, float tau, int mode,
                            uint16_t* w, uint16_t* w_soft, uint16_t* p_out, int64_t N, int64_t K,
                            void* stream);

/* Batched build W: the linears of a layer (or of several) in one launch, each with its own
 * logits, palette and outputs and either its own noise tensor or its own Philox key; the same
 * tau and mode for all. Replaces fused_compute_P_W_batched (fused_lut_kernel.cu:2071-2211,
 * fused_lut_linear_cuda.py:1016-1075), which draws each layer's noise in the kernel from the
 * step seed XOR a per-layer value (fused_lut_kernel.cu:2129): a descriptor whose noise is NULL
 * draws element (n, k, c) as plz_gumbel_philox(noise_seed, offset) would store it, Philox
 * counter offset + n*K + k with the launch's offset, so layers are decorrelated by key. */
typedef struct plz_build_w_desc {
  const uint16_t* logits;  /* [N, K, 4] bf16 or fp16 */
  const float* noise;      /* [N, K, 4] fp32, or NULL: Philox noise drawn in the kernel */
  const float* palette;    /* [N, K/256, 4] fp32 */
  uint16_t* w;             /* [N, K] bf16 */
  uint16_t* w_soft;        /* [N, K] bf16 or NULL */
  int64_t N, K;
  int32_t logits_dtype;    /* PLZ_DT_BF16 or PLZ_DT_FP16 */
  int32_t reserved;
  int64_t block_begin;     /* filled by plz_build_w_plan */
  uint64_t noise_seed;     /* Philox key of a descriptor without a noise tensor */
  uint64_t noise_counter;  /* its counter base: weight (n, k) draws at offset + noise_counter
                              + n*K + k (0 for the layout above) */
  uint16_t* p_out;         /* [N, K, 4] fp16 or NULL: P = softmax((logits + noise) / tau), what
                              the reference's forward saves as P_aos for its backward
                              (fused_lut_linear_cuda.py:903-905, 919, 957-959);
                              plz_soft_bwd_lora reads it */
} plz_build_w_desc;
/* Checks n host descriptors, fills block_begin and returns the launch's block count (or a
 * negative status). */
int64_t plz_build_w_plan(plz_build_w_desc* descs, int n);
/* descs_device: a device copy of the planned descriptors. */
int plz_soft_build_w_batched(const plz_build_w_desc* descs_device, int n, int64_t total_blocks,
                             float tau, int mode, void* stream);
/* plz_soft_build_w_batched with the Philox counter offset of the descriptors that draw their
 * noise in the kernel (plz_soft_build_w_batched uses offset 0). */
int plz_soft_build_w_batched_philox(const plz_build_w_desc* descs_device, int n,
                                    int64_t total_blocks, uint64_t noise_offset, float tau,
                                    int mode, void* stream);

/* Soft backward, fused in the epilogue of dW = grad_y^T x (dW never leaves the chip):
 *   grad_logits[n,k,c] = s * dW[n,k] P_c (pal_c - sum_d P_d pal_d)   (logits dtype)
 *   grad_palette[n,g,c] = sum_{k in g} dW[n,k] P_c                   (fp32)
 * with s = 1 (the reference, which omits 1/tau: fused_lut_kernel.cu:1914-1917,
 * triton_soft_backward.py:276-279) or s = 1/tau when scale_grad_by_inv_tau != 0.
 * Replaces soft_bwd_elementwise_aos_kernel (fused_lut_kernel.cu:1877-1924) together with
 * the grad_W matmul before it (fused_lut_linear_cuda.py:952). */
size_t plz_soft_bwd_workspace(int64_t M, int64_t N, int64_t K);
int plz_soft_bwd(const uint16_t* x, const uint16_t* grad_y, const uint16_t* logits,
                 int logits_dtype, const float* noise, const float* palette, float tau,
                 int scale_grad_by_inv_tau, uint16_t* grad_logits, float* grad_palette,
                 void* workspace, size_t workspace_bytes, int64_t M, int64_t N, int64_t K,
                 void* stream);
/* The same with the forward's Philox noise redrawn in the epilogue (see
 * plz_soft_build_w_philox); same workspace. */
int plz_soft_bwd_philox(const uint16_t* x, const uint16_t* grad_y, const uint16_t* logits,
                        int logits_dtype, uint64_t seed, uint64_t offset, const float* palette,
                        float tau, int scale_grad_by_inv_tau, uint16_t* grad_logits,
                        float* grad_palette, void* workspace, size_t workspace_bytes, int64_t M,
                        int64_t N, int64_t K, void* stream);
/* The soft backward from the forward's P (p_out of a build: fp16 [N, K, 4], 16-byte aligned)
 * instead of logits and noise, as the reference's backward reads its saved P_aos with grad_W
 * (fused_lut_linear_cuda.py:952-959, soft_bwd_elementwise_aos_kernel fused_lut_kernel.cu:
 * 1877-1924): grad_logits (grad_logits_dtype, PLZ_DT_BF16 or PLZ_DT_FP16) and grad_palette as
 * plz_soft_bwd with that P, pal_c - sum_d P_d pal_d formed as sum_d P_d (pal_c - pal_d) so that
 * the rounding of P does not cancel; same workspace as plz_soft_bwd. */
int plz_soft_bwd_probs(const uint16_t* x, const uint16_t* grad_y, const uint16_t* probs,
                       const float* palette, float tau, int scale_grad_by_inv_tau,
                       uint16_t* grad_logits, int grad_logits_dtype, float* grad_palette,
                       void* workspace, size_t workspace_bytes, int64_t M, int64_t N, int64_t K,
                       void* stream);
/* The soft backward (noise == NULL: the Philox noise of seed and offset, as
 * plz_soft_bwd_philox) plus both LoRA weight gradients from the same dW tiles, as
 * plz_lut_linear_bwd_palette_lora computes them for the hard path: grad_a [rank, K] =
 * scale * lora_b^T dW and grad_b [N, rank] = scale * dW lora_a^T, dW = grad_y^T x, rank a
 * multiple of 8 in [8, 32], grads_dtype PLZ_DT_BF16 or PLZ_DT_FP32. grad_logits and
 * grad_palette are those of plz_soft_bwd bit for bit. Replaces, for a soft PalettizedLinear
 * under QwenLoRA, the LoRA weight gradients of QwenLoRA.forward's autograd
 * (qwen_model.py:291-304) beside the soft backward's grad_W matmul
 * (fused_lut_linear_cuda.py:952). Deterministic; the workspace (query below, 16-byte aligned)
 * holds the soft backward's and the LoRA partials. grad_sq (optional, fp32 [N, K/128]): the
 * sum of squares of each run of 512 consecutive grad_logits values as stored (row n, k
 * 128 j .. 128 j + 127), what the gradient-norm clip of the optimizer step
 * (train_qwen.py:1303-1319) sums; plz_adamw_desc.grad_sq takes it in place of reading the
 * gradient again. probs (optional, fp16 [N, K, 4], 16-byte aligned): the forward's P as a
 * build with plz_build_w_desc.p_out wrote it; the epilogues then read P instead of drawing the
 * noise again and recomputing the softmax, as the reference's backward reads its saved P_aos
 * (fused_lut_linear_cuda.py:957-959), and noise, seed, offset and the logits' values go unused
 * (logits_dtype still sets grad_logits' type). */
size_t plz_soft_bwd_lora_workspace(int64_t M, int64_t N, int64_t K, int rank);
int plz_soft_bwd_lora(const uint16_t* x, const uint16_t* grad_y, const uint16_t* logits,
                      int logits_dtype, const float* noise, uint64_t seed, uint64_t offset,
                      const uint16_t* probs, const float* palette, float tau,
                      int scale_grad_by_inv_tau,
                      const uint16_t* lora_a, const uint16_t* lora_b, int rank, float scale,
                      uint16_t* grad_logits, float* grad_palette, void* grad_a, void* grad_b,
                      int grads_dtype, float* grad_sq, void* workspace, size_t workspace_bytes,
                      int64_t M, int64_t N, int64_t K, void* stream);

/* ---- LoRA (QwenLoRA, qwen_model.py:213-304): y += scale * (x A^T) B^T ------------------ */
/* t[M,rank] = scale * x[M,K] lora_a[rank,K]^T  (bf16). rank in {8,16,24,32}. */
int plz_lora_project(const uint16_t* x, const uint16_t* lora_a, float scale, uint16_t* t,
                     int64_t M, int64_t K, int rank, void* stream);
/* gt[M,rank] = scale * grad_y[M,N] lora_b[N,rank]  (bf16) */
int plz_lora_grad_t(const uint16_t* grad_y, const uint16_t* lora_b, float scale, uint16_t* gt,
                    int64_t M, int64_t N, int rank, void* stream);
/* grad_b[N,rank] = scale * grad_y^T t  and  grad_a[rank,K] = gt^T x.
 * With t from plz_lora_project (already scaled) and gt from plz_lora_grad_t, scale = 1
 * gives the gradients of y += s (x A^T) B^T. out_dtype PLZ_DT_BF16 or PLZ_DT_FP32. */
size_t plz_lora_weight_grads_workspace(int64_t M, int64_t N, int64_t K, int rank);
int plz_lora_weight_grads(const uint16_t* x, const uint16_t* grad_y, const uint16_t* t,
                          const uint16_t* gt, float scale, void* grad_a, void* grad_b,
                          int out_dtype, void* workspace, size_t workspace_bytes, int64_t M,
                          int64_t N, int64_t K, int rank, void* stream);

/* ---- decode GEMV (M <= 16), no counterpart in the reference ---------------------------- */
/* One palettized linear of a grouped launch. All pointers are device pointers. */
typedef struct plz_gemv_desc {
  const uint16_t* x;      /* [M, K] bf16 */
  const int32_t* packed;  /* [N, K/16] */
  const float* palette;   /* [N, K/256, 4] */
  uint16_t* y;            /* [M, N] bf16 */
  int64_t N, K;
  int64_t block_begin;    /* filled by plz_gemv_plan: first 128-row work item of this linear */
  int64_t cost_begin;     /* filled by plz_gemv_plan: sum of K over the items before it */
  const uint32_t* palette_items; /* decode layout (plz_gemv_pack_palettes): read instead of
                                    `palette` by decode-layout launches; may be NULL otherwise */
  const int32_t* packed_items;    /* decode layout (plz_gemv_pack_indices): read instead of
                                     `packed` by decode-layout launches; may be NULL otherwise */
} plz_gemv_desc;

/* y[M,N] = x[M,K] W^T for 1 <= M <= 16 (bandwidth-bound; one pass over the packed weights).
 * The reference would run fused_lut_linear_fwd_tc_kernel (fused_lut_kernel.cu:309-518) with
 * a 64-row tile at M = 1. */
int plz_lut_gemv(const uint16_t* x, const int32_t* packed, const float* palette, uint16_t* y,
                 int64_t M, int64_t N, int64_t K, void* stream);
/* Decode palette layout (one-time repack, e.g. at model load): each row's 4-entry palette per
 * 256-k group, rounded to bf16 as the GEMMs do, stored as the dequantiser's two lookup words
 * (low bytes of entries 0..3, then their high bytes), regrouped as [ceil(N/128)][K/256][128]
 * [lo, hi] (rows past N zero). A GEMV stage reads its 128 rows' tables as one contiguous 1 KB
 * block; 8 B per row and group instead of the fp32 palette's 16 B. */
size_t plz_gemv_palette_items_bytes(int64_t N, int64_t K);
int plz_gemv_pack_palettes(const float* palette, uint32_t* palette_items, int64_t N, int64_t K,
                           void* stream);
/* Decode index layout (one-time repack): the packed indices [N, K/16] regrouped per 128-row
 * item and 256-k stage into one contiguous 8 KB block each, in the order the GEMV's waves read
 * them, with the 2-bit fields of every word permuted so that the dequantiser produces natural k
 * order. Same bytes per weight (rows padded to a multiple of 128). */
size_t plz_gemv_packed_items_bytes(int64_t N, int64_t K);
int plz_gemv_pack_indices(const int32_t* packed, int32_t* packed_items, int64_t N, int64_t K,
                          void* stream);
/* plz_lut_gemv on weights in the two decode layouts (plz_gemv_pack_indices and
 * plz_gemv_pack_palettes). */
int plz_lut_gemv_decode(const uint16_t* x, const int32_t* packed_items,
                        const uint32_t* palette_items, uint16_t* y, int64_t M, int64_t N,
                        int64_t K, void* stream);
/* Weight layout of a grouped launch: PLZ_GEMV_NATIVE reads every descriptor's `packed` and
 * `palette`, PLZ_GEMV_DECODE its `packed_items` and `palette_items`. */
#define PLZ_GEMV_NATIVE 0
#define PLZ_GEMV_DECODE 1
/* Fills block_begin and cost_begin of n host descriptors for a launch in `layout` and returns
 * the total number of 128-row work items (or a negative status). A descriptor with N > 0
 * needs K > 0, and a non-empty one must hold the two arrays the layout streams (non-null):
 * a plan for the decode layout over a descriptor without decode arrays fails with
 * -PLZ_EINVAL. */
int64_t plz_gemv_plan(plz_gemv_desc* descs, int n, int M, int layout);
/* Runs n independent GEMVs (all with the same M) in one launch. descs_device is a copy of
 * the planned descriptors in device memory; total_blocks is plz_gemv_plan's result, and
 * `layout` must be the layout the table was planned for. */
int plz_lut_gemv_grouped(const plz_gemv_desc* descs_device, int n, int64_t total_blocks, int M,
                         int layout, void* stream);

/* Bit-plane decode (layout PLZ_GEMV_PLANES): the GEMV of plz_lut_gemv_decode computed as
 *   sum_k x_k w_k = p0 X + d1 S(b0) + d2 S(b1) + d3 S(b0 b1)   per row and 256-k group,
 * with b0, b1 the bits of each 2-bit index, S(f) = sum_k x_k f_k, X = sum_k x_k, d1 = p1 - p0,
 * d2 = p2 - p0, d3 = p3 - p2 - p1 + p0: the bit planes are FP4 operands of gfx950's scaled
 * FP8 x FP4 MFMA, cut from the packed words by masks, and x enters as two e4m3 pieces per
 * element with a power-of-two scale per token and group (x = 2^s (x1 + x2), exact except
 * where x2 underflows e4m3: an error below 2^-17 of the group's largest |x|). Same outputs as
 * the decode kernel up to that and fp32 summation order. Replaces, like plz_lut_gemv, the
 * reference's 64-row-tile forward at M = 1 (fused_lut_kernel.cu:309-518).
 * Indices: a one-time repack (same size as plz_gemv_packed_items_bytes) in which lane
 * l = 16g + r of a 16-row block holds four words of its row: nibble i of word j holds the index
 * of k = 32g + 8j + i (bits 4i, 4i+1) and that of k = 128 + 32g + 8j + i (bits 4i+2, 4i+3).
 * Palettes: the decode lookup words (plz_gemv_pack_palettes).
 * The workspace (plz_gemv_planes_workspace) receives the x pieces of every linear and group,
 * written by a small kernel launched first on the same stream. */
#define PLZ_GEMV_PLANES 2
int plz_gemv_pack_planes(const int32_t* packed, int32_t* planes_items, int64_t N, int64_t K,
                         void* stream);
/* bytes of workspace for n linears whose largest K is max_K, at M tokens */
size_t plz_gemv_planes_workspace(int n, int64_t max_K, int M);
int plz_lut_gemv_planes(const uint16_t* x, const int32_t* planes_items,
                        const uint32_t* palette_items, uint16_t* y, int64_t M, int64_t N, int64_t K,
                        void* workspace, size_t workspace_bytes, void* stream);
/* descs_device: a table planned by plz_gemv_plan(..., PLZ_GEMV_PLANES), whose packed_items
 * hold plz_gemv_pack_planes layouts; max_K: the largest K in the table (the workspace is laid
 * out by it). */
int plz_lut_gemv_grouped_planes(const plz_gemv_desc* descs_device, int n, int64_t total_blocks,
                                int M, int64_t max_K, void* workspace, size_t workspace_bytes,
                                void* stream);

/* ---- on-disk format converters ---------------------------------------------------------
 * .idx2 = the (K, N) index matrix (W^T) flattened row-major, 4 indices per byte, LSB first
 * (palettize_core.py:31-47 pack_idx2 / pack_indices_transposed_2bit; read back by
 * palettize_core.py:159-172 unpack_idx2 / load_indices); .lut_scalar = fp16 palettes (G, 4),
 * one per 256 output rows (palettize_pytorch.py:150-159 write_lut_scalar). */
/* .idx2 bytes (device) -> native packed [N, K/16]. N % 4 == 0, K % 16 == 0. Replaces
 * load_indices (palettize_core.py:167-172) followed by pack_indices on the device. */
int plz_idx2_to_packed(const uint8_t* idx2, int32_t* packed, int64_t N, int64_t K, void* stream);
/* native packed [N, K/16] -> .idx2 bytes (the save path, train_qwen.py:826-835 with frozen
 * indices; palettize_core.py:45-47). */
int plz_packed_to_idx2(const int32_t* packed, uint8_t* idx2, int64_t N, int64_t K, void* stream);
/* argmax over the 4 index-logit planes (4, K, N) (fp16 or bf16, logits_dtype) written as .idx2
 * bytes; the first maximal plane wins, as torch.argmax (train_qwen.py:826-829 save_state). */
int plz_logits_argmax_idx2(const uint16_t* logits, int logits_dtype, uint8_t* idx2, int64_t N,
                           int64_t K, void* stream);
/* .lut_scalar fp16 (ceil(N/group_size), 4) -> native fp32 palette [N, K/256, 4]
 * (qwen_model.py:97-102: row n uses palette n / group_size for every k). */
int plz_lut_to_palette(const uint16_t* lut, float* palette, int64_t N, int64_t K, int group_size,
                       void* stream);

/* ---- fused optimizer step ---------------------------------------------------------------
 * Replaces FP32MasterOptimizer.step (train_qwen.py:154-221: bf16 grads -> fp32 masters,
 * torch.optim.AdamW, copy back), the two-tier clip_grad_norm_ (:1303-1319) and the logits
 * clamp to +-5 tau (:1343-1348) by two streaming passes over all parameters. */
typedef struct plz_adamw_desc {
  void* param;           /* bf16 or fp32 parameter */
  const void* grad;      /* its gradient, same dtype */
  float* master;         /* fp32 master (required for bf16 params; NULL: param is the master) */
  float* exp_avg;        /* fp32 first moment */
  float* exp_avg_sq;     /* fp32 second moment */
  int64_t n;             /* elements */
  int32_t dtype;         /* PLZ_DT_BF16 or PLZ_DT_FP32 */
  int32_t clip_group;    /* 0 or 1: which clip_grad_norm_ group the gradient belongs to */
  float lr, clamp_lo, clamp_hi, reserved;  /* clamp_lo/hi = -/+inf for no clamp */
  int64_t block_begin;   /* filled by plz_adamw_plan */
  const float* grad_sq;  /* optional: the gradient's sum of squares per 512 consecutive
                            elements (n % 512 == 0), e.g. plz_soft_bwd_lora's grad_sq; the
                            clip norm then reads these n / 512 floats instead of the gradient */
} plz_adamw_desc;
/* Checks n host descriptors, fills block_begin, returns the block count (or -status). */
int64_t plz_adamw_plan(plz_adamw_desc* descs, int n);
size_t plz_adamw_workspace(int64_t total_blocks);
/* One step (step = 1, 2, ...): gradients clipped per group to max_norm0 / max_norm1 (<= 0: no
 * clipping), AdamW(beta1, beta2, eps, weight_decay) on the masters, clamp, params rewritten.
 * norms_out (device, optional): the two groups' unclipped gradient norms. */
int plz_adamw_step(const plz_adamw_desc* descs_device, int n, int64_t total_blocks,
                   float max_norm0, float max_norm1, double beta1, double beta2, float eps,
                   float weight_decay, int64_t step, float* norms_out, void* workspace,
                   size_t workspace_bytes, void* stream);
/* The step above that also builds the next forward's soft weights from the logits it has just
 * updated (the train loop's optimizer step followed by the next forward's
 * fused_compute_P_W_batched, fused_lut_linear_cuda.py:1016-1075): builds[i] (n entries, w NULL
 * for none) rebuilds descriptor i's bf16 [N, K, 4] logits (builds[i].logits == param) as
 * plz_soft_build_w_batched_philox(noise_offset, tau, mode) would from the stored values, bit
 * for bit. No counterpart in the reference, which runs the two passes apart; here the build's
 * arithmetic rides on the update's memory-bound pass. The descriptors with a build come after
 * all others; the others (the palettes the builds read) are updated by a first launch, the
 * built ones by a second. plz_adamw_plan_build plans both tables and returns the block count,
 * with *split_block = the first built block. */
int64_t plz_adamw_plan_build(plz_adamw_desc* descs, const plz_build_w_desc* builds, int n,
                             int64_t* split_block);
int plz_adamw_step_build(const plz_adamw_desc* descs_device, const plz_build_w_desc* builds_device,
                         int n, int64_t total_blocks, int64_t split_block, uint64_t noise_offset,
                         float tau, int mode, float max_norm0, float max_norm1, double beta1,
                         double beta2, float eps, float weight_decay, int64_t step,
                         float* norms_out, void* workspace, size_t workspace_bytes,
                         void* stream);

/* ---- fused RMSNorm and SwiGLU ------------------------------------------------------------
 * The reference runs the HF Qwen3 modules unfused (Qwen3RMSNorm and Qwen3MLP, transformers
 * models/qwen3/modeling_qwen3.py:50-83, used by the decoder layers that qwen_model.py wraps). */
/* y = bf16(weight * bf16(x * rsqrt(mean(x^2) + eps))) per row, fp32 statistics; rstd fp32
 * [rows] saved for the backward. cols % 8 == 0. */
int plz_rmsnorm_fwd(const uint16_t* x, const uint16_t* weight, uint16_t* y, float* rstd,
                    int64_t rows, int64_t cols, float eps, void* stream);
/* grad_x bf16 [rows, cols]; grad_weight fp32 [cols] (deterministic two-stage reduction). */
size_t plz_rmsnorm_bwd_workspace(int64_t rows, int64_t cols);
int plz_rmsnorm_bwd(const uint16_t* x, const uint16_t* weight, const float* rstd,
                    const uint16_t* grad_y, uint16_t* grad_x, float* grad_weight,
                    void* workspace, size_t workspace_bytes, int64_t rows, int64_t cols,
                    void* stream);
/* A residual add followed by RMSNorm, as the HF Qwen3 decoder layer runs them
 * (hidden = residual + attn_out; post_attention_layernorm(hidden)): sum = bf16(x + residual),
 * written, and y, rstd of plz_rmsnorm_fwd on sum, bit for bit. */
int plz_add_rmsnorm_fwd(const uint16_t* x, const uint16_t* residual, const uint16_t* weight,
                        uint16_t* sum, uint16_t* y, float* rstd, int64_t rows, int64_t cols,
                        float eps, void* stream);
/* grad_x = bf16(plz_rmsnorm_bwd's grad_x) + grad_add (the gradient that reaches the norm's
 * input along the residual stream), without the weight gradient (frozen norm weights). */
int plz_rmsnorm_bwd_add(const uint16_t* x, const uint16_t* weight, const float* rstd,
                        const uint16_t* grad_y, const uint16_t* grad_add, uint16_t* grad_x,
                        int64_t rows, int64_t cols, void* stream);
/* h = silu(gate) * up, elementwise over n elements (n % 8 == 0). */
int plz_swiglu_fwd(const uint16_t* gate, const uint16_t* up, uint16_t* h, int64_t n,
                   void* stream);
int plz_swiglu_bwd(const uint16_t* gate, const uint16_t* up, const uint16_t* grad_h,
                   uint16_t* grad_gate, uint16_t* grad_up, int64_t n, void* stream);
/* The same on rows x F elements with row pitches in elements (multiples of 8, >= F): gate and up
 * may sit side by side in one [rows, 2F] tensor (a fused gate/up projection: up = gate + F,
 * ld_in = 2F), and the gradients likewise. Replaces the HF Qwen3 MLP's act_fn(gate) * up
 * (transformers models/qwen3/modeling_qwen3.py) and its autograd, as plz_swiglu_fwd/bwd do. */
int plz_swiglu_fwd_rows(const uint16_t* gate, const uint16_t* up, int64_t ld_in, uint16_t* h,
                        int64_t ld_h, int64_t rows, int64_t F, void* stream);
int plz_swiglu_bwd_rows(const uint16_t* gate, const uint16_t* up, int64_t ld_in,
                        const uint16_t* grad_h, int64_t ld_h, uint16_t* grad_gate,
                        uint16_t* grad_up, int64_t ld_g, int64_t rows, int64_t F, void* stream);

/* ---- layer step around the linears -------------------------------------------------- */
/* Rotary position embedding, HF Qwen3 rotate_half convention, fp32 math on bf16:
 * y[row, head, j] = x[j] cos[pos, j] + rotate_half(x)[j] sin[pos, j], pos = row % seq;
 * x, y bf16 [rows, heads, head_dim] (head_dim % 16 == 0), cos/sin fp32 [seq, head_dim].
 * Replaces the torch expression of apply_rotary_pos_emb that the reference's HF Qwen layers
 * run (transformers models/qwen3/modeling_qwen3.py, called through qwen_model.py:590).
 * plz_rope_bwd is its transpose (grad_y -> grad_x). Bit-exact with the torch expression. */
int plz_rope_fwd(const uint16_t* x, const float* cos_table, const float* sin_table, uint16_t* y,
                 int64_t rows, int64_t seq, int heads, int head_dim, void* stream);
int plz_rope_bwd(const uint16_t* grad_y, const float* cos_table, const float* sin_table,
                 uint16_t* grad_x, int64_t rows, int64_t seq, int heads, int head_dim,
                 void* stream);
/* Per-head RMSNorm followed by the rotary embedding, in one pass: for each of the rows x heads
 * vectors of 128 (x bf16 [rows, heads, 128], rows = tokens, pos = row % seq),
 * y = rope(rmsnorm(x, weight, eps)) with the values of plz_rmsnorm_fwd then plz_rope_fwd (bit for
 * bit), rstd fp32 [rows * heads] (optional) as plz_rmsnorm_fwd saves it. Replaces the q_norm /
 * k_norm + apply_rotary_pos_emb pair of the HF Qwen3 attention the reference's layers run
 * (transformers models/qwen3/modeling_qwen3.py, through qwen_model.py:590). */
int plz_head_norm_rope_fwd(const uint16_t* x, const uint16_t* weight, const float* cos_table,
                           const float* sin_table, uint16_t* y, float* rstd, int64_t rows,
                           int64_t seq, int heads, int head_dim, float eps, void* stream);
/* Its backward for grad_x (plz_rope_bwd then plz_rmsnorm_bwd, bit for bit); the norm weight's
 * gradient is not formed, for callers whose norm weights are frozen. */
int plz_head_norm_rope_bwd(const uint16_t* x, const uint16_t* weight, const float* rstd,
                           const float* cos_table, const float* sin_table, const uint16_t* grad_y,
                           uint16_t* grad_x, int64_t rows, int64_t seq, int heads, int head_dim,
                           void* stream);
/* Causal grouped-query attention forward (flash-style): q, o bf16 [batch, seq, heads, 128],
 * k, v bf16 [batch, seq, kv_heads, 128], heads % kv_heads == 0, seq % 128 == 0;
 * o = softmax(q k^T * scale, causal) v per head (kv head = head / (heads / kv_heads)),
 * lse fp32 [batch, heads, seq] = log-sum-exp of the scaled scores. Replaces
 * torch scaled_dot_product_attention(is_causal=True) of the HF Qwen3 attention the reference
 * runs (transformers modeling_qwen3.py via qwen_model.py:590). head_dim != 128:
 * PLZ_EUNSUPPORTED. */
int plz_attn_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, float* lse,
                 int batch, int seq, int heads, int kv_heads, int head_dim, float scale,
                 void* stream);
/* Backward of plz_attn_fwd (the autograd of the same sdpa call): grad_q bf16 [batch, seq, heads,
 * 128], grad_k, grad_v bf16 [batch, seq, kv_heads, 128] (summed over the heads sharing a kv
 * head), from q, k, v, the forward's o and lse, and grad_o. Deterministic (no atomics); the
 * workspace (fp32 [2][batch, heads, seq]: rowsum(grad_o * o), then -lse log2 e) comes from the
 * query. */
size_t plz_attn_bwd_workspace(int batch, int seq, int heads);
int plz_attn_bwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* o,
                 const uint16_t* grad_o, const float* lse, uint16_t* grad_q, uint16_t* grad_k,
                 uint16_t* grad_v, void* workspace, size_t workspace_bytes, int batch, int seq,
                 int heads, int kv_heads, int head_dim, float scale, void* stream);
/* Distillation loss of train_qwen.py:229-249 (compute_loss, '1-cos+norm_mse'):
 * loss = wc mean_rows(1 - cos(s_r, t_r)) + wm mean((s-t)^2) / max(mean(t^2), 1e-6), weights
 * normalised to sum 1, cos = s.t / (max(|s|, eps) max(|t|, eps)) with each norm clamped on its
 * own as torch's F.cosine_similarity does; student/teacher bf16 [rows, dim]. out4 (device
 * fp32 [4]) receives {loss, l_cos, t_var, l_mse}; the workspace (per-row sums) is reused by the backward, which
 * writes grad_student = grad_loss[0] * d loss / d student (bf16). */
size_t plz_distill_loss_workspace(int64_t rows);
int plz_distill_loss_fwd(const uint16_t* student, const uint16_t* teacher, float w_cos,
                         float w_mse, float eps, float* out4, void* workspace,
                         size_t workspace_bytes, int64_t rows, int64_t dim, void* stream);
int plz_distill_loss_bwd(const uint16_t* student, const uint16_t* teacher, const float* out4,
                         const float* grad_loss, float w_cos, float w_mse, float eps,
                         uint16_t* grad_student, const void* workspace, size_t workspace_bytes,
                         int64_t rows, int64_t dim, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PALETTIZE_HIP_H */
