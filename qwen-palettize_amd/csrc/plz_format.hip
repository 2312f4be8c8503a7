// On-disk format converters for the palettized weights (HBM-bound byte work).
//
//   .idx2        2-bit indices of W^T: the (K, N) index matrix flattened row-major, 4 per byte,
//                LSB first (palettize_core.py:31-47 pack_idx2 / pack_indices_transposed_2bit,
//                :159-172 unpack_idx2 / load_indices; train_qwen.py:826-835 save_state)
//   .lut_scalar  fp16 palettes (G, 4), one per 256 output rows (palettize_pytorch.py:150-159)
//
// and this library's native layouts: packed int32 [N, K/16] (16 indices of a row per word,
// LSB first along K) and fp32 palettes [N, K/256, 4].
//
//   idx2_to_packed_kernel    (K, N) 2-bit  -> [N, K/16]: one thread per 4 rows x 1 word; it
//                            reads the 16 bytes of its 16 k at byte column n0/4 and writes 4
//                            words (consecutive threads walk K, so the writes of a row coalesce)
//   packed_to_idx2_kernel    [N, K/16] -> (K, N): one thread per output byte (4 rows at one k)
//   logits_argmax_idx2_kernel  index logits (4, K, N) fp16/bf16 -> (K, N) argmax as .idx2 bytes;
//                            the first maximal plane wins (torch.argmax, train_qwen.py:827)
//   lut_to_palette_kernel    (G, 4) fp16 -> [N, K/256, 4] fp32 (qwen_model.py:97-102 gathers
//                            flat_palette[(n / group_size) * 4 + idx] for every k)
#include "plz_common.h"
#include "palettize_hip.h"

namespace plz {
namespace fmt {

__global__ void idx2_to_packed_kernel(const uint8_t* __restrict__ idx2, uint32_t* __restrict__ packed,
                                      int64_t N, int64_t K) {
  const int64_t W = K / 16, t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (N / 4) * W) return;
  const int64_t w = t % W, n4 = t / W;  // word w of rows 4*n4 .. 4*n4+3
  uint32_t out[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t b = idx2[(16 * w + i) * (N / 4) + n4];  // (k, 4*n4 .. 4*n4+3)
#pragma unroll
    for (int r = 0; r < 4; ++r) out[r] |= ((b >> (2 * r)) & 3u) << (2 * i);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) packed[(4 * n4 + r) * W + w] = out[r];
}

__global__ void packed_to_idx2_kernel(const uint32_t* __restrict__ packed, uint8_t* __restrict__ idx2,
                                      int64_t N, int64_t K) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // byte (k, n4)
  if (t >= K * (N / 4)) return;
  const int64_t k = t / (N / 4), n4 = t % (N / 4), W = K / 16;
  uint32_t b = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) b |= ((packed[(4 * n4 + r) * W + k / 16] >> (2 * (k % 16))) & 3u) << (2 * r);
  idx2[t] = (uint8_t)b;
}

__device__ __forceinline__ float logit_at(const uint16_t* p, int64_t i, int f16) {
  return f16 ? h2f(p[i]) : bf2f(p[i]);
}
__global__ void logits_argmax_idx2_kernel(const uint16_t* __restrict__ logits, int f16,
                                          uint8_t* __restrict__ idx2, int64_t N, int64_t K) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // byte (k, n4)
  const int64_t plane = K * N;
  if (t >= plane / 4) return;
  uint32_t b = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t e = 4 * t + r;  // element (k, n) = k * N + n
    float best = logit_at(logits, e, f16);
    uint32_t arg = 0;
#pragma unroll
    for (int c = 1; c < 4; ++c) {
      const float v = logit_at(logits, c * plane + e, f16);
      if (v > best) {  // strict: the first maximal plane wins
        best = v;
        arg = (uint32_t)c;
      }
    }
    b |= arg << (2 * r);
  }
  idx2[t] = (uint8_t)b;
}

__global__ void lut_to_palette_kernel(const uint16_t* __restrict__ lut, float4* __restrict__ palette,
                                      int64_t N, int64_t KG, int group_size) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // (n, kg)
  if (t >= N * KG) return;
  const int64_t g = (t / KG) / group_size;
  palette[t] = make_float4(h2f(lut[4 * g]), h2f(lut[4 * g + 1]), h2f(lut[4 * g + 2]),
                           h2f(lut[4 * g + 3]));
}

static unsigned blocks(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace fmt
}  // namespace plz

using namespace plz;
using namespace plz::fmt;

extern "C" {

int plz_idx2_to_packed(const uint8_t* idx2, int32_t* packed, int64_t N, int64_t K, void* stream) {
  PLZ_REQUIRE(N >= 0 && K >= 0 && N % 4 == 0 && K % 16 == 0,
              "plz_idx2_to_packed: need N %% 4 == 0 and K %% 16 == 0 (N=%lld, K=%lld)",
              (long long)N, (long long)K);
  if (N == 0 || K == 0) return PLZ_OK;
  PLZ_REQUIRE(idx2 && packed, "plz_idx2_to_packed: null pointer");
  hipLaunchKernelGGL(idx2_to_packed_kernel, dim3(blocks((N / 4) * (K / 16))), dim3(256), 0,
                     (hipStream_t)stream, idx2, reinterpret_cast<uint32_t*>(packed), N, K);
  return check_launch("plz_idx2_to_packed");
}

int plz_packed_to_idx2(const int32_t* packed, uint8_t* idx2, int64_t N, int64_t K, void* stream) {
  PLZ_REQUIRE(N >= 0 && K >= 0 && N % 4 == 0 && K % 16 == 0,
              "plz_packed_to_idx2: need N %% 4 == 0 and K %% 16 == 0 (N=%lld, K=%lld)",
              (long long)N, (long long)K);
  if (N == 0 || K == 0) return PLZ_OK;
  PLZ_REQUIRE(idx2 && packed, "plz_packed_to_idx2: null pointer");
  hipLaunchKernelGGL(packed_to_idx2_kernel, dim3(blocks(K * (N / 4))), dim3(256), 0,
                     (hipStream_t)stream, reinterpret_cast<const uint32_t*>(packed), idx2, N, K);
  return check_launch("plz_packed_to_idx2");
}

int plz_logits_argmax_idx2(const uint16_t* logits, int logits_dtype, uint8_t* idx2, int64_t N,
                           int64_t K, void* stream) {
  PLZ_REQUIRE(N >= 0 && K >= 0 && N % 4 == 0,
              "plz_logits_argmax_idx2: need N %% 4 == 0 (N=%lld)", (long long)N);
  PLZ_REQUIRE(logits_dtype == PLZ_DT_FP16 || logits_dtype == PLZ_DT_BF16,
              "plz_logits_argmax_idx2: logits dtype must be fp16 or bf16");
  if (N == 0 || K == 0) return PLZ_OK;
  PLZ_REQUIRE(logits && idx2, "plz_logits_argmax_idx2: null pointer");
  hipLaunchKernelGGL(logits_argmax_idx2_kernel, dim3(blocks(K * N / 4)), dim3(256), 0,
                     (hipStream_t)stream, logits, (int)(logits_dtype == PLZ_DT_FP16), idx2, N, K);
  return check_launch("plz_logits_argmax_idx2");
}

int plz_lut_to_palette(const uint16_t* lut, float* palette, int64_t N, int64_t K, int group_size,
                       void* stream) {
  PLZ_REQUIRE(N >= 0 && K >= 0 && K % 256 == 0 && group_size > 0,
              "plz_lut_to_palette: need K %% 256 == 0 and group_size > 0");
  if (N == 0 || K == 0) return PLZ_OK;
  PLZ_REQUIRE(lut && palette && ((uintptr_t)palette & 15) == 0,
              "plz_lut_to_palette: null or misaligned pointer");
  const int64_t KG = K / 256;
  hipLaunchKernelGGL(lut_to_palette_kernel, dim3(blocks(N * KG)), dim3(256), 0, (hipStream_t)stream,
                     lut, reinterpret_cast<float4*>(palette), N, KG, group_size);
  return check_launch("plz_lut_to_palette");
}

}  // extern "C"
