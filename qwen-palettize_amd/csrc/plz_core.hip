// Error state, index packing and the dequantisation kernel.
//
// The dequant kernel is the bit-exact "palette lookup" contract of the hard path:
//   W[n,k] = bf16(palette[n, k/256, idx[n,k]])
// restating the flat gather W = flat_palette[group_id*4 + idx] of
// qwen_model.py:97-102 and :185-186 (group_id = n*(K/256) + k/256 in this layout).
#include "plz_common.h"
#include "palettize_hip.h"
#include <stdarg.h>
#include <stdio.h>

namespace plz {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return PLZ_EHIP;
  }
  return PLZ_OK;
}

// Zero fill by a kernel rather than hipMemsetAsync: a memset node recorded into a captured
// HIP graph is not reliable on replay, and callers may capture any entry point. Used only for
// the degenerate shapes (an empty reduction) whose outputs are all zero; bytes is even.
__global__ void zero_kernel(uint16_t* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

int reserve_lds(const void* fn, size_t bytes, uint64_t& done, const char* what) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  const uint64_t bit = dev >= 0 && dev < 64 ? (uint64_t)1 << dev : 0;
  if (bit != 0 && (done & bit) != 0) return PLZ_OK;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e != hipSuccess) {
    set_error("%s: cannot reserve %zu bytes of LDS: %s", what, bytes, hipGetErrorString(e));
    return PLZ_EHIP;
  }
  done |= bit;
  return PLZ_OK;
}

void zero_async(void* p, size_t bytes, hipStream_t stream) {
  const int64_t n = (int64_t)(bytes / 2);
  if (n > 0)
    hipLaunchKernelGGL(zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       reinterpret_cast<uint16_t*>(p), n);
}

// ---- canonical packing: idx[r, c] (uint8 0..3) -> packed[r, c/16] -------------
__global__ void pack_kernel(const uint8_t* __restrict__ idx, int32_t* __restrict__ packed,
                            int64_t n_words) {
  int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (w >= n_words) return;
  const uint4 v = *reinterpret_cast<const uint4*>(idx + w * 16);
  uint32_t bytes[4] = {v.x, v.y, v.z, v.w};
  uint32_t q = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int j = 0; j < 4; ++j) q |= ((bytes[b] >> (8 * j)) & 3u) << (2 * (4 * b + j));
  packed[w] = (int32_t)q;
}

__global__ void unpack_kernel(const int32_t* __restrict__ packed, uint8_t* __restrict__ idx,
                              int64_t n_words) {
  int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (w >= n_words) return;
  uint32_t q = (uint32_t)packed[w];
  uint32_t out[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    uint32_t d = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) d |= ((q >> (2 * (4 * b + j))) & 3u) << (8 * j);
    out[b] = d;
  }
  *reinterpret_cast<uint4*>(idx + w * 16) = make_uint4(out[0], out[1], out[2], out[3]);
}

// One thread per packed word: 16 weights of one row.
__global__ void dequant_kernel(const int32_t* __restrict__ packed, const float* __restrict__ pal,
                               uint16_t* __restrict__ w, int64_t N, int64_t K) {
  const int64_t wpr = K / kIdxPerWord;
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N * wpr) return;
  int64_t n = t / wpr, kw = t % wpr;
  int64_t kg = (kw * kIdxPerWord) / kPalGroup;
  const float4 p = *reinterpret_cast<const float4*>(pal + (n * (K / kPalGroup) + kg) * 4);
  PalLut lut = make_lut(p.x, p.y, p.z, p.w);
  uint32_t o[8];
  dequant16((uint32_t)packed[t], lut, o);
  uint4* dst = reinterpret_cast<uint4*>(w + n * K + kw * kIdxPerWord);
  dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
  dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
}

}  // namespace plz

using namespace plz;

extern "C" {

const char* plz_last_error(void) { return g_err; }

int plz_abi_version(void) { return PLZ_ABI_VERSION; }

int plz_pack_indices(const uint8_t* idx, int32_t* packed, int64_t rows, int64_t cols,
                     void* stream) {
  PLZ_REQUIRE(rows >= 0 && cols >= 0, "plz_pack_indices: negative shape");
  PLZ_REQUIRE(cols % 16 == 0, "plz_pack_indices: cols (%lld) must be a multiple of 16",
              (long long)cols);
  int64_t n = rows * (cols / 16);
  if (n == 0) return PLZ_OK;
  PLZ_REQUIRE(idx && packed, "plz_pack_indices: null pointer");
  PLZ_REQUIRE(((uintptr_t)idx & 15) == 0, "plz_pack_indices: idx must be 16-byte aligned");
  int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, idx,
                     packed, n);
  return check_launch("plz_pack_indices");
}

int plz_unpack_indices(const int32_t* packed, uint8_t* idx, int64_t rows, int64_t cols,
                       void* stream) {
  PLZ_REQUIRE(rows >= 0 && cols >= 0, "plz_unpack_indices: negative shape");
  PLZ_REQUIRE(cols % 16 == 0, "plz_unpack_indices: cols (%lld) must be a multiple of 16",
              (long long)cols);
  int64_t n = rows * (cols / 16);
  if (n == 0) return PLZ_OK;
  PLZ_REQUIRE(idx && packed, "plz_unpack_indices: null pointer");
  PLZ_REQUIRE(((uintptr_t)idx & 15) == 0, "plz_unpack_indices: idx must be 16-byte aligned");
  int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(unpack_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     packed, idx, n);
  return check_launch("plz_unpack_indices");
}

int plz_dequant(const int32_t* packed, const float* palette, uint16_t* w, int64_t N, int64_t K,
                void* stream) {
  PLZ_REQUIRE(N >= 0 && K >= 0, "plz_dequant: negative shape");
  PLZ_REQUIRE(K % 256 == 0, "plz_dequant: K (%lld) must be a multiple of 256", (long long)K);
  int64_t n = N * (K / 16);
  if (n == 0) return PLZ_OK;
  PLZ_REQUIRE(packed && palette && w, "plz_dequant: null pointer");
  PLZ_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)palette & 15) == 0,
              "plz_dequant: w and palette must be 16-byte aligned");
  int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     packed, palette, w, N, K);
  return check_launch("plz_dequant");
}

}  // extern "C"
