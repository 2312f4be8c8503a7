// Rank-r adapter products of QwenLoRA (qwen_model.py:291-304): y += s (x A^T) B^T.
//
//   plz_lora_project        t  = s x A^T          [M, r]   reduction over K (contiguous in x)
//   plz_lora_grad_t         gt = s grad_y B       [M, r]   reduction over N (contiguous in grad_y)
//   plz_lora_weight_grads   grad_A = gt^T x       [r, K]   reduction over M (strided)
//                           grad_B = s grad_y^T t [N, r]
//
// All four stream one M x L activation (x or grad_y) and touch a rank-r operand that stays in
// L2, so they are HBM-bound: the work per activation element is r <= 32 MACs. Two kernels:
//
// rows_ring_kernel  (t, gt): a workgroup owns 64 rows of the activation and streams them
//   through a 3-slot LDS ring of 256-element stages (whole 512-byte row segments per copy);
//   its 8 waves take one 32-wide 16x16x32 k-step of each stage and meet in LDS at the end.
//   lora_a [r, L] is staged in the same row layout, lora_b [L, r] as its contiguous block.
// cols_kernel  (grad_A, grad_B): the reduction index m is the activation's row, so fragments
//   need a transpose. 32 x 256 activation tiles go global->LDS (buffer_load ... lds, 4-stage
//   ring of 20 KB stages, two workgroups per CU) and are read with ds_read_b64_tr_b16, which
//   hands each lane 4 consecutive rows of one column. Split over M (one split length for both
//   problems, enough splits to fill every CU); reduce_kernel sums the split partials in a
//   fixed order. Both weight gradients share one cols_kernel launch and one reduce_kernel
//   launch.
#include "plz_common.h"
#include "palettize_hip.h"

namespace plz {
namespace lora {

typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
typedef __attribute__((address_space(3))) u32x4 lds_w4;
typedef __attribute__((address_space(3))) uint16_t lds_u16;

// workgroup barrier once this wave's LDS accesses are done (its global->LDS copies are waited
// for separately, by wait_vmcnt)
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xF | (3 << 14) | (7 << 4));  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// wait until at most N vector-memory operations of this wave are outstanding
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ bf16x8 as_frag(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// ---------------------------------------------------------------------------------------
// rows_ring_kernel: out[M, r] = scale * X[M, L] Bop[L, r]
//   BOP_T: Bop(l, j) = bop[j * L + l]  (lora_a, [r, L]);  else Bop(l, j) = bop[l * r + j]
//   RG = 16-column groups (r <= 16 * RG)
// The activation is staged through LDS. A workgroup owns
// 64 rows; a stage is their next 256 reduction elements (32 KB) plus the matching slice of
// Bop, copied global -> LDS by buffer_load ... lds into a 3-slot ring two stages ahead. Every
// copy instruction moves 1 KB of whole 512-byte row segments, so the stream reads whole cache
// lines in order instead of 16 rows x 64 B per instruction (an 84 MB probe of the two
// patterns: 15 against 18-19 us). The 8 waves split each stage's 256 elements (32 each: one
// 16x16x32 k-step per row group).
//   X stage:  row m (512 B) holds 32 chunks of 16 B, logical chunk c at c ^ (m & 15): the 16
//             rows of a fragment read land on 16 distinct 16-byte bank groups.
//   Bop (BOP_T, lora_a [r, L]): rows j of the same layout.
//   Bop (else, lora_b [L, r]): the stage's contiguous [256][r] block as it is in memory.
// ---------------------------------------------------------------------------------------
constexpr int RR_ROWS = 64;                       // activation rows per workgroup
constexpr int RR_KC = 256;                        // reduction elements per stage
constexpr int RR_NS = 3;                          // ring slots (copies two stages ahead)
constexpr int RR_XBYTES = RR_ROWS * RR_KC * 2;    // 32 KB
constexpr int RR_XI = RR_XBYTES / (512 * 16);     // X copies per thread per stage (4)
template <int RG>
constexpr int rr_stage_bytes() { return RR_XBYTES + RG * 8192; }  // + Bop: RG x 8 KB

template <bool BOP_T, int RG>
__global__ __launch_bounds__(512) void rows_ring_kernel(const uint16_t* __restrict__ X,
                                                        const uint16_t* __restrict__ bop,
                                                        uint16_t* __restrict__ out, float scale,
                                                        int64_t M, int L, int r) {
  extern __shared__ uint4 smem[];
  lds_u8* lds = (lds_u8*)smem;
  constexpr int STAGE = rr_stage_bytes<RG>();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rr = lane & 15, q = lane >> 4;
  const int64_t m0 = (int64_t)blockIdx.x * RR_ROWS;
  const int rows = (int)min((int64_t)RR_ROWS, M - m0);
  const int nst = (L + RR_KC - 1) / RR_KC;
  // rows past the end of X, and reduction indices past L, read as zero (range check or kBufOob)
  const BufRsrc xr = make_rsrc(X + m0 * L, (uint32_t)rows * (uint32_t)L * 2u);
  const BufRsrc br = make_rsrc(bop, (uint32_t)r * (uint32_t)L * 2u);

  // Copies of stage s into slot ss; stages past the last one copy nothing (every lane still
  // issues the same count, so one vmcnt serves every stage).
  auto issue = [&](int s, lds_u8* ss) {
    const bool live = s < nst;
    const int k0 = RR_KC * s;
#pragma unroll
    for (int it = 0; it < RR_XI; ++it) {
      const int p = (wave * RR_XI + it) * 64 + lane;  // physical chunk: row p / 32
      const int m = p >> 5, k = k0 + 8 * ((p & 31) ^ (m & 15));
      const uint32_t off = live && k < L ? ((uint32_t)m * (uint32_t)L + (uint32_t)k) * 2u : kBufOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_u8*)(ss + (wave * RR_XI + it) * 1024), 16,
                                               off, 0, 0, 0);
    }
#pragma unroll
    for (int it = 0; it < RG; ++it) {
      const int p = (wave * RG + it) * 64 + lane;
      uint32_t off = kBufOob;
      if constexpr (BOP_T) {
        const int j = p >> 5, k = k0 + 8 * ((p & 31) ^ (j & 15));
        if (live && j < r && k < L) off = ((uint32_t)j * (uint32_t)L + (uint32_t)k) * 2u;
      } else {  // 16-byte chunk p of the contiguous [256][r] block (past L: out of range)
        if (live && 8 * p < RR_KC * r) off = ((uint32_t)k0 * (uint32_t)r + 8u * p) * 2u;
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          br, (lds_u8*)(ss + RR_XBYTES + (wave * RG + it) * 1024), 16, off, 0, 0, 0);
    }
  };

  f32x4 acc[4][RG];
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int cg = 0; cg < RG; ++cg) acc[g][cg] = f32x4{0.f, 0.f, 0.f, 0.f};
  // lane (rr, q) of wave w: logical chunk 4w + q (reduction elements 32w + 8q .. +7 of the stage)
  const int c = 4 * wave + q;
  const int xoff = rr * 512 + ((c ^ rr) << 4);  // row rr of a group; (16g + rr) & 15 == rr
  // the copies of stage s + RR_NS - 1 go to slot ws before the MFMAs read slot xs (distinct
  // slots: __restrict__ keeps the compiler from waiting on the new copies first)
  auto step = [&](int s, const lds_u8* __restrict__ xs, lds_u8* __restrict__ ws) {
    issue(s + RR_NS - 1, ws);
    bf16x8 a[4], b[RG];
#pragma unroll
    for (int g = 0; g < 4; ++g)
      a[g] = __builtin_bit_cast(bf16x8, *(const lds_w4*)(xs + g * 16 * 512 + xoff));
    const lds_u8* bs = xs + RR_XBYTES;
#pragma unroll
    for (int cg = 0; cg < RG; ++cg) {
      if constexpr (BOP_T) {
        b[cg] = __builtin_bit_cast(bf16x8, *(const lds_w4*)(bs + cg * 16 * 512 + xoff));
      } else {  // Bop(k, j) at (k r + j): 8 consecutive k of column j = 16 cg + rr
        const int j = 16 * cg + rr;
        uint32_t w[4] = {0u, 0u, 0u, 0u};
        if (j < r) {
          const lds_u16* bp = reinterpret_cast<const lds_u16*>(bs) + 8 * c * r + j;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            w[e] = (uint32_t)bp[(2 * e) * r] | ((uint32_t)bp[(2 * e + 1) * r] << 16);
        }
        b[cg] = __builtin_bit_cast(bf16x8, u32x4{w[0], w[1], w[2], w[3]});
      }
    }
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int cg = 0; cg < RG; ++cg) acc[g][cg] = mfma16(a[g], b[cg], acc[g][cg]);
  };
#pragma unroll
  for (int s = 0; s < RR_NS - 1; ++s) issue(s, lds + s * STAGE);
  for (int s = 0; s < nst; ++s) {
    wait_vmcnt<(RR_XI + RG) * (RR_NS - 2)>();  // this lane's copies of stage s have landed
    lds_barrier();                               // everyone's have; slot (s-1) % RR_NS is free
    step(s, lds + (s % RR_NS) * STAGE, lds + ((s + RR_NS - 1) % RR_NS) * STAGE);
  }
  __builtin_amdgcn_s_waitcnt(0);  // drain the trailing (empty) copies
  lds_barrier();                  // the ring is free: the cross-wave sums reuse it

  // C fragment of block (g, cg): rows 16 g + 4 q + e, column 16 cg + rr; summed over the 8
  // waves in wave order
  constexpr int RS = RG * 16 + 1;
  float* red = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int cg = 0; cg < RG; ++cg)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        red[(wave * RR_ROWS + 16 * g + 4 * q + e) * RS + 16 * cg + rr] = acc[g][cg][e];
  __syncthreads();
  for (int idx = threadIdx.x; idx < rows * r; idx += 512) {
    const int row = idx / r, j = idx - row * r;
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < 8; ++w) sum += red[(w * RR_ROWS + row) * RS + j];
    out[(m0 + row) * r + j] = (uint16_t)f2bf(scale * sum);
  }
}

// ---------------------------------------------------------------------------------------
// cols_kernel: partial[z](l, j) = scale * sum_{m in split z} X[m, l] T[m, j]
//   X [M, L] and T [M, r] row-major. Workgroup: 256 columns l (4 waves x 64) x one M split.
// ---------------------------------------------------------------------------------------
#ifndef PLZ_CL_BM
#define PLZ_CL_BM 32
#endif
#ifndef PLZ_CL_NS
#define PLZ_CL_NS 4
#endif
#ifndef PLZ_CL_MINST
#define PLZ_CL_MINST 16
#endif
constexpr int CL_L = 256;
constexpr int CL_BM = PLZ_CL_BM;                 // rows per stage
constexpr int CL_NS = PLZ_CL_NS;                 // LDS ring depth
constexpr int CL_XBYTES = CL_BM * CL_L * 2;      // 16 KB
constexpr int CL_TBYTES = 4096;                  // one 1 KB copy per wave (<= 64 rows x 32 ranks x 2 B)
constexpr int CL_STAGE = CL_XBYTES + CL_TBYTES;
constexpr int CL_LDS = CL_NS * CL_STAGE;         // 80 KB
constexpr int CL_XI = CL_XBYTES / (256 * 16);    // X copies per thread per stage (4)
constexpr int CL_LOADS = CL_XI + 1;              // copies per thread per stage: 4 + 1

// X tile layout: row m (512 B) holds 32 chunks of 16 B; chunk c sits at c ^ xsw(m). Rows
// m..m+3 and m+8..m+11 (what one half-wave of a transposing read touches) land their two
// chunks on 8 distinct bank pairs, so the fragment reads are conflict-free.
__device__ __forceinline__ int xsw(int m) { return 2 * (m & 3) + 8 * ((m >> 3) & 1); }


// One workgroup = one (problem, column tile, M split); problem 0 is grad_B, problem 1 grad_A,
// so both weight gradients run in one launch.
struct ColProb {
  const uint16_t* X;  // [M, L]
  const uint16_t* T;  // [M, r]
  float* partial;     // [Z, L, r]
  float scale;
  int L, tiles;
  int transpose;      // partials (and output) [r, L] instead of [L, r]
  int64_t split;      // rows per M split (a multiple of CL_BM)
};
struct ColsArgs {
  ColProb p[2];
  int nwg0;  // workgroups of problem 0
  int64_t M;
  int r;
};

template <int RG>
__global__ __launch_bounds__(256) void cols_kernel(const ColsArgs args) {
  extern __shared__ uint4 smem[];
  lds_u8* lds = (lds_u8*)smem;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool second = (int)blockIdx.x >= args.nwg0;
  const ColProb& pb = second ? args.p[1] : args.p[0];
  const int bid = (int)blockIdx.x - (second ? args.nwg0 : 0);
  const uint16_t* __restrict__ X = pb.X;
  const uint16_t* __restrict__ T = pb.T;
  const int L = pb.L, r = args.r, zi = bid / pb.tiles;
  const int64_t M = args.M, split = pb.split;
  const int lb = (bid % pb.tiles) * CL_L;
  const int64_t mb = (int64_t)zi * split;
  const int64_t me = min(M, mb + split);
  const int rows = me > mb ? (int)(me - mb) : 0;
  const int nst = (rows + CL_BM - 1) / CL_BM;
  // rows past the split fall outside both descriptors' ranges and read as zero
  const BufRsrc xr = make_rsrc(X + mb * L, (uint32_t)rows * (uint32_t)L * 2u);
  const BufRsrc tr = make_rsrc(T + mb * r, (uint32_t)rows * (uint32_t)r * 2u);

  // Copies of stage s into ring slot s % CL_NS: X by CL_XI instructions per lane (instruction
  // it of wave w fills LDS bytes [(CL_XI w + it) KB, +1 KB) = rows 2(CL_XI w + it), +1), T by
  // one (the 2 RG CL_BM chunks of T land in the first slots; the other lanes write unread
  // duplicates so that every lane issues the same count).
  auto issue = [&](int s, lds_u8* xs) {  // xs: ring slot s % CL_NS
    const bool live = s < nst;
#pragma unroll
    for (int it = 0; it < CL_XI; ++it) {
      const int p = (wave * CL_XI + it) * 64 + lane;  // physical chunk
      const int m = p >> 5, gc = (p & 31) ^ xsw(m);
      const int l = lb + 8 * gc;
      const uint32_t off =
          live && l < L ? ((uint32_t)(CL_BM * s + m) * (uint32_t)L + (uint32_t)l) * 2u : kBufOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_u8*)(xs + (wave * CL_XI + it) * 1024), 16, off,
                                               0, 0, 0);
    }
    const int p = threadIdx.x % (RG * 2 * CL_BM);  // T chunk: row p / (2 RG), 8 ranks (p % (2 RG))
    const int m = p / (2 * RG), c = p % (2 * RG);
    const uint32_t off = live && 8 * c < r ? ((uint32_t)(CL_BM * s + m) * (uint32_t)r + 8u * c) * 2u
                                           : kBufOob;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(tr, (lds_u8*)(xs + CL_XBYTES + wave * 1024), 16, off,
                                             0, 0, 0);
  };

  f32x4 acc[4][RG];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int cg = 0; cg < RG; ++cg) acc[i][cg] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int i16 = lane & 15, g = lane >> 4;
  // One stage: the copies of stage s + CL_NS - 1 into slot ws, then the MFMAs on slot xs. The
  // two slots are distinct, and saying so (__restrict__) keeps the compiler from waiting for
  // the copies just issued before the first read of xs.
  auto step = [&](int s, const lds_u8* __restrict__ xs, lds_u8* __restrict__ ws) {
    issue(s + CL_NS - 1, ws);
    const lds_u8* ts = xs + CL_XBYTES;
#pragma unroll
    for (int ks = 0; ks < CL_BM / 32; ++ks) {
      // lane (i16, g) points at rows 32ks + 8g + i16/4 (+4) and 4 consecutive columns; the
      // transposing read returns column i16 of the 16-wide block at 4 consecutive rows
      const int m1 = 32 * ks + 8 * g + (i16 >> 2), m2 = m1 + 4;
      bf16x8 a[4], b[RG];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int lc = 64 * wave + 16 * i + 4 * (i16 & 3);  // column within the tile
        const int c = lc >> 3, o = (lc & 7) * 2;
        const v4i16 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_v4i16*)(xs + m1 * 512 + ((c ^ xsw(m1)) << 4) + o));
        const v4i16 v2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_v4i16*)(xs + m2 * 512 + ((c ^ xsw(m2)) << 4) + o));
        a[i] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(v1, v2, 0, 1, 2, 3, 4, 5, 6, 7));
      }
#pragma unroll
      for (int cg = 0; cg < RG; ++cg) {
        const int jc = 16 * cg + 4 * (i16 & 3);
        const v4i16 v1 =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(ts + m1 * (RG * 32) + jc * 2));
        const v4i16 v2 =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(ts + m2 * (RG * 32) + jc * 2));
        b[cg] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(v1, v2, 0, 1, 2, 3, 4, 5, 6, 7));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int cg = 0; cg < RG; ++cg) acc[i][cg] = mfma16(a[i], b[cg], acc[i][cg]);
    }
  };
#pragma unroll
  for (int s = 0; s < CL_NS - 1; ++s) issue(s, lds + s * CL_STAGE);
  for (int s = 0; s < nst; ++s) {
    wait_vmcnt<CL_LOADS*(CL_NS - 2)>();  // this lane's copies of stage s have landed
    lds_barrier();                         // everyone's have; slot (s-1) % CL_NS is free
    step(s, lds + (s % CL_NS) * CL_STAGE, lds + ((s + CL_NS - 1) % CL_NS) * CL_STAGE);
  }
  __builtin_amdgcn_s_waitcnt(0);  // drain the trailing (out-of-range) copies before exit

  // C fragment: rows (columns l of X) 4g..4g+3, column (rank j) i16 of each 16x16 block.
  // The split's partial is stored in the layout of the output ([L, r], or [r, L] transposed:
  // then a lane's 4 consecutive l are one 16-byte store), so the reduction reads it in order.
  float* P = pb.partial + (int64_t)zi * L * r;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int cg = 0; cg < RG; ++cg) {
      const int j = 16 * cg + i16;
      const int l0 = lb + 64 * wave + 16 * i + 4 * g;  // L is a multiple of 8: all 4 or none
      if (j >= r || l0 >= L) continue;
      if (pb.transpose) {
        *reinterpret_cast<float4*>(P + (int64_t)j * L + l0) =
            make_float4(pb.scale * acc[i][cg][0], pb.scale * acc[i][cg][1],
                        pb.scale * acc[i][cg][2], pb.scale * acc[i][cg][3]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) P[(int64_t)(l0 + e) * r + j] = pb.scale * acc[i][cg][e];
      }
    }
}

// out = sum_z partial[z] in z order, as bf16 or fp32; the partials are in the output's layout
// ([L, r] or [r, L]), so one thread per output element reads and writes in order. Both
// problems of a cols_kernel launch are reduced by one launch: threads [0, n0) problem a, the
// rest b.
struct RedProb {
  const float* partial;
  void* out;
  int64_t L;
  int Z;
};
__global__ void reduce_kernel(const RedProb a, const RedProb b, int64_t n0, int64_t n, int r,
                              int out_bf16) {
  int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= n) return;
  const bool second = o >= n0;
  const RedProb& p = second ? b : a;
  if (second) o -= n0;
  const float* src = p.partial + o;
  const int64_t zs = p.L * r;
  // the loads of 8 splits are issued together, the adds stay in z order
  float s = 0.f;
  int z = 0;
  for (; z + 8 <= p.Z; z += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = src[(int64_t)(z + u) * zs];
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
  }
  for (; z < p.Z; ++z) s += src[(int64_t)z * zs];
  if (out_bf16)
    reinterpret_cast<uint16_t*>(p.out)[o] = (uint16_t)f2bf(s);
  else
    reinterpret_cast<float*>(p.out)[o] = s;
}

static int cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        v <= 0)
      v = 256;
    cache[dev] = v;
  }
  return cache[dev];
}

// M split of the column kernel: one split length for both problems (so every workgroup
// streams the same rows), the z that minimises waves x (stages per split + CL_RAMP), where a
// wave is CL_PER_CU workgroups on every CU and a split keeps at least PLZ_CL_MINST stages
// (CL_RAMP: the stages' worth of time a workgroup spends filling its copy ring). Returns the
// split length in rows (a multiple of CL_BM).
constexpr int CL_PER_CU = 160 * 1024 / CL_LDS;
#ifndef PLZ_CL_RAMP
#define PLZ_CL_RAMP 4
#endif
constexpr int CL_RAMP = PLZ_CL_RAMP;
static int64_t col_split(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = (N + CL_L - 1) / CL_L + (K + CL_L - 1) / CL_L;
  const int64_t stages = (M + CL_BM - 1) / CL_BM;
  const int64_t slots = (int64_t)CL_PER_CU * cu_count();
  int64_t best = 1;
  double best_t = 1e300;
  for (int64_t z = 1; z <= 64 && (z == 1 || stages / z >= PLZ_CL_MINST); ++z) {
    const int64_t per = (stages + z - 1) / z;
    const int64_t waves = (tiles * z + slots - 1) / slots;
    const double t = (double)waves * (double)(per + CL_RAMP);
    if (t < best_t) {
      best_t = t;
      best = z;
    }
  }
  return (stages + best - 1) / best * CL_BM;
}
static int col_splits(int64_t M, int64_t N, int64_t K) {
  const int64_t s = col_split(M, N, K);
  return s > 0 ? (int)((M + s - 1) / s) : 0;
}

// grad_B = scale * grad_y^T t ([N, r]) and grad_A = (x^T gt)^T ([r, K]): one cols_kernel launch
// over both, then one reduction launch. Workspace: split partials of B, then of A.
static size_t cols_workspace_floats(int64_t M, int64_t N, int64_t K, int r) {
  return (size_t)col_splits(M, N, K) * (size_t)(N + K) * r;
}
static int cols(const uint16_t* x, const uint16_t* grad_y, const uint16_t* t, const uint16_t* gt,
                float scale, void* grad_a, void* grad_b, int out_bf16, float* ws, int64_t M,
                int64_t N, int64_t K, int r, hipStream_t s, const char* what) {
  ColsArgs g = {};
  g.M = M;
  g.r = r;
  const int64_t Ls[2] = {N, K};
  const int64_t split = col_split(M, N, K);
  float* part = ws;
  int nwg[2];
  RedProb red[2];
  for (int i = 0; i < 2; ++i) {
    ColProb& p = g.p[i];
    p.X = i == 0 ? grad_y : x;
    p.T = i == 0 ? t : gt;
    p.scale = i == 0 ? scale : 1.f;
    p.L = (int)Ls[i];
    p.tiles = (int)((Ls[i] + CL_L - 1) / CL_L);
    p.transpose = i;  // grad_A is [r, K]
    p.split = split;
    p.partial = part;
    const int z = (int)((M + p.split - 1) / p.split);
    nwg[i] = p.tiles * z;
    red[i] = RedProb{part, i == 0 ? grad_b : grad_a, Ls[i], z};
    part += (size_t)z * Ls[i] * r;
  }
  g.nwg0 = nwg[0];
  if (nwg[0] + nwg[1] == 0) return PLZ_OK;
  const dim3 grid((unsigned)(nwg[0] + nwg[1]));
  int rc;
  // one device mask per kernel: each instance needs its own LDS attribute
  static uint64_t lds_done1 = 0, lds_done2 = 0;
  if (r <= 16) {
    if ((rc = reserve_lds((const void*)cols_kernel<1>, CL_LDS, lds_done1, what))) return rc;
    hipLaunchKernelGGL(cols_kernel<1>, grid, dim3(256), CL_LDS, s, g);
  } else {
    if ((rc = reserve_lds((const void*)cols_kernel<2>, CL_LDS, lds_done2, what))) return rc;
    hipLaunchKernelGGL(cols_kernel<2>, grid, dim3(256), CL_LDS, s, g);
  }
  if ((rc = check_launch(what))) return rc;
  const int64_t n0 = N * r, n = n0 + K * r;
  hipLaunchKernelGGL(reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, red[0],
                     red[1], n0, n, r, out_bf16);
  return check_launch(what);
}

template <bool BOP_T>
static int rows(const uint16_t* X, const uint16_t* bop, float scale, uint16_t* out, int64_t M,
                int64_t L, int r, hipStream_t s, const char* what) {
  const dim3 grid((unsigned)((M + RR_ROWS - 1) / RR_ROWS));
  static uint64_t done1 = 0, done2 = 0;
  int rc;
  if (r <= 16) {
    constexpr size_t lds = (size_t)RR_NS * rr_stage_bytes<1>();
    if ((rc = reserve_lds((const void*)rows_ring_kernel<BOP_T, 1>, lds, done1, what))) return rc;
    hipLaunchKernelGGL((rows_ring_kernel<BOP_T, 1>), grid, dim3(512), lds, s, X, bop, out, scale,
                       M, (int)L, r);
  } else {
    constexpr size_t lds = (size_t)RR_NS * rr_stage_bytes<2>();
    if ((rc = reserve_lds((const void*)rows_ring_kernel<BOP_T, 2>, lds, done2, what))) return rc;
    hipLaunchKernelGGL((rows_ring_kernel<BOP_T, 2>), grid, dim3(512), lds, s, X, bop, out, scale,
                       M, (int)L, r);
  }
  return check_launch(what);
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace lora
}  // namespace plz

using namespace plz;
using namespace plz::lora;

extern "C" {

int plz_lora_project(const uint16_t* x, const uint16_t* lora_a, float scale, uint16_t* t,
                     int64_t M, int64_t K, int rank, void* stream) {
  PLZ_REQUIRE(M >= 0 && K >= 0 && rank > 0 && rank <= 32 && rank % 8 == 0,
              "plz_lora_project: need M, K >= 0 and rank a multiple of 8 in [8, 32]");
  PLZ_REQUIRE(K % 8 == 0, "plz_lora_project: K must be a multiple of 8");
  PLZ_REQUIRE(K < (1 << 24) && RR_ROWS * K * 2 < (int64_t)1 << 31,
              "plz_lora_project: K (%lld) too large", (long long)K);
  if (M == 0) return PLZ_OK;
  PLZ_REQUIRE(x && lora_a && t && aligned16(x) && aligned16(lora_a),
              "plz_lora_project: null or misaligned pointer");
  return rows<true>(x, lora_a, scale, t, M, K, rank, (hipStream_t)stream, "plz_lora_project");
}

int plz_lora_grad_t(const uint16_t* grad_y, const uint16_t* lora_b, float scale, uint16_t* gt,
                    int64_t M, int64_t N, int rank, void* stream) {
  PLZ_REQUIRE(M >= 0 && N >= 0 && rank > 0 && rank <= 32 && rank % 8 == 0,
              "plz_lora_grad_t: need M, N >= 0 and rank a multiple of 8 in [8, 32]");
  PLZ_REQUIRE(N % 8 == 0, "plz_lora_grad_t: N must be a multiple of 8");
  PLZ_REQUIRE(N < (1 << 24) && RR_ROWS * N * 2 < (int64_t)1 << 31,
              "plz_lora_grad_t: N (%lld) too large", (long long)N);
  if (M == 0) return PLZ_OK;
  PLZ_REQUIRE(grad_y && lora_b && gt && aligned16(grad_y) && aligned16(lora_b),
              "plz_lora_grad_t: null or misaligned pointer");
  return rows<false>(grad_y, lora_b, scale, gt, M, N, rank, (hipStream_t)stream,
                     "plz_lora_grad_t");
}

size_t plz_lora_weight_grads_workspace(int64_t M, int64_t N, int64_t K, int rank) {
  if (M <= 0 || rank <= 0) return 0;
  return cols_workspace_floats(M, N, K, rank) * sizeof(float);
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
  PLZ_REQUIRE((grad_a || K == 0) && (grad_b || N == 0), "plz_lora_weight_grads: null output");
  hipStream_t s = (hipStream_t)stream;
  const int bf = out_dtype == PLZ_DT_BF16;
  if (M == 0) {  // empty reduction: zero gradients (the inputs may be null)
    zero_async(grad_b, (size_t)N * rank * (bf ? 2 : 4), s);
    zero_async(grad_a, (size_t)K * rank * (bf ? 2 : 4), s);
    return check_launch("plz_lora_weight_grads");
  }
  PLZ_REQUIRE(x && grad_y && t && gt && grad_a && grad_b, "plz_lora_weight_grads: null pointer");
  PLZ_REQUIRE(aligned16(x) && aligned16(grad_y) && aligned16(t) && aligned16(gt),
              "plz_lora_weight_grads: inputs must be 16-byte aligned");
  const int64_t split = col_split(M, N, K);
  PLZ_REQUIRE(split * N * 2 < (int64_t)1 << 31 && split * K * 2 < (int64_t)1 << 31,
              "plz_lora_weight_grads: M split x N or K too large");
  const size_t need = plz_lora_weight_grads_workspace(M, N, K, rank);
  if (!workspace || workspace_bytes < need) {
    set_error("plz_lora_weight_grads: workspace of %zu bytes needed, %zu given", need,
              workspace_bytes);
    return PLZ_EWORKSPACE;
  }
  return cols(x, grad_y, t, gt, scale, grad_a, grad_b, bf, reinterpret_cast<float*>(workspace), M,
              N, K, rank, s, "plz_lora_weight_grads");
}

}  // extern "C"
