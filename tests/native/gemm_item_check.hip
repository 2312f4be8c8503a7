// Host-side check of the MFMA GEMM's work-item index math (plz_gemm2.cuh: map_item,
// tile_coords, split_len, palette_splits_on, soft_splits, tail_plan_on), built with asserts on
// and run on the CPU by tests/test_index_math.py. For every launch the entry points of
// plz_gemm2.hip make -- the hard forward / grad_x / grad_palette, the dense GEMMs, the soft
// backward, the no-allocation grad_palette -- over many shapes and CU counts it enumerates
// every workgroup (blockIdx.x, blockIdx.z) as the kernel sees it and checks that
//   * every tile index, tile coordinate, split and tail part is in range,
//   * every (split, tile) and every (tail tile, part) is run by exactly one workgroup,
//   * the reduction ranges of the splits / parts are non-empty, disjoint and cover [0, R),
//   * the grad_palette partials each workgroup writes stay inside the workspace it sizes.
#undef NDEBUG
#include <cassert>
#include <cstdio>
#include <set>
#include <utility>
#include <vector>

#include "plz_gemm2.cuh"

using namespace plz::g2;

static long checks = 0;

static void check_ranges(const std::vector<std::pair<int64_t, int64_t>>& r, int64_t R) {
  // r: [begin, end) per split or part, in index order
  int64_t at = 0;
  for (const auto& p : r) {
    assert(p.first == at && "reduction ranges must be contiguous from 0");
    assert(p.second > p.first && "a reduction range must not be empty");
    at = p.second;
  }
  assert(at == R && "reduction ranges must cover [0, R)");
  ++checks;
}

// one launch: I x J outputs, reduction R, z splits of r_split, optional tail plan, tile walk
static void check_launch(int64_t I, int64_t J, int64_t R, int z, int64_t r_split, TailPlan tp,
                         bool tail_ok, int group, int64_t partial_floats) {
  const int tiles_i = (int)((I + TILE - 1) / TILE), tiles_j = (int)((J + TILE - 1) / TILE);
  const int T = tiles_i * tiles_j;
  if (T == 0) return;
  const bool tail = tail_ok && tp.split > 1;
  const int gx = tail ? tp.first + (T - tp.first) * tp.split : T;
  const int gz = z;
  std::set<std::pair<int, int>> seen_whole, seen_part;
  std::set<std::pair<int, int>> seen_tile;
  for (int bz = 0; bz < gz; ++bz)
    for (int bx = 0; bx < gx; ++bx) {
      const Item it = map_item(T, tail, tp.first, tp.split, bx, bz, gz);
      int ti, tj;
      tile_coords(group, tiles_i, tiles_j, it.bid, ti, tj);
      assert(ti >= 0 && ti < tiles_i && tj >= 0 && tj < tiles_j);
      if (it.tail_part) {
        assert(tail && it.bid >= tp.first && it.bid < T);
        assert(it.part >= 0 && it.part < tp.split && it.zsl == 0);
        assert(seen_part.insert({it.bid, it.part}).second && "tail part run twice");
      } else {
        assert(it.bid >= 0 && it.bid < (tail ? tp.first : T));
        assert(it.zsl >= 0 && it.zsl < gz);
        assert(seen_whole.insert({it.zsl, it.bid}).second && "item run twice");
        seen_tile.insert({ti, tj});
        if (partial_floats > 0) {  // grad_palette partials [z][I][J/128][4] of this tile
          const int64_t n_last = std::min<int64_t>(I, (int64_t)(ti + 1) * TILE) - 1;
          const int64_t seg_last = std::min<int64_t>(J, (int64_t)(tj + 1) * TILE) / 128 - 1;
          const int64_t hi = (((int64_t)it.zsl * I + n_last) * (J / 128) + seg_last) * 4 + 4;
          assert(hi <= partial_floats && "partials outside the workspace");
        }
      }
    }
  assert((int64_t)seen_whole.size() == (int64_t)gz * (tail ? tp.first : T));
  if (tail) assert((int)seen_part.size() == (T - tp.first) * tp.split);
  if (!tail) assert((int)seen_tile.size() == T && "every tile must be covered");
  // reduction ranges, as the kernel derives them
  std::vector<std::pair<int64_t, int64_t>> rs;
  for (int zs = 0; zs < gz; ++zs) {
    const int64_t b = (int64_t)zs * r_split, e = std::min(R, b + r_split);
    rs.push_back({b, e});
  }
  check_ranges(rs, R);
  if (tail) {
    std::vector<std::pair<int64_t, int64_t>> ps;
    for (int p = 0; p < tp.split; ++p) {
      const int64_t b = (int64_t)p * tp.len, e = std::min(R, b + tp.len);
      ps.push_back({b, e});
    }
    check_ranges(ps, R);
  }
  ++checks;
}

int main() {
  const int64_t Ms[] = {1, 7, 77, 256, 300, 512, 2048, 4160, 8192, 16384, 16448};
  const int64_t NKs[][2] = {{4096, 2560}, {1024, 2560}, {2560, 4096}, {9728, 2560}, {2560, 9728},
                            {256, 256}, {8, 256}, {136, 1024}, {1032, 768}, {2560, 2560},
                            {264, 768}, {4160, 2560}};
  const int64_t Cs[] = {256, 304, 80, 128, 1};
  int launches = 0;
  for (int64_t C : Cs)
    for (int64_t M : Ms)
      for (const auto& nk : NKs) {
        const int64_t N = nk[0], K = nk[1];
        // hard / dense forward: I = M, J = N, R = K (tail plan when a workspace is given)
        check_launch(M, N, K, 1, K, tail_plan_on(M, N, K, C), true, 1, 0);
        check_launch(M, N, K, 1, K, tail_plan_on(M, N, K, C), true, 8, 0);
        // grad_x: I = M, J = K, R = N
        check_launch(M, K, N, 1, N, tail_plan_on(M, K, N, C), true, 1, 0);
        check_launch(M, K, N, 1, N, tail_plan_on(M, K, N, C), true, 8, 0);
        // SwiGLU gate/up: no tail
        check_launch(M, 2 * N, K, 1, K, TailPlan{}, false, 8, 0);
        // grad_palette: I = N, J = K, R = M, split over M, walk by the larger operand
        const int z = palette_splits_on(M, N, K, C);
        const int64_t ws = (int64_t)z * N * (K / 128) * 4;
        check_launch(N, K, M, z, split_len(M, z), TailPlan{}, false, K > N ? -1 : 1, ws);
        // the no-allocation variant: the split count lowered to fit a 32 MiB scratch
        const int64_t per_split = N * (K / 128) * 4;
        const int zfit = (int)(((int64_t)32 << 20) / 4 / per_split);
        if (zfit >= 1) {
          const int zn = z < zfit ? z : zfit;
          check_launch(N, K, M, zn, split_len(M, zn), TailPlan{}, false, K > N ? -1 : 1,
                       (int64_t)zn * per_split);
        }
        // soft backward: split over M when soft_splits says so
        const int zs = soft_splits(M, N, K);
        check_launch(N, K, M, zs, zs > 1 ? split_len(M, zs) : M, TailPlan{}, false,
                     K > N ? -1 : 1, 0);
        launches += 9;
      }
  printf("gemm item map: %d launches, %ld checks passed\n", launches, checks);
  return 0;
}
