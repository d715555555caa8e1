// Host check of the persistent GEMMs' tile walk (TileWalk in afd_common.h, compiled here as
// host code): for every row-tile count 1..300, several column-tile counts and grid sizes, and
// the walk block heights the kernels use, every output tile is taken exactly once
//   * statically: workgroup b takes dense positions first, first + stride, ... < tiles of its
//     walk (its XCD's, when the rows are split over the 8 XCDs);
//   * dynamically: each workgroup claims two positions from its walk's counter at the start
//     and one more during each tile that has a successor (as the kernels do), with the claims
//     of all workgroups interleaved in a seeded random order.
// Prints the number of walks checked; exits 1 on the first failure.
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "../sgl-afd-plugin_amd/csrc/afd_common.h"

using afd::TileWalk;

template <int BR>
static bool check_cover(const char* how, int rows, int ntn, int grid, const std::vector<int>& hits) {
  for (int mt = 0; mt < rows; ++mt)
    for (int nt = 0; nt < ntn; ++nt)
      if (hits[mt * ntn + nt] != 1) {
        std::printf("FAIL %s BR=%d rows=%d ntn=%d grid=%d: tile (%d, %d) taken %d times\n", how, BR,
                    rows, ntn, grid, mt, nt, hits[mt * ntn + nt]);
        return false;
      }
  return true;
}

template <int BR>
static bool take(std::vector<int>& hits, const TileWalk<BR>& w, int i, int rows, int ntn) {
  int mt, nt;
  w.at_dense(i, mt, nt);
  if (mt < 0 || mt >= rows || nt < 0 || nt >= ntn) {
    std::printf("FAIL BR=%d rows=%d ntn=%d: position %d -> tile (%d, %d) out of range\n", BR, rows, ntn, i, mt, nt);
    return false;
  }
  // a walk only holds its own row range
  if (mt < w.mt0 || mt >= w.mt0 + w.rows_here) {
    std::printf("FAIL BR=%d rows=%d: row tile %d outside the walk's [%d, %d)\n", BR, rows, mt, w.mt0,
                w.mt0 + w.rows_here);
    return false;
  }
  ++hits[mt * ntn + nt];
  return true;
}

template <int BR>
static bool static_walk(int rows, int ntn, int grid) {
  std::vector<int> hits(rows * ntn, 0);
  for (int b = 0; b < grid; ++b) {
    const TileWalk<BR> w(rows, ntn, b, grid);
    for (int i = w.first; i < w.tiles; i += w.stride)
      if (!take(hits, w, i, rows, ntn)) return false;
  }
  return check_cover<BR>("static", rows, ntn, grid, hits);
}

template <int BR>
static bool dynamic_walk(int rows, int ntn, int grid, std::mt19937& rng) {
  std::vector<int> hits(rows * ntn, 0);
  std::vector<uint32_t> counters(8 * afd::kWalkCounterStride, 0u);
  struct Wg {
    TileWalk<BR> w;
    int i, i_next;
    bool started, done;
  };
  std::vector<Wg> wgs;
  for (int b = 0; b < grid; ++b) {
    TileWalk<BR> w(rows, ntn, b, grid, counters.data());
    wgs.push_back({w, 0, 0, false, false});
  }
  // one step of a workgroup = one claim (a counter increment), in random order
  auto claim = [](Wg& g) { return g.w.resolve((*g.w.ctr)++); };
  std::vector<int> live(grid);
  for (int b = 0; b < grid; ++b) live[b] = b;
  while (!live.empty()) {
    const size_t pick = rng() % live.size();
    Wg& g = wgs[live[pick]];
    if (!g.started) {
      g.started = true;
      const int a = claim(g), b2 = claim(g);  // two claims in flight together
      g.i = a < g.w.tiles ? a : g.w.tiles;
      g.i_next = b2 < g.w.tiles ? b2 : g.w.tiles;
    } else {
      // one tile: process i, claiming the tile after next if i_next exists
      int after = g.w.tiles;
      if (g.i_next < g.w.tiles) after = claim(g);
      if (!take(hits, g.w, g.i, rows, ntn)) return false;
      g.i = g.i_next;
      g.i_next = after;
    }
    if (g.i >= g.w.tiles) {
      live[pick] = live.back();
      live.pop_back();
    }
  }
  return check_cover<BR>("dynamic", rows, ntn, grid, hits);
}

template <int BR>
static int run(std::mt19937& rng) {
  int walks = 0;
  const int ntns[] = {1, 2, 3, 4, 6, 8, 12, 16};
  const int grids[] = {256, 255, 64, 8, 3};
  for (int rows = 1; rows <= 300; ++rows)
    for (int ntn : ntns)
      for (int grid : grids) {
        if (!static_walk<BR>(rows, ntn, grid) || !dynamic_walk<BR>(rows, ntn, grid, rng)) return -1;
        walks += 2;
      }
  return walks;
}

int main() {
  std::mt19937 rng(12345);
  const int a = run<2>(rng);  // the MXFP4 GEMMs' 2 x 16 blocks
  if (a < 0) return 1;
  const int c = run<4>(rng);  // the bf16-activation GEMMs' 4 x 8 blocks
  if (c < 0) return 1;
  const int b = run<8>(rng);  // the FP8 GEMMs' 8 x 4 blocks
  if (b < 0) return 1;
  std::printf("ok: %d walks, every tile taken exactly once\n", a + b + c);
  return 0;
}
