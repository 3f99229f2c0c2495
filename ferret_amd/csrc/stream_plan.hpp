// Host-side launch plan of the persistent stream kernel (stream_kernel.hpp):
// which shapes it takes and how the units are dealt to work-groups.  Plain
// C++17 with no HIP dependency, so that the CPU tests compile it on its own
// and walk every work-group of every configuration the library instantiates
// (tests/test_stream_plan.py): no unit may address a weight row at or past N,
// an output row past the output, a K-step past K, or a tile-table span
// larger than the work-group's LDS copy.
#pragma once

#include <cstdint>

namespace ferret {

constexpr int kStreamMaxTiles = 64;  // token tiles one work-group may touch (tile table in LDS)

struct StreamPlan {
  bool ok = false;      // false: the shape is not covered (the caller uses the per-unit kernel)
  int ks = 0;           // K-steps per wave and unit
  int unit_rows = 0;    // weight rows per unit (SiLU: one 16-row block of gate and one of up)
  int units_n = 0;      // units per token tile
  long long units = 0;  // all units (x nsplit for split-K)
  long long per = 0;    // units per work-group (the last ones get fewer)
  int nsplit = 1;       // K splits (bf16 dense split-K only)
};

// silu: SiLU epilogue (unit = 16 gate rows + 16 up rows, N/2 output rows);
// rb: 16-row blocks per unit (store epilogue); nw: waves per work-group;
// tiles: dense token tiles, or the tile table's max_tiles when grouped;
// nsplit: K splits (1 = none).  Mirrors the checks of try_stream.
inline StreamPlan stream_plan(bool silu, int rb, int nw, int N, int K, int tiles, bool grouped, int nsplit,
                              int grid) {
  StreamPlan p;
  p.unit_rows = silu ? 16 : 16 * rb;
  const int out_rows = silu ? N / 2 : N;
  if (N <= 0 || K <= 0 || K % 128 != 0 || tiles <= 0 || grid <= 0 || nsplit < 1) return p;
  if (out_rows % p.unit_rows != 0) return p;
  p.units_n = out_rows / p.unit_rows;
  const int nkb = K >> 7;
  if (nkb % (nw * nsplit) != 0) return p;
  p.ks = nkb / nsplit / nw;
  if (p.ks != 2 && p.ks != 4 && p.ks != 7 && p.ks != 8) return p;
  // Past 8 waves a wave has 128 VGPRs: at most 4 K-steps of activations.
  if (nw > 8 && p.ks > 4) return p;
  p.nsplit = nsplit;
  p.units = (long long)tiles * p.units_n * nsplit;
  p.per = (p.units + grid - 1) / grid;
  // A work-group's units span at most per / units_n + 2 token tiles; the
  // grouped kernel copies that span of the tile table to LDS.
  if (grouped && p.per / p.units_n + 2 > kStreamMaxTiles) return p;
  p.ok = true;
  return p;
}

}  // namespace ferret
