"""CPU proof that the stream kernel's launch plan stays in bounds.

Compiles ferret_amd/csrc/stream_plan.hpp (the host-only plan that try_stream in
skinny.hip uses) with g++ together with a small bounds walker, and walks every
work-group of every configuration the library instantiates, over a sweep of
shapes, tile counts, split counts and grid sizes.  For each plan the shape is
accepted for, the walk follows the kernel's index arithmetic
(stream_kernel.hpp: unit -> split, token tile, row unit; rows of a unit's
blocks; each wave's K-steps; the span of the tile table a work-group copies to
LDS) and fails if any unit addresses a weight row >= N, an output row past the
output, a K-step >= K / 128, or a tile-table span > kStreamMaxTiles.  The
configuration that once faulted the GPU (two 16-row blocks per unit while the
unit count assumed one) is a mutant of the plan that the walk rejects.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "ferret_amd", "csrc")

CHECKER = r"""
#include <algorithm>
#include <cstdio>
#include <vector>
#include "stream_plan.hpp"
using namespace ferret;

struct Cfg { const char* name; bool silu; int rb; int nw; bool grouped; int max_split; };
// every try_stream<F, EPI, RB, D, NW> instantiation in skinny.hip
static const Cfg kCfgs[] = {
  {"bf16 linear, 8 waves (+ split-K)", false, 1, 8, false, 8},
  {"bf16 linear, 4 waves", false, 1, 4, false, 1},
  {"fp8 dense, two blocks per unit", false, 2, 8, false, 1},
  {"fp8 dense, 14 waves", false, 1, 14, false, 1},
  {"fp8 dense, 8 waves", false, 1, 8, false, 1},
  {"fp8 moe w13 (SiLU)", true, 2, 8, true, 1},
  {"fp8 moe w2, four blocks per unit", false, 4, 4, true, 1},
  {"int4 moe w13 (SiLU)", true, 2, 8, true, 1},
};

static long long violations = 0, plans = 0;
static void fail(const char* what, const Cfg& c, int N, int K, int tiles, int ns, int grid) {
  if (violations++ < 20)
    std::printf("VIOLATION %s: %s N=%d K=%d tiles=%d nsplit=%d grid=%d\n", what, c.name, N, K, tiles, ns, grid);
}

// The kernel's arithmetic for one accepted plan; ntiles = the device tile count (<= tiles when grouped).
static void walk(const Cfg& c, int N, int K, int tiles, int ns, int grid, int ntiles, const StreamPlan& p,
                 int rb_used) {
  const long long ups = (long long)ntiles * p.units_n;
  const long long units = ups * ns;
  const long long per = (units + grid - 1) / grid;
  const int nkb = K / 128;
  // rows of the last row unit (rows only depend on the row unit nu < units_n)
  const int nu = p.units_n - 1;
  for (int rb = 0; rb < (c.silu ? 2 : rb_used); ++rb) {
    const long long row0 = c.silu ? (rb == 0 ? nu * 16LL : N / 2 + nu * 16LL) : ((long long)nu * rb_used + rb) * 16;
    if (row0 + 16 > N) fail("weight row >= N", c, N, K, tiles, ns, grid);
    if (c.silu && nu * 16LL + 16 > N / 2) fail("output row >= N/2", c, N, K, tiles, ns, grid);
  }
  for (int split = 0; split < ns; ++split)
    for (int w = 0; w < c.nw; ++w)
      if (((long long)split * c.nw + w) * p.ks + p.ks > nkb) fail("K-step >= K/128", c, N, K, tiles, ns, grid);
  if (c.grouped) {
    for (long long b = 0; b < grid; ++b) {
      const long long ub = std::min(units, b * per), ue = std::min(units, ub + per);
      if (ub >= ue) continue;
      const long long span = (ue - 1) / p.units_n - (ub % ups) / p.units_n + 1;
      if (span > kStreamMaxTiles) fail("tile-table span > kStreamMaxTiles", c, N, K, tiles, ns, grid);
    }
  }
}

int main() {
  const int Ns[] = {16, 32, 48, 64, 96, 128, 256, 512, 1024, 2048, 3072, 4096, 6144, 7168, 24576, 153600};
  const int Ks[] = {128, 256, 384, 512, 896, 1024, 1536, 2048, 3584, 4096, 7168, 8192, 12288, 16384};
  const int Tiles[] = {1, 2, 3, 7, 8, 16, 63, 64, 65, 127, 300, 1000, 4096};
  const int Grids[] = {80, 256, 304};
  for (const Cfg& c : kCfgs)
    for (int N : Ns)
      for (int K : Ks)
        for (int tiles : Tiles)
          for (int grid : Grids)
            for (int ns = 1; ns <= c.max_split; ++ns) {
              const StreamPlan p = stream_plan(c.silu, c.rb, c.nw, N, K, tiles, c.grouped, ns, grid);
              if (!p.ok) continue;
              ++plans;
              if (p.units_n * p.unit_rows != (c.silu ? N / 2 : N)) fail("units_n does not tile N", c, N, K, tiles, ns, grid);
              walk(c, N, K, tiles, ns, grid, tiles, p, c.rb);
              if (c.grouped) walk(c, N, K, tiles, ns, grid, tiles > 3 ? tiles / 3 : 1, p, c.rb);
#ifdef MUTANT_RB_MISMATCH
              // a kernel with RB = 2 launched on the unit count of RB = 1
              if (!c.silu && c.rb == 1) {
                StreamPlan q = stream_plan(c.silu, 1, c.nw, N, K, tiles, c.grouped, ns, grid);
                walk(c, N, K, tiles, ns, grid, tiles, q, 2);
              }
#endif
            }
  std::printf("plans %lld violations %lld\n", plans, violations);
  return violations == 0 ? 0 : 1;
}
"""


def _build(tmp_path, *defines):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    src = tmp_path / "plan_check.cpp"
    src.write_text(CHECKER)
    exe = tmp_path / ("plan_check" + "".join(d.lower() for d in defines))
    cmd = [gxx, "-std=c++17", "-O2", "-I", CSRC, *[f"-D{d}" for d in defines], str(src), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return exe


def test_every_instantiated_stream_plan_stays_in_bounds(tmp_path):
    exe = _build(tmp_path)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    plans = int(res.stdout.split()[1])
    assert plans > 1000, res.stdout            # the sweep reaches many accepted shapes


def test_walker_rejects_the_rb_mismatch_that_faulted(tmp_path):
    exe = _build(tmp_path, "MUTANT_RB_MISMATCH")
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert res.returncode != 0 and "weight row >= N" in res.stdout


def _instantiations():
    """(silu, RB, NW, grouped) of every try_stream<F, EPI, RB, D[, NW]>(a, dense_tiles, max_tiles, st)
    call in skinny.hip (NW defaults to 8; a call with dense_tiles 0 is grouped)."""
    import re
    src = open(os.path.join(CSRC, "skinny.hip")).read()
    pat = re.compile(r"try_stream<\s*(\w+)\s*,\s*(\w+)\s*,\s*(\d+)\s*,\s*(\d+)\s*(?:,\s*(\d+)\s*)?>\s*"
                     r"\(\s*a\s*,\s*([^,]+?)\s*,\s*([^,]+?)\s*,\s*st\s*\)")
    calls = [(m.group(2) == "kSilu", int(m.group(3)), int(m.group(5) or 8), m.group(6) == "0")
             for m in pat.finditer(src)]
    return calls, src.count("try_stream<")   # the template's definition is `try_stream(`


def _walker_cfgs():
    import re
    body = CHECKER[CHECKER.index("kCfgs[] = {"):CHECKER.index("};", CHECKER.index("kCfgs[] = {"))]
    return {(m.group(1) == "true", int(m.group(2)), int(m.group(3)), m.group(4) == "true")
            for m in re.finditer(r'\{"[^"]*",\s*(true|false),\s*(\d+),\s*(\d+),\s*(true|false),\s*\d+\}', body)}


def test_walker_covers_every_try_stream_instantiation():
    """kCfgs above is written by hand: every try_stream instantiation in
    skinny.hip must appear in it, so an added or changed one cannot escape the
    bounds walk."""
    calls, n_sites = _instantiations()
    assert len(calls) == n_sites >= 9, (len(calls), n_sites)   # the regex saw every call site
    cfgs = _walker_cfgs()
    assert len(cfgs) >= 6   # distinct (silu, RB, NW, grouped) tuples of the eight entries
    missing = sorted(set(calls) - cfgs)
    assert not missing, f"try_stream instantiations not walked by the plan walk (silu, RB, NW, grouped): {missing}"
