"""The grouped GEMMs' XCD-aware tile order (``schedule_tile_with``,
csrc/gemm_tile.h) on the host: the device function itself (host-and-device)
is compiled into a small host program that walks every virtual block of the
grids the launch code forms and checks that each (m-tile, n-tile) of the
problem is produced exactly once and nothing outside it.  The tile order
only decides which block computes which tile, so a slip in it (a tile twice,
one never, an n-tile past the end) shows as wrong outputs at some shapes
only; here it is checked over thousands of shapes in a second."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "tokamax-tpu-kernel-lab_amd", "csrc")

HARNESS = r"""
#include <cstdio>
#include <vector>
#include "gemm_tile.h"
using namespace lmoe::gemm;

// the virtual-block counts the launch code forms (launch_dma / try_stream /
// the MX launches): gm == 0 stripes n-tiles over the XCDs (ntiles % 8 == 0);
// gm > 0 deals groups of gm m-tiles round-robin over the XCDs
static int64_t grid_blocks(int64_t tm_bound, int64_t ntiles, int gm) {
  if (gm == 0) return tm_bound * ntiles;
  return kXcds * (((tm_bound + gm - 1) / gm + kXcds - 1) / kXcds) * gm * ntiles;
}

// 0: every tile exactly once; 1: a tile out of range; 2: a tile missed or repeated
static int check(int64_t ntiles, int gm, int64_t tm_bound, int64_t tm) {
  const int64_t blocks = grid_blocks(tm_bound, ntiles, gm);
  std::vector<int> seen(static_cast<size_t>(tm * ntiles), 0);
  for (int64_t vb = 0; vb < blocks; ++vb) {
    int64_t nt = -1;
    const TileInfo ti = schedule_tile_with(ntiles, gm, vb, tm, nt, [](int64_t mt) {
      TileInfo t{0, mt, 1, false};
      return t;
    });
    if (ti.group < 0) continue;
    if (ti.row0 < 0 || ti.row0 >= tm || nt < 0 || nt >= ntiles) return 1;
    ++seen[static_cast<size_t>(ti.row0 * ntiles + nt)];
  }
  for (int c : seen)
    if (c != 1) return 2;
  return 0;
}

int main() {
  int cases = 0, bad = 0;
  const int64_t ntiles_list[] = {1, 2, 3, 7, 8, 9, 15, 16, 24, 40, 56, 64, 112};
  const int gms[] = {0, 1, 2, 4};
  for (int64_t ntiles : ntiles_list)
    for (int gm : gms) {
      if (gm == 0 && ntiles % kXcds) continue;
      for (int64_t tm_bound = 1; tm_bound <= 70; tm_bound += (tm_bound < 20 ? 1 : 7))
        for (int64_t tm = 0; tm <= tm_bound; ++tm) {
          ++cases;
          const int r = check(ntiles, gm, tm_bound, tm);
          if (r) {
            if (bad < 5) printf("FAIL ntiles=%lld gm=%d tm_bound=%lld tm=%lld code %d\n", (long long)ntiles, gm,
                                (long long)tm_bound, (long long)tm, r);
            ++bad;
          }
        }
    }
  // the config-5 gate/up launch: 8804 routed rows in 64-row tiles over 113 groups, 8 n-tiles
  ++cases;
  bad += check(8, 0, 8804 / 64 + 113 + 1, 8804 / 64 + 100) != 0;
  printf("%d %d\n", cases, bad);
  return bad != 0;
}
"""


def test_tile_order_covers_every_tile_once(tmp_path):
  src = tmp_path / "sched.hip"
  src.write_text(HARNESS)
  exe = tmp_path / "sched"
  r = subprocess.run(["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-std=c++17", "-O1", "-Wall", "-I", CSRC,
                      str(src), "-o", str(exe)], capture_output=True, text=True, timeout=300)
  assert r.returncode == 0, r.stderr[-2000:]
  r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
  assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
  cases, bad = (int(v) for v in r.stdout.split()[-2:])
  assert bad == 0 and cases > 2000, r.stdout
