"""Launch geometry of the attention kernels, checked on the CPU.

The kernels and their launchers share ``csrc/hier_launch.h``: the grid for a
number of logical work items (item x head) and the XCD-aware map from
workgroup id to logical item.  This test compiles that header with g++ and
checks, for many item counts, that the grid is a multiple of the 8 XCDs and
covers every item, that the map is a bijection on [0, grid), that every item
below the count is run by exactly one workgroup (the others exit at the
``logical >= total`` guard), and that consecutive logical items of one XCD's
share are consecutive workgroups of that XCD (bid = 8 j + x).
"""

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "multics_amd" / "csrc"

PROGRAM = r"""
#include <stdio.h>
#include <stdint.h>
#include <vector>
#include "hier_launch.h"
int main() {
  const int64_t totals[] = {1, 2, 7, 8, 9, 15, 16, 17, 63, 64, 65, 378, 2322, 9072, 9073,
                            24 * 1233, 100003};
  for (int64_t total : totals) {
    const int64_t g = hier::xcd_grid(total);
    if (g % hier::kXcds != 0 || g < total || g - total >= hier::kXcds) {
      printf("FAIL grid total=%lld grid=%lld\n", (long long)total, (long long)g); return 1;
    }
    std::vector<int> seen(g, 0);
    int64_t run = 0;
    for (int bid = 0; bid < g; ++bid) {
      const int l = hier::xcd_logical(bid, (int)g);
      if (l < 0 || l >= g) { printf("FAIL range total=%lld bid=%d l=%d\n", (long long)total, bid, l); return 1; }
      seen[l]++;
      if (l < total) ++run;
      // the workgroups of one XCD (bid % 8) run one contiguous share of items
      if (bid >= hier::kXcds && l != hier::xcd_logical(bid - hier::kXcds, (int)g) + 1) {
        printf("FAIL contiguity total=%lld bid=%d\n", (long long)total, bid); return 1;
      }
    }
    for (int64_t l = 0; l < g; ++l)
      if (seen[l] != 1) { printf("FAIL bijection total=%lld l=%lld\n", (long long)total, (long long)l); return 1; }
    if (run != total) { printf("FAIL guard total=%lld run=%lld\n", (long long)total, (long long)run); return 1; }
  }
  if (hier::xcd_grid(0) != 0 || hier::xcd_grid(-5) != 0) { printf("FAIL empty\n"); return 1; }
  // the largest accepted launch still has a grid that fits an int
  if (hier::xcd_grid(hier::kMaxLaunchItems) > 2147483647ll) { printf("FAIL max\n"); return 1; }
  printf("OK\n");
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_xcd_grid_and_map(tmp_path):
    src = tmp_path / "launch.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "launch"
    subprocess.run(["g++", "-std=c++17", "-O1", f"-I{CSRC}", str(src), "-o", str(exe)], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True)
    assert res.returncode == 0 and res.stdout.strip() == "OK", res.stdout


def test_kernels_use_the_shared_launch_math():
    """Every attention kernel maps workgroups through the shared header (no
    private copy of the arithmetic that this test would not see)."""
    for name in ("hier_attn_fwd.hip", "hier_attn_bwd.hip"):
        text = (CSRC / name).read_text()
        assert "hier_launch.h" in text, name
        assert "bid & 7" not in text and "+ 7) / 8 * 8" not in text, name
        assert "xcd_logical(blockIdx.x, gridDim.x)" in text, name
