"""CPU test of the dense kernels' tile-row arithmetic (geoweave_amd/csrc/gw_tile_rows.h, the
code the dense forward's and backward's tile loads compile). A 64-row tile at k0 loads rows
srow and srow + 32 (srow < 32) of an n-row operand from a base row plus a 32-bit lane offset
(row offset times the row stride in a 24-bit multiply). Padded query and key blocks start at
or past n; an offset taken from k0 there went negative and wrapped, and the kernel read out
of bounds. The header is compiled with g++ into a small program that checks, for every tile
a kernel can load (k0 up to past the padded length) and every srow:
  * the rows read are min(k0 + srow, n - 1) and min(k0 + srow + 32, n - 1): in range;
  * the offsets lie in [0, 63], so offset x stride stays below 2^30 for strides below 2^24
    bytes (the hosts' limit), inside the 24-bit multiply's operand range;
and that the unclamped base (k0) of the old code fails the same check (the checker sees the
mistake it is meant to catch). No GPU work.
"""
import shutil
import subprocess
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parents[1] / "geoweave_amd" / "csrc"

PROGRAM = r"""
#include <stdio.h>
#include "gw_tile_rows.h"

static int check(bool clamped) {
  int bad = 0;
  const int lens[] = {1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257, 1000, 1374, 5496,
                      32976, 43968, 87936, (1 << 24) - 1, (1 << 24), (1 << 24) + 1, (1 << 25) - 256};
  for (int n : lens) {
    const int npad = (n + 255) / 256 * 256;          // query blocks padded to whole workgroups
    for (int k0 = 0; k0 <= npad + 64; k0 += 64) {
      if (n > 100000 && k0 > 256 && k0 < n - 512) k0 = n - 512;  // long operands: the start and the end
      for (int srow = 0; srow < 32; ++srow) {
        gw::TileRows tr = gw::tile_rows(k0, srow, n);
        if (!clamped) tr.base = k0, tr.r0 = (uint32_t)(gw::tile_imin(k0 + srow, n - 1) - k0),
                      tr.r1 = (uint32_t)(gw::tile_imin(k0 + srow + 32, n - 1) - k0);
        const long long row0 = (long long)tr.base + tr.r0, row1 = (long long)tr.base + tr.r1;
        const long long want0 = k0 + srow < n - 1 ? k0 + srow : n - 1;
        const long long want1 = k0 + srow + 32 < n - 1 ? k0 + srow + 32 : n - 1;
        const bool ok = tr.base >= 0 && tr.base <= n - 1 && tr.r0 <= 63u && tr.r1 <= 63u && row0 == want0 &&
                        row1 == want1 && (unsigned long long)tr.r1 * ((1ull << 24) - 1) < (1ull << 30);
        if (!ok) {
          if (bad < 3) printf("n=%d k0=%d srow=%d base=%d r0=%u r1=%u\n", n, k0, srow, tr.base, tr.r0, tr.r1);
          ++bad;
        }
      }
    }
  }
  return bad;
}

int main() {
  const int bad_clamped = check(true), bad_naive = check(false);
  printf("clamped %d naive %d\n", bad_clamped, bad_naive);
  return bad_clamped == 0 && bad_naive > 0 ? 0 : 1;
}
"""


def test_tile_rows_stay_in_bounds(tmp_path):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ not found")
    src = tmp_path / "tile_rows.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "tile_rows"
    subprocess.run([cxx, "-std=c++17", "-O1", f"-I{CSRC}", str(src), "-o", str(exe)], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True)
    print(res.stdout)
    assert res.returncode == 0, res.stdout
    assert "clamped 0 " in res.stdout
