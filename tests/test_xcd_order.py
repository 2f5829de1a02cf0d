"""The XCD-aware work order of the forward, dQ and local dK/dV launches
(xcd_grid / xcd_item in csrc/cra_internal.hpp), checked on the host: for
every head count and tile count in a range, the grid's blocks take every
(rank, head) item exactly once, each XCD (block % 8) takes its items in the
plain order's sequence (heaviest first, as the launches without it), and
each item lands on the XCD whose contiguous eighth of the units holds its
unit {rank p, rank nt - 1 - p} of its head. The checker is compiled from
the header with hipcc (host code only)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "cron-root-attention_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

CHECKER = r"""
#include "cra_internal.hpp"
#include <cstdio>
#include <vector>
using namespace cra;
int main() {
  long bad = 0, cases = 0, padding = 0, items = 0;
  for (int nbh = 1; nbh <= 40; ++nbh)
    for (int nt = 1; nt <= 100; ++nt) {
      ++cases;
      const int grid = xcd_grid(nbh, nt);
      std::vector<int> seen(nbh * nt, 0);
      std::vector<long> last(8, -1);
      for (int b = 0; b < grid; ++b) {
        const int it = xcd_item(b, nbh, nt);
        if (it < 0) { ++padding; continue; }
        ++items;
        if (it >= nbh * nt) { ++bad; continue; }
        seen[it]++;
        if (it <= last[b % 8]) ++bad;  // per XCD: the plain order's sequence
        last[b % 8] = it;
        const int r = it / nbh, h = it % nbh, P = (nt + 1) / 2;
        const int p = r < P ? r : nt - 1 - r, u = h * P + p;
        const XcdChunk c = xcd_chunk(b % 8, nbh, nt);
        if (u < c.q0 * c.P + c.r0 || u >= c.q1 * c.P + c.r1) ++bad;
      }
      for (int i = 0; i < nbh * nt; ++i) bad += seen[i] != 1;
    }
  printf("%ld %ld %ld %ld\n", cases, bad, items, padding);
  return 0;
}
"""


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_xcd_order_is_a_heaviest_first_bijection(tmp_path):
    src = tmp_path / "xcd_check.cpp"
    exe = tmp_path / "xcd_check"
    src.write_text(CHECKER)
    subprocess.run([HIPCC, "-std=c++17", "-O1", "-I", CSRC, str(src), "-o", str(exe)],
                   check=True, capture_output=True, timeout=300)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=120)
    cases, bad, items, padding = (int(x) for x in out.stdout.split())
    assert cases == 40 * 100
    assert bad == 0
    # every item once; a few padding blocks per case at most
    assert items == sum(n * t for n in range(1, 41) for t in range(1, 101))
    assert padding < 16 * cases
