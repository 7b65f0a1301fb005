"""The kernels' query-row clamp (csrc/query_rows.h), built for the host with g++ from the
same header the HIP kernels include, checked exhaustively on small ranges: whatever
query_start_loc holds, every row a sequence is given lies inside [0, num_tokens)."""

from __future__ import annotations

import pathlib
import subprocess

import pytest

HEADER = pathlib.Path(__file__).resolve().parents[1] / "sglang_restomod_amd" / "csrc" / "query_rows.h"

PROGRAM = r"""
#include <cstdio>
#include "query_rows.h"
int main() {
  long checked = 0, bad = 0;
  for (int n = -2; n <= 12; ++n)
    for (int start = -5; start <= 16; ++start)
      for (int end = -5; end <= 16; ++end) {
        const ma::QueryRows r = ma::clamp_query_rows(start, end, n);
        const int cap = n < 0 ? 0 : n;
        ++checked;
        // inside the buffers, never negative
        if (r.ntok < 0 || r.tok0 < 0 || r.tok0 + r.ntok > cap) ++bad;
        // consistent metadata inside the buffers is kept as it is
        if (start >= 0 && start <= end && end <= cap && (r.tok0 != start || r.ntok != end - start)) ++bad;
        // a range cut by the buffer end keeps its start and loses only rows past the end
        if (start >= 0 && start <= cap && end > cap && (r.tok0 != start || r.ntok != cap - start)) ++bad;
        // a decreasing range is empty
        if (end <= start && r.ntok != 0) ++bad;
      }
  std::printf("%ld %ld\n", checked, bad);
  return bad ? 1 : 0;
}
"""


def test_clamp_keeps_every_row_inside_the_buffers(tmp_path):
    src = tmp_path / "t.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "t"
    build = subprocess.run(["g++", "-std=c++17", "-O1", f"-I{HEADER.parent}", str(src), "-o", str(exe)],
                           capture_output=True, text=True)
    if build.returncode != 0:
        pytest.fail(build.stderr)
    run = subprocess.run([str(exe)], capture_output=True, text=True)
    checked, bad = map(int, run.stdout.split())
    assert checked == 15 * 22 * 22 and bad == 0, run.stdout
