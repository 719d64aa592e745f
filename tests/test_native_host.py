"""Host-only checks of libmk's native helpers, compiled with the system C++
compiler (no GPU): the per-device "done once" flag that guards the
dynamic-LDS kernel attribute (mkernel_amd/csrc/mk_once.h)."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent

PROG = r"""
#include <cstdio>
#include <thread>
#include <vector>
#include "mk_once.h"
int main() {
  mk::PerDeviceFlag f;
  // every device starts clear, and setting one leaves the others clear
  for (int d : {0, 1, 7, 63, 64, 65, 200}) if (f.is_set(d)) return 1;
  f.set(1);
  if (!f.is_set(1) || f.is_set(0) || f.is_set(2)) return 2;
  f.set(70);
  if (!f.is_set(70) || f.is_set(69) || f.is_set(71) || f.is_set(6)) return 3;
  if (f.is_set(-1)) return 4;
  f.set(-1);  // ignored
  // concurrent setters on distinct devices: every bit lands
  mk::PerDeviceFlag g;
  std::vector<std::thread> ts;
  for (int d = 0; d < 96; ++d) ts.emplace_back([&g, d] { g.set(d); });
  for (auto& t : ts) t.join();
  for (int d = 0; d < 96; ++d) if (!g.is_set(d)) return 5;
  if (g.is_set(96)) return 6;
  std::puts("ok");
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="no host C++ compiler")
def test_per_device_flag(tmp_path):
    src = tmp_path / "once_test.cpp"
    src.write_text(PROG)
    exe = tmp_path / "once_test"
    subprocess.run(["g++", "-std=c++17", "-O1", "-pthread", "-I", str(ROOT / "mkernel_amd" / "csrc"), str(src),
                    "-o", str(exe)], check=True, capture_output=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True)
    assert res.returncode == 0 and res.stdout.strip() == "ok", (res.returncode, res.stdout, res.stderr)
