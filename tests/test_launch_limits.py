"""The launch-shape arithmetic every launcher uses (chelis_amd/csrc/
launch_limits.h), compiled on the host: HIP's 2^32 work-item bound per grid
dimension, and the saturating block count."""
import os
import subprocess
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = r"""
#include "launch_limits.h"
#include <cstdio>
int main() {
    using chelis::grid_fits;
    using chelis::grid_for;
    int bad = 0;
    // 2^24 - 1 blocks of 256 threads is the largest grid below 2^32 items
    bad |= !grid_fits(16777215, 256) << 0;
    bad |= grid_fits(16777216, 256) << 1;
    bad |= !grid_fits(0, 256) << 2;
    bad |= grid_fits(1, 0) << 3;
    bad |= grid_fits(-1, 64) << 4;
    bad |= !grid_fits(4294967295LL, 1) << 5;
    bad |= grid_fits(4294967296LL, 1) << 6;
    // a sum over axis 1 of an f32 [1e8, 8] tensor: 2.5e7 blocks of 256 threads
    bad |= grid_fits(grid_for(100000000LL, 4), 256) << 7;
    bad |= (grid_for(0, 256) != 1u) << 8;
    bad |= (grid_for(257, 256) != 2u) << 9;
    bad |= (grid_for(int64_t(1) << 40, 1) != 0xffffffffu) << 10;
    bad |= grid_fits(grid_for(int64_t(1) << 40, 1), 2) << 11;
    std::printf("%d\n", bad);
    return bad != 0;
}
"""


def test_grid_limits_on_the_host():
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "t.cpp"), os.path.join(d, "t")
        open(src, "w").write(SRC)
        r = subprocess.run(["g++", "-std=c++17", "-I" + os.path.join(ROOT, "chelis_amd", "csrc"), src, "-o", exe],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
        out = subprocess.run([exe], capture_output=True, text=True)
        assert out.returncode == 0 and out.stdout.strip() == "0", out.stdout
