"""The split of a large host copy over threads (cleave_amd/csrc/copy_split.hpp,
used by the `_host` entry points' bounce-buffer copies in host.cpp): for every
length the ranges must cover every byte exactly once, start on 64-byte
boundaries, and stay inside the array.  Checked on the CPU by compiling the
header into a small C++ program; no GPU needed."""
from __future__ import annotations

import subprocess

from conftest import ROOT

CHECK = r"""
#include <cstdio>
#include "copy_split.hpp"

// Checks every 4-byte-multiple length in [lo, hi] for 1..8 threads with the
// 2 MiB least slice host.cpp uses.  Prints the first failure, or "ok N".
int main(int argc, char** argv) {
    const size_t lo = size_t(4) << 20, hi = size_t(16) << 20, slice = size_t(2) << 20;
    long long checked = 0;
    for (size_t threads = 1; threads <= 8; ++threads) {
        for (size_t n = lo; n <= hi; n += 4) {
            const ch::CopySplit s = ch::copy_split(n, threads, slice);
            if (s.parts < 1 || s.parts > threads) { printf("bad parts n=%zu t=%zu\n", n, threads); return 1; }
            size_t next = 0;
            for (size_t p = 0; p < s.parts; ++p) {
                size_t off, len;
                ch::copy_range(s, n, p, &off, &len);
                if (len == 0) continue;
                if (off != next || off % 64 != 0 || off + len > n) {
                    printf("bad range n=%zu t=%zu p=%zu off=%zu len=%zu next=%zu\n", n, threads, p, off, len, next);
                    return 1;
                }
                next = off + len;
            }
            if (next != n) { printf("uncovered n=%zu t=%zu covered=%zu\n", n, threads, next); return 1; }
            ++checked;
        }
    }
    // the length the old split dropped bytes at: 2,621,441 floats over 5 threads
    const size_t n = size_t(2621441) * 4;
    const ch::CopySplit s = ch::copy_split(n, 5, slice);
    size_t off, len;
    ch::copy_range(s, n, s.parts - 1, &off, &len);
    if (off + len != n) { printf("tail n=%zu ends at %zu\n", n, off + len); return 1; }
    printf("ok %lld\n", checked);
    return 0;
}
"""


def test_copy_split_covers_every_byte(tmp_path):
    src = tmp_path / "check.cpp"
    src.write_text(CHECK)
    exe = tmp_path / "check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", str(ROOT / "cleave_amd" / "csrc"), str(src), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0 and out.stdout.startswith("ok"), out.stdout + out.stderr
    assert int(out.stdout.split()[1]) == 8 * (((16 << 20) - (4 << 20)) // 4 + 1)
