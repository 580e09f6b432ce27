"""Build recipe for libcleave_hip.so and libcleave_hip.a (gfx950).

Each HIP source compiles to an object under cleave_amd/_build/ in parallel,
then one `hipcc -shared` link produces cleave_amd/libcleave_hip.so (in-tree,
so it travels with the source tree to the GPU box), and `ar` packs the same
objects into cleave_amd/libcleave_hip.a for hosts that link statically (the
counterpart of cleave-rt's staticlib crate type, cleave-rt/Cargo.toml:15-16;
the final link needs hipcc or -lamdhip64).

Flags:
  --offload-arch=gfx950          MI355X only, no other targets
  -ffp-contract=off              no implicit mul+add fusion: every f32 op rounds
                                 where the reference's scalar loops round
  -target-feature -packed-fp32-ops
                                 keep the compiler from emitting packed FP32 ops
  -fvisibility=hidden            only the extern "C" ABI (marked default) is exported

Every compile also asks for the kernel resource report; a kernel that uses
scratch memory (private arrays or register spills, a silent 10x slowdown for
the GEMMs) fails the build.
"""
from __future__ import annotations

import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libcleave_hip.so"
ARCHIVE = PKG / "libcleave_hip.a"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-fvisibility=hidden",
]
SOURCES = ["runtime.hip", "gemm_f32.hip", "gemm_bf16.hip", "gemm_f64.hip", "gemv.hip", "elementwise.hip", "reduce.hip",
           "mandelbrot.hip", "mlp.hip", "index.hip", "broadcast.hip", "memref.cpp",
           "host.cpp", "symbols.cpp"]


REPORT = "-Rpass-analysis=kernel-resource-usage"


def scratch_users(text: str) -> list[str]:
    """Kernels with a non-zero ScratchSize in a kernel-resource-usage report."""
    bad, name = [], None
    for line in text.splitlines():
        m = re.search(r"remark:\s+Function Name: (\S+)", line)
        if m:
            name = m.group(1)
        m = re.search(r"remark:\s+ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and int(m.group(1)) > 0:
            bad.append(f"{name}: {m.group(1)} bytes/lane")
    return bad


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {cmd[-1]}")
    out = r.stdout + r.stderr
    bad = scratch_users(out)
    if bad:
        raise RuntimeError("kernels use scratch memory (spills or private arrays):\n  " + "\n  ".join(bad))
    # The host pass does not know the packed-fp32 target feature; drop that
    # noise and the resource report itself.
    noise = ("'-packed-fp32-ops' is not a recognized feature", "remark:", "kernel-resource-usage",
             "In file included from", "|", "^")
    msgs = [l for l in out.splitlines() if l.strip() and not any(n in l for n in noise)
            and not l.strip()[:1].isdigit()]
    if msgs:
        sys.stderr.write("\n".join(msgs) + "\n")


def build_library(jobs: int = 8) -> Path:
    BUILD.mkdir(exist_ok=True)

    def compile_one(src: str) -> Path:
        obj = BUILD / (src.rsplit(".", 1)[0] + ".o")
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        report = [REPORT] if src.endswith(".hip") else []
        _run([HIPCC, *HIP_FLAGS, *report, *lang, "-c", str(CSRC / src), "-o", str(obj)])
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    atmp = ARCHIVE.with_suffix(".a.tmp")
    if atmp.exists():
        atmp.unlink()
    _run(["ar", "rcs", str(atmp), *map(str, objs)])
    os.replace(atmp, ARCHIVE)
    return LIB


def main() -> None:
    print("built", build_library())


if __name__ == "__main__":
    main()
