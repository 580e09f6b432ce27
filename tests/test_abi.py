"""The drop-in boundary: libcleave_hip.so loads, exports exactly the C ABI of
include/cleave_hip.h, registers it in its symbol table (the shape of
register_cleave_rt_symbols, /root/reference/cleave/src/pipeline.rs:159-198),
and validates arguments on the host before touching a device.  No GPU needed.
"""
from __future__ import annotations

import ctypes as C
import re
import subprocess
from pathlib import Path
import sys

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "cleave_hip.h"
HEADERS = [HEADER, ROOT / "include" / "cleave_hip_memref.h"]


def header_functions() -> list[str]:
    names = []
    for h in HEADERS:
        names += re.findall(r"^CLEAVE_HIP_API [^(]*?\b((?:_mlir_ciface_)?cleave_hip_[a-z0-9_]+)\(", h.read_text(), re.M)
    return list(dict.fromkeys(names))


def test_header_declares_the_expected_surface():
    names = header_functions()
    assert len(names) >= 40
    for must in ["cleave_hip_matmul_f32", "cleave_hip_matmul_bf16", "cleave_hip_matmul_batched_bf16",
                 "cleave_hip_sigmoid_f32", "cleave_hip_sum_f32", "cleave_hip_mandelbrot_u32",
                 "cleave_hip_mlp_step_f32", "cleave_hip_symbols", "cleave_hip_buf_alloc"]:
        assert must in names


def test_library_exports_every_declared_symbol_and_nothing_else():
    from cleave_amd import _lib

    lib = _lib.load()
    for name in header_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert exported == set(header_functions())


def test_static_archive_defines_every_declared_symbol():
    from cleave_amd import build

    assert build.ARCHIVE.exists(), "libcleave_hip.a is built beside the shared library"
    out = subprocess.run(["nm", "--defined-only", str(build.ARCHIVE)], capture_output=True,
                         text=True, check=True).stdout
    defined = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert set(header_functions()) <= defined


def test_static_archive_links_into_a_host_program(tmp_path):
    # the AOT path: a C host links libcleave_hip.a (plus the HIP runtime) and
    # walks the symbol table, with or without a visible device
    from cleave_amd import build

    hipcc = Path(build.HIPCC)
    if not hipcc.exists():
        pytest.skip("hipcc not installed")
    src = tmp_path / "host.c"
    src.write_text(
        "#include <stdio.h>\n#include <string.h>\n#include \"cleave_hip.h\"\n"
        "int main(void) {\n"
        "  int64_t n = 0;\n"
        "  const cleave_hip_symbol* t = cleave_hip_symbols(&n);\n"
        "  int found = 0;\n"
        "  for (int64_t i = 0; i < n; ++i)\n"
        "    if (!strcmp(t[i].name, \"cleave_hip_matmul_f32\") && t[i].fn == (void*)cleave_hip_matmul_f32) found = 1;\n"
        "  printf(\"%lld %d %d\\n\", (long long)n, found, (int)cleave_hip_device_available());\n"
        "  return 0;\n"
        "}\n")
    obj, exe = tmp_path / "host.o", tmp_path / "host"
    subprocess.run(["gcc", "-c", "-I", str(ROOT / "include"), str(src), "-o", str(obj)], check=True)
    subprocess.run([str(hipcc), "--offload-arch=gfx950", str(obj), str(build.ARCHIVE), "-o", str(exe)],
                   check=True, capture_output=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True, timeout=60).stdout.split()
    assert int(out[0]) == len(header_functions()) and out[1] == "1" and out[2] in ("0", "1")


def test_symbol_table_matches_header_and_addresses():
    from cleave_amd import _lib

    lib = _lib.load()
    table = _lib.symbol_table()
    assert set(table) == set(header_functions())
    for name, addr in table.items():
        assert addr == C.cast(getattr(lib, name), C.c_void_p).value, name


def test_python_signatures_cover_the_header():
    from cleave_amd import _lib

    assert set(_lib.SIGNATURES) == set(header_functions())


def test_integration_rust_binding_declares_every_c_function_with_its_arity():
    # The FFI stub a cleave maintainer would copy must stay in step with the header.
    text = (ROOT / "INTEGRATION.md").read_text()
    block = text[text.index("unsafe extern \"C\" {"):]
    block = block[:block.index("\n}\n")]
    rust = {m.group(1): m.group(2) for m in re.finditer(r"pub fn (cleave_hip_\w+)\(([^)]*)\)", block, re.S)}
    src = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    c = {m.group(1): m.group(2) for m in re.finditer(r"^CLEAVE_HIP_API [^(]*?\b(cleave_hip_\w+)\(([^)]*)\);", src, re.M | re.S)}
    assert set(rust) == set(c)

    def arity(params: str) -> int:
        params = " ".join(params.split())
        return 0 if params in ("", "void") else params.count(",") + 1

    for name in c:
        assert arity(rust[name]) == arity(c[name]), name


def _lib_noabort():
    from cleave_amd import _lib

    lib = _lib.load()
    lib.cleave_hip_set_abort_on_error(0)
    return lib, _lib


@pytest.mark.parametrize("fn,args,needle", [
    ("cleave_hip_matmul_f32", (None, 5, None, 4, None, 4, 2, 2, 2, 0, 0), "alen"),
    ("cleave_hip_matmul_f32", (None, 4, None, 4, None, 4, 2, 2, 2, 2, 0), "trans"),
    ("cleave_hip_matmul_f32", (None, 0, None, 0, None, 0, 0, 2, 2, 0, 0), "positive"),
    ("cleave_hip_matmul_bf16", (None, 4, None, 6, None, 4, 2, 2, 2, 0, 0), "blen"),
    ("cleave_hip_matmul_batched_bf16", (None, 8, None, 8, None, 7, 2, 2, 2, 2, 0, 0), "lengths"),
    ("cleave_hip_matmul_batched_bf16", (None, 8, None, 8, None, 8, 2, 2, 2, 2, 0, 3), "trans"),
    ("cleave_hip_matmul_batched_f32", (None, 8, None, 8, None, 8, 0, 2, 2, 2, 0, 0), "batch"),
    # batch * M * K = 2^64: refused, not wrapped to lengths of 0
    ("cleave_hip_matmul_batched_f64", (None, 0, None, 0, None, 0, 16, 1 << 30, 1 << 30, 1 << 30, 0, 0), "lengths"),
    ("cleave_hip_matmul_batched_f32", (None, 0, None, 0, None, 0, 65535, 2147483647, 2147483647, 2147483647, 0, 0),
     "lengths"),
    ("cleave_hip_add_f32", (None, 3, None, 4, None, 3), "broadcast"),
    ("cleave_hip_sigmoid_f32", (None, 3, None, 2, ), "length"),
    ("cleave_hip_sgd_update_f32", (None, 3, None, 2, 0.1), "glen"),
    ("cleave_hip_reduce_sum_f32", (None, 0, None), ">= 1"),
    ("cleave_hip_reduce_max_f32", (None, 0, None, None), ">= 1"),
    ("cleave_hip_mandelbrot_u32", (None, 10, 4, 4, -2.0, -1.5, 0.1, 0.1, 10), "outlen"),
    ("cleave_hip_mandelbrot_u32", (None, 16, 4, 4, -2.0, -1.5, 0.1, 0.1, -1), "max_iter"),
    ("cleave_hip_mlp_step_f32", (None, 9, None, 2, None, 15, None, 3, None, 0, None, 0, None,
                                 2, 5, 3, 0.01), "xlen"),
    ("cleave_hip_cast_f32_bf16", (None, 4, None, 3), "null"),
])
def test_argument_validation_happens_before_any_device_work(fn, args, needle):
    lib, _lib = _lib_noabort()
    status = getattr(lib, fn)(*args)
    code, msg = _lib.last_error()
    assert status == _lib.ERR_ARG and code == _lib.ERR_ARG
    assert fn in msg and needle in msg, msg


def test_broadcast_shapes_and_lengths_are_checked_before_any_device_work():
    import numpy as np

    lib, _lib = _lib_noabort()
    big = np.array([65536] * 4, np.int32)  # 2^64 elements: past int64, refused rather than wrapped to 0
    one = np.array([1], np.int32)
    cases = [
        (lib.cleave_hip_add_bcast_f32, (None, 0, big.ctypes.data, 4, None, 1, one.ctypes.data, 1, None, 0),
         "do not match"),
        (lib.cleave_hip_mul_bcast_f64, (None, -1, one.ctypes.data, 1, None, 1, one.ctypes.data, 1, None, 1),
         "negative length"),
        (lib.cleave_hip_sum_to_shape_f32, (None, 0, big.ctypes.data, 4, None, 1, one.ctypes.data, 1),
         "do not match"),
        (lib.cleave_hip_sum_to_shape_f64, (None, 1, one.ctypes.data, 1, None, -1, one.ctypes.data, 1),
         "negative length"),
    ]
    for fn, args, needle in cases:
        assert fn(*args) == _lib.ERR_ARG
        code, msg = _lib.last_error()
        assert code == _lib.ERR_ARG and needle in msg, msg


def test_zero_length_maps_are_no_ops_without_a_device():
    lib, _lib = _lib_noabort()
    assert lib.cleave_hip_add_f32(None, 0, None, 0, None, 0) == 0
    assert lib.cleave_hip_neg_f32(None, 0, None, 0) == 0
    assert lib.cleave_hip_zero_f32(None, 0) == 0


def test_missing_device_is_a_runtime_error_not_a_fallback():
    lib, _lib = _lib_noabort()
    if lib.cleave_hip_device_available():
        pytest.skip("a device is present; this checks the no-device path")
    assert lib.cleave_hip_init() == _lib.ERR_RUNTIME
    assert lib.cleave_hip_matmul_f32(1, 4, 1, 4, 1, 4, 2, 2, 2, 0, 0) == _lib.ERR_RUNTIME
    assert lib.cleave_hip_buf_alloc(64) is None
    assert "device" in _lib.last_error()[1]


def test_default_error_mode_aborts_like_cleave_rt():
    # cleave-rt panics on bad input (cleave-rt/src/lib.rs:69, :120); by default
    # the library prints the message and aborts.
    code = (
        "import ctypes, sys; L = ctypes.CDLL(sys.argv[1]);"
        "L.cleave_hip_add_f32.argtypes = [ctypes.c_void_p, ctypes.c_int64] * 3;"
        "L.cleave_hip_add_f32(None, 3, None, 4, None, 3)"
    )
    from cleave_amd import _lib

    r = subprocess.run([sys.executable, "-c", code, str(_lib.LIB_PATH)], capture_output=True, text=True)
    assert r.returncode != 0
    assert "cleave_hip: error -2: cleave_hip_add_f32" in r.stderr


def test_product_package_does_not_reach_the_oracle():
    # The product path must never import, link or load the checker.
    for path in (ROOT / "cleave_amd").rglob("*"):
        if path.suffix in {".py", ".hip", ".cpp", ".hpp", ".h"}:
            text = path.read_text()
            assert "liboracle" not in text and "from oracle" not in text and "import oracle" not in text, path
    out = subprocess.run(["ldd", str(ROOT / "cleave_amd" / "libcleave_hip.so")], capture_output=True,
                         text=True).stdout
    assert "oracle" not in out


def test_index_bounds_and_rank_are_checked_on_the_host():
    # Index<Tensor>::index (stdlib/linalg/tensor.cleave:113-133): a bad index
    # is an argument error before any device work, so a placeholder (never
    # dereferenced) device pointer is enough here.
    import numpy as np

    from cleave_amd import _lib

    lib = _lib.load()
    fake = 4096
    dims = np.array([2, 3], np.int32)
    cases = [
        (np.array([1, 3], np.int32), 6, "out of range"),
        (np.array([-1, 0], np.int32), 6, "out of range"),
        (np.array([1], np.int32), 6, "indices for a rank-2"),
        (np.array([1, 1], np.int32), 7, "dims describe 6 elements"),
    ]
    for idx, length, needle in cases:
        st = lib.cleave_hip_index_bwd_f32(1.0, fake, length, dims.ctypes.data, dims.size,
                                          idx.ctypes.data, idx.size)
        code, msg = _lib.last_error()
        assert st == _lib.ERR_ARG and needle in msg, (idx, msg)
        v = lib.cleave_hip_index_f32(fake, length, dims.ctypes.data, dims.size, idx.ctypes.data, idx.size)
        code, msg = _lib.last_error()
        assert v != v and code == _lib.ERR_ARG and needle in msg, (idx, msg)
