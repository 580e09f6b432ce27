"""The memref-descriptor entry points (include/cleave_hip_memref.h), on the CPU:
descriptor parsing and layout checks happen on the host before any device
work, so every malformed call below is rejected without a GPU.  Data pointers
here are never dereferenced (validation fails first, or the call is empty)."""
from __future__ import annotations

import numpy as np
import pytest

FAKE = 0x100000  # a device address that validation never touches


@pytest.fixture(scope="module")
def mr():
    from cleave_amd import memref, _lib
    _lib.load()
    return memref


def _err(mr, fn, *args, match):
    from cleave_amd._lib import CleaveHipError
    with pytest.raises(CleaveHipError, match=match) as e:
        mr.call(fn, *args)
    assert e.value.code == -2  # argument error, not a runtime one


def _m(mr, sizes, strides=None):
    strides = mr.row_major_strides(sizes) if strides is None else strides
    return mr.MemRef(FAKE, sizes, strides)


def test_ranked_descriptor_layout_is_mlirs(mr):
    # { allocated, aligned, offset, sizes[r], strides[r] }: 8-byte fields in that order
    import ctypes as C
    d = _m(mr, [3, 5])
    words = (C.c_int64 * 7).from_address(C.addressof(d.ranked))
    assert list(words) == [FAKE, FAKE, 0, 3, 5, 5, 1]
    assert d.unranked.rank == 2 and d.unranked.descriptor == C.addressof(d.ranked)


def test_matmul_rejects_bad_layouts(mr):
    a, b, c = _m(mr, [4, 8]), _m(mr, [8, 6]), _m(mr, [4, 6])
    _err(mr, "cleave_hip_matmul_f32", _m(mr, [32]), b, c, match="rank 1, expected 2")
    _err(mr, "cleave_hip_matmul_f32", a, _m(mr, [7, 6]), c, match="do not chain")
    _err(mr, "cleave_hip_matmul_f32", a, b, _m(mr, [4, 7]), match="do not chain")
    # padded rows (leading stride 16 for 8 columns) are neither layout
    _err(mr, "cleave_hip_matmul_f32", _m(mr, [4, 8], [16, 1]), b, c, match="neither row-major nor transposed")
    # C must be row-major: a transposed output is rejected
    _err(mr, "cleave_hip_matmul_f32", a, b, _m(mr, [4, 6], [1, 4]), match="c must be row-major")
    _err(mr, "cleave_hip_matmul_f32", a, b, _m(mr, [1, 4, 6]), match="ranks differ")
    # batch entries must be packed back to back
    _err(mr, "cleave_hip_matmul_f32", _m(mr, [2, 4, 8], [64, 8, 1]), _m(mr, [2, 8, 6]), _m(mr, [2, 4, 6]),
         match="packed back to back")
    _err(mr, "cleave_hip_matmul_f32", None, b, c, match="null memref descriptor")


def test_elementwise_operands_need_equal_shapes_not_just_lengths(mr):
    a = _m(mr, [2, 3])
    _err(mr, "cleave_hip_add_f32", a, _m(mr, [3, 2]), _m(mr, [2, 3]), match="shape differs")
    _err(mr, "cleave_hip_sigmoid_f32", a, _m(mr, [6]), match="shape differs")
    _err(mr, "cleave_hip_mul_f32", a, _m(mr, [2, 3], [6, 2]), _m(mr, [2, 3]), match="not row-major contiguous")
    _err(mr, "cleave_hip_div_bwd_f32", a, a, a, a, _m(mr, [2, 4]), match="db: shape differs")


def test_index_and_mlp_shape_checks(mr):
    t = _m(mr, [3, 4, 5])
    # the tensor's rank fixes the index length; too short is rejected
    idx = mr.host(np.array([1, 2], np.int32))
    from cleave_amd import _lib
    assert np.isnan(mr.call("cleave_hip_index_f32", t, idx))
    assert "memref<3 x i32>" in _lib.last_error()[1]
    _err(mr, "cleave_hip_index_bwd_f32", 1.0, t, idx, match="memref<3 x i32>")
    x, y, w1, w2 = _m(mr, [8, 4]), _m(mr, [8]), _m(mr, [4, 16]), _m(mr, [16])
    _err(mr, "cleave_hip_mlp_step_f32", x, _m(mr, [7]), w1, w2, None, None, None, 0.1, match="expected x")
    _err(mr, "cleave_hip_mlp_step_f32", x, y, w1, w2, _m(mr, [16, 4]), None, None, 0.1, match="dw1: shape differs")
    _err(mr, "cleave_hip_mlp_step_f32", x, y, w1, w2, None, None, _m(mr, [2]), 0.1, match="loss must hold one")
    _err(mr, "cleave_hip_mandelbrot_u32", _m(mr, [16]), -2.0, -1.5, 0.1, 0.1, 100, match="height x width")


def test_empty_tensors_pass_validation_without_a_device(mr):
    # a well-formed descriptor over zero elements reaches the pointer form,
    # whose empty-map early return needs no device
    z = mr.MemRef(None, [0, 5], [5, 1])
    assert mr.call("cleave_hip_add_f32", z, z, z) == 0
    assert mr.call("cleave_hip_relu_f32", z, z) == 0
    assert mr.call("cleave_hip_zero_f32", z) == 0
