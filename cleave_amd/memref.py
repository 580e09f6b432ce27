"""MLIR memref descriptors for the `_mlir_ciface_cleave_hip_*` entry points
(include/cleave_hip_memref.h).

A ranked memref<d0 x .. x T> is passed as {allocated, aligned, offset,
sizes[rank], strides[rank]} and an unranked memref<* x T> as {rank, pointer to
the ranked descriptor}: MLIR's C-compatible wrapper ABI, what a lowering that
declares its externs with `llvm.emit_c_interface` passes.  This module builds
those structures over device tensors (and host index arrays) so the entry
points can be called and tested from Python.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib

_RANKED: dict[int, type] = {}


def ranked_type(rank: int) -> type:
    """ctypes structure of a ranked descriptor of the given rank."""
    if rank not in _RANKED:
        fields = [("allocated", C.c_void_p), ("aligned", C.c_void_p), ("offset", C.c_int64)]
        if rank:
            fields += [("sizes", C.c_int64 * rank), ("strides", C.c_int64 * rank)]
        _RANKED[rank] = type(f"MemRef{rank}D", (C.Structure,), {"_fields_": fields})
    return _RANKED[rank]


class Unranked(C.Structure):
    _fields_ = [("rank", C.c_int64), ("descriptor", C.c_void_p)]


class MemRef:
    """An unranked descriptor plus the ranked one it points at (kept alive together)."""

    def __init__(self, ptr: int | None, sizes, strides, offset: int = 0, keep=None):
        sizes, strides = [int(s) for s in sizes], [int(s) for s in strides]
        if len(sizes) != len(strides):
            raise ValueError("sizes and strides differ in rank")
        rank = len(sizes)
        self.ranked = ranked_type(rank)()
        self.ranked.allocated = ptr
        self.ranked.aligned = ptr
        self.ranked.offset = offset
        for i in range(rank):
            self.ranked.sizes[i] = sizes[i]
            self.ranked.strides[i] = strides[i]
        self.unranked = Unranked(rank, C.cast(C.pointer(self.ranked), C.c_void_p))
        self._keep = keep

    @property
    def ref(self) -> C.c_void_p:
        """Pointer to the unranked descriptor, the argument the entry points take."""
        return C.cast(C.pointer(self.unranked), C.c_void_p)


def row_major_strides(shape) -> list[int]:
    strides, acc = [], 1
    for n in reversed(list(shape)):
        strides.append(acc)
        acc *= int(n)
    return strides[::-1]


def of(t, shape=None) -> MemRef:
    """Row-major descriptor over a device tensor (optionally viewed with another shape)."""
    shape = list(t.shape if shape is None else shape)
    if int(np.prod(shape, dtype=np.int64)) != t.size:
        raise ValueError(f"shape {shape} does not cover {t.size} elements")
    return MemRef(t.ptr, shape, row_major_strides(shape), keep=t)


def transposed(t, shape=None) -> MemRef:
    """The transpose of a row-major [.., R x C] device tensor, as the [.., C x R]
    view with strides {.., 1, C}: what memref.transpose hands over, no copy."""
    shape = list(t.shape if shape is None else shape)
    if len(shape) not in (2, 3):
        raise ValueError("transposed views are 2-D or batched 2-D")
    st = row_major_strides(shape)
    sizes = shape[:-2] + [shape[-1], shape[-2]]
    strides = st[:-2] + [1, shape[-1]]
    return MemRef(t.ptr, sizes, strides, keep=t)


def host(a: np.ndarray) -> MemRef:
    """Descriptor over a contiguous host array (index arrays are host memory)."""
    a = np.ascontiguousarray(a)
    return MemRef(a.ctypes.data, a.shape, [s // a.itemsize for s in a.strides], keep=a)


def call(name: str, *args):
    """Call `_mlir_ciface_<name>`; MemRef arguments are passed by descriptor
    pointer, None as a null descriptor, anything else as is."""
    conv = [a.ref if isinstance(a, MemRef) else a for a in args]
    return _lib.call("_mlir_ciface_" + name, *conv)
