"""ctypes binding of libcleave_hip.so (the C ABI declared in include/cleave_hip.h
and, for the memref-descriptor forms, include/cleave_hip_memref.h).

This is the reference-side binding a host would add (the Python equivalent of
the `extern(symbol) fn ...` declarations of /root/reference/stdlib/io/io.cleave:16-21):
every function gets explicit argtypes/restype, the library's abort-on-error
mode is switched off, and a negative status becomes a CleaveHipError.

The library is loaded from this package directory (or, for comparing two
builds, from the path in CLEAVE_HIP_LIBRARY).  If it has not been built,
import fails loudly -- there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("CLEAVE_HIP_LIBRARY") or (Path(__file__).resolve().parent / "libcleave_hip.so"))

OK, ERR_RUNTIME, ERR_ARG, ERR_OOM = 0, -1, -2, -3


class CleaveHipError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"cleave_hip error {code}: {message}")
        self.code = code


f32p = C.POINTER(C.c_float)
u16p = C.POINTER(C.c_uint16)
u32p = C.POINTER(C.c_uint32)
u64p = C.POINTER(C.c_uint64)
i64p = C.POINTER(C.c_int64)
vp = C.c_void_p
i32, i64, u64, f32, f64 = C.c_int32, C.c_int64, C.c_uint64, C.c_float, C.c_double


class Symbol(C.Structure):
    _fields_ = [("name", C.c_char_p), ("fn", C.c_void_p)]


# name -> (restype, argtypes).  Device pointers are passed as c_void_p.
SIGNATURES: dict[str, tuple] = {
    "cleave_hip_init": (i32, []),
    "cleave_hip_device_available": (i32, []),
    "cleave_hip_buf_alloc": (vp, [i64]),
    "cleave_hip_buf_free": (None, [vp]),
    "cleave_hip_buf_trim": (i64, []),
    "cleave_hip_buf_cached_bytes": (i64, []),
    "cleave_hip_upload": (i64, [vp, vp, i64]),
    "cleave_hip_download": (i64, [vp, vp, i64]),
    "cleave_hip_sync": (i32, []),
    "cleave_hip_set_abort_on_error": (None, [i32]),
    "cleave_hip_last_error": (i32, []),
    "cleave_hip_last_error_message": (C.c_char_p, []),
    "cleave_hip_event_create": (vp, []),
    "cleave_hip_event_record": (i32, [vp]),
    "cleave_hip_event_elapsed_ms": (f32, [vp, vp]),
    "cleave_hip_event_destroy": (None, [vp]),
    "cleave_hip_symbols": (C.POINTER(Symbol), [i64p]),
    "cleave_hip_fill_uniform_f32": (i32, [vp, i64, u64, f32, f32]),
    "cleave_hip_fill_normal_f32": (i32, [vp, i64, u64, f32, f32]),
    "cleave_hip_fill_bernoulli_f32": (i32, [vp, i64, u64, f32]),
    "cleave_hip_cast_f32_bf16": (i32, [vp, i64, vp, i64]),
    "cleave_hip_matmul_f32": (i32, [vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, i32]),
    "cleave_hip_matmul_batched_f32": (i32, [vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, i32, i32]),
    "cleave_hip_matmul_bf16": (i32, [vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, i32]),
    "cleave_hip_matmul_batched_bf16": (i32, [vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, i32, i32]),
    "cleave_hip_add_f32": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_sub_f32": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_mul_f32": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_div_f32": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_neg_f32": (i32, [vp, i64, vp, i64]),
    "cleave_hip_zero_f32": (i32, [vp, i64]),
    "cleave_hip_relu_f32": (i32, [vp, i64, vp, i64]),
    "cleave_hip_sigmoid_f32": (i32, [vp, i64, vp, i64]),
    "cleave_hip_tanh_f32": (i32, [vp, i64, vp, i64]),
    "cleave_hip_sigmoid_bwd_f32": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_tanh_bwd_f32": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_relu_bwd_f32": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_div_bwd_f32": (i32, [vp, i64, vp, i64, vp, i64, vp, i64, vp, i64]),
    "cleave_hip_sgd_update_f32": (i32, [vp, i64, vp, i64, f32]),
    "cleave_hip_add_row_bias_f32": (i32, [vp, i64, vp, i64, vp, i64, i32, i32]),
    "cleave_hip_sum_rows_f32": (i32, [vp, i64, vp, i64, i32, i32]),
    "cleave_hip_reduce_sum_f32": (i32, [vp, i64, vp]),
    "cleave_hip_reduce_max_f32": (i32, [vp, i64, vp, vp]),
    "cleave_hip_reduce_sum_u32_u64": (i32, [vp, i64, vp]),
    "cleave_hip_reduce_sum_f32_noalloc": (i32, [vp, i64, vp]),
    "cleave_hip_sum_f32": (f32, [vp, i64]),
    "cleave_hip_mean_f32": (f32, [vp, i64]),
    "cleave_hip_max_of_f32": (f32, [vp, i64]),
    "cleave_hip_argmax_f32": (i64, [vp, i64]),
    "cleave_hip_sum_u32_u64": (u64, [vp, i64]),
    "cleave_hip_index_f32": (f32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_index_bwd_f32": (i32, [f32, vp, i64, vp, i64, vp, i64]),
    "cleave_hip_mandelbrot_u32": (i32, [vp, i64, i32, i32, f32, f32, f32, f32, i32]),
    "cleave_hip_mlp_step_f32": (i32, [vp, i64, vp, i64, vp, i64, vp, i64, vp, i64, vp, i64,
                                      vp, i32, i32, i32, f32]),
    # host-array forms: the device form's signature, every tensor operand a host array
    "cleave_hip_matmul_f32_host": (i32, [vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, i32]),
    "cleave_hip_matmul_batched_f32_host": (i32, [vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, i32, i32]),
    "cleave_hip_matmul_bf16_host": (i32, [vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, i32]),
    "cleave_hip_matmul_batched_bf16_host": (i32, [vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, i32, i32]),
    "cleave_hip_add_f32_host": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_sub_f32_host": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_mul_f32_host": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_div_f32_host": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_neg_f32_host": (i32, [vp, i64, vp, i64]),
    "cleave_hip_zero_f32_host": (i32, [vp, i64]),
    "cleave_hip_relu_f32_host": (i32, [vp, i64, vp, i64]),
    "cleave_hip_sigmoid_f32_host": (i32, [vp, i64, vp, i64]),
    "cleave_hip_tanh_f32_host": (i32, [vp, i64, vp, i64]),
    "cleave_hip_sigmoid_bwd_f32_host": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_tanh_bwd_f32_host": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_relu_bwd_f32_host": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_div_bwd_f32_host": (i32, [vp, i64, vp, i64, vp, i64, vp, i64, vp, i64]),
    "cleave_hip_sgd_update_f32_host": (i32, [vp, i64, vp, i64, f32]),
    "cleave_hip_add_row_bias_f32_host": (i32, [vp, i64, vp, i64, vp, i64, i32, i32]),
    "cleave_hip_sum_rows_f32_host": (i32, [vp, i64, vp, i64, i32, i32]),
    "cleave_hip_sum_f32_host": (f32, [vp, i64]),
    "cleave_hip_mean_f32_host": (f32, [vp, i64]),
    "cleave_hip_max_of_f32_host": (f32, [vp, i64]),
    "cleave_hip_argmax_f32_host": (i64, [vp, i64]),
    "cleave_hip_sum_u32_u64_host": (u64, [vp, i64]),
    "cleave_hip_index_f32_host": (f32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_index_bwd_f32_host": (i32, [f32, vp, i64, vp, i64, vp, i64]),
    "cleave_hip_mandelbrot_u32_host": (i32, [vp, i64, i32, i32, f32, f32, f32, f32, i32]),
    "cleave_hip_mlp_step_f32_host": (i32, [vp, i64, vp, i64, vp, i64, vp, i64, vp, i64, vp, i64,
                                           vp, i32, i32, i32, f32]),
    "cleave_hip_reduce_sum_i32_i64": (i32, [vp, i64, vp]),
    "cleave_hip_sum_i32_i64": (i64, [vp, i64]),
    "cleave_hip_sum_i32_i64_host": (i64, [vp, i64]),
    "cleave_hip_matmul_f32_into": (i64, [vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, i32]),
    "cleave_hip_add_f32_into": (i64, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_sub_f32_into": (i64, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_mul_f32_into": (i64, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_div_f32_into": (i64, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_neg_f32_into": (i64, [vp, i64, vp, i64]),
    "cleave_hip_relu_f32_into": (i64, [vp, i64, vp, i64]),
    "cleave_hip_sigmoid_f32_into": (i64, [vp, i64, vp, i64]),
    "cleave_hip_tanh_f32_into": (i64, [vp, i64, vp, i64]),
    "cleave_hip_sigmoid_bwd_f32_into": (i64, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_tanh_bwd_f32_into": (i64, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_relu_bwd_f32_into": (i64, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_escape_grid_i32": (i64, [vp, i64, i32, i32, f32, f32, f32, f32, i32]),
    "cleave_hip_matmul_f64": (i32, [vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, i32]),
    "cleave_hip_matmul_batched_f64": (i32, [vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, i32, i32]),
    "cleave_hip_add_f64": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_sub_f64": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_mul_f64": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_div_f64": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_neg_f64": (i32, [vp, i64, vp, i64]),
    "cleave_hip_zero_f64": (i32, [vp, i64]),
    "cleave_hip_relu_f64": (i32, [vp, i64, vp, i64]),
    "cleave_hip_sigmoid_f64": (i32, [vp, i64, vp, i64]),
    "cleave_hip_tanh_f64": (i32, [vp, i64, vp, i64]),
    "cleave_hip_sigmoid_bwd_f64": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_tanh_bwd_f64": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_relu_bwd_f64": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_div_bwd_f64": (i32, [vp, i64, vp, i64, vp, i64, vp, i64, vp, i64]),
    "cleave_hip_sgd_update_f64": (i32, [vp, i64, vp, i64, f64]),
    "cleave_hip_add_row_bias_f64": (i32, [vp, i64, vp, i64, vp, i64, i32, i32]),
    "cleave_hip_sum_rows_f64": (i32, [vp, i64, vp, i64, i32, i32]),
    "cleave_hip_reduce_sum_f64": (i32, [vp, i64, vp]),
    "cleave_hip_reduce_max_f64": (i32, [vp, i64, vp, vp]),
    "cleave_hip_sum_f64": (f64, [vp, i64]),
    "cleave_hip_mean_f64": (f64, [vp, i64]),
    "cleave_hip_max_of_f64": (f64, [vp, i64]),
    "cleave_hip_argmax_f64": (i64, [vp, i64]),
    "cleave_hip_index_f64": (f64, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_index_bwd_f64": (i32, [f64, vp, i64, vp, i64, vp, i64]),
    "cleave_hip_matmul_f64_host": (i32, [vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, i32]),
    "cleave_hip_matmul_batched_f64_host": (i32, [vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, i32, i32]),
    "cleave_hip_add_f64_host": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_sub_f64_host": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_mul_f64_host": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_div_f64_host": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_neg_f64_host": (i32, [vp, i64, vp, i64]),
    "cleave_hip_zero_f64_host": (i32, [vp, i64]),
    "cleave_hip_relu_f64_host": (i32, [vp, i64, vp, i64]),
    "cleave_hip_sigmoid_f64_host": (i32, [vp, i64, vp, i64]),
    "cleave_hip_tanh_f64_host": (i32, [vp, i64, vp, i64]),
    "cleave_hip_sigmoid_bwd_f64_host": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_tanh_bwd_f64_host": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_relu_bwd_f64_host": (i32, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_div_bwd_f64_host": (i32, [vp, i64, vp, i64, vp, i64, vp, i64, vp, i64]),
    "cleave_hip_sgd_update_f64_host": (i32, [vp, i64, vp, i64, f64]),
    "cleave_hip_add_row_bias_f64_host": (i32, [vp, i64, vp, i64, vp, i64, i32, i32]),
    "cleave_hip_sum_rows_f64_host": (i32, [vp, i64, vp, i64, i32, i32]),
    "cleave_hip_sum_f64_host": (f64, [vp, i64]),
    "cleave_hip_mean_f64_host": (f64, [vp, i64]),
    "cleave_hip_max_of_f64_host": (f64, [vp, i64]),
    "cleave_hip_argmax_f64_host": (i64, [vp, i64]),
    "cleave_hip_index_f64_host": (f64, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_index_bwd_f64_host": (i32, [f64, vp, i64, vp, i64, vp, i64]),
    "cleave_hip_matmul_f64_into": (i64, [vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, i32]),
    "cleave_hip_add_f64_into": (i64, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_sub_f64_into": (i64, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_mul_f64_into": (i64, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_div_f64_into": (i64, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_neg_f64_into": (i64, [vp, i64, vp, i64]),
    "cleave_hip_relu_f64_into": (i64, [vp, i64, vp, i64]),
    "cleave_hip_sigmoid_f64_into": (i64, [vp, i64, vp, i64]),
    "cleave_hip_tanh_f64_into": (i64, [vp, i64, vp, i64]),
    "cleave_hip_sigmoid_bwd_f64_into": (i64, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_tanh_bwd_f64_into": (i64, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_relu_bwd_f64_into": (i64, [vp, i64, vp, i64, vp, i64]),
    "cleave_hip_sigmoid_hidden_fwd_f32": (i32, [vp, i64, vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32]),
    "cleave_hip_sigmoid_hidden_bwd_f32": (i32, [vp, i64, vp, i64, vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32]),
    "cleave_hip_add_bcast_f32": (i32, [vp, i64, vp, i32, vp, i64, vp, i32, vp, i64]),
    "cleave_hip_sub_bcast_f32": (i32, [vp, i64, vp, i32, vp, i64, vp, i32, vp, i64]),
    "cleave_hip_mul_bcast_f32": (i32, [vp, i64, vp, i32, vp, i64, vp, i32, vp, i64]),
    "cleave_hip_div_bcast_f32": (i32, [vp, i64, vp, i32, vp, i64, vp, i32, vp, i64]),
    "cleave_hip_sum_to_shape_f32": (i32, [vp, i64, vp, i32, vp, i64, vp, i32]),
    "cleave_hip_add_bcast_f64": (i32, [vp, i64, vp, i32, vp, i64, vp, i32, vp, i64]),
    "cleave_hip_sub_bcast_f64": (i32, [vp, i64, vp, i32, vp, i64, vp, i32, vp, i64]),
    "cleave_hip_mul_bcast_f64": (i32, [vp, i64, vp, i32, vp, i64, vp, i32, vp, i64]),
    "cleave_hip_div_bcast_f64": (i32, [vp, i64, vp, i32, vp, i64, vp, i32, vp, i64]),
    "cleave_hip_sum_to_shape_f64": (i32, [vp, i64, vp, i32, vp, i64, vp, i32]),
    "cleave_hip_add_bcast_f32_host": (i32, [vp, i64, vp, i32, vp, i64, vp, i32, vp, i64]),
    "cleave_hip_sub_bcast_f32_host": (i32, [vp, i64, vp, i32, vp, i64, vp, i32, vp, i64]),
    "cleave_hip_mul_bcast_f32_host": (i32, [vp, i64, vp, i32, vp, i64, vp, i32, vp, i64]),
    "cleave_hip_div_bcast_f32_host": (i32, [vp, i64, vp, i32, vp, i64, vp, i32, vp, i64]),
    "cleave_hip_sum_to_shape_f32_host": (i32, [vp, i64, vp, i32, vp, i64, vp, i32]),
    "cleave_hip_add_bcast_f64_host": (i32, [vp, i64, vp, i32, vp, i64, vp, i32, vp, i64]),
    "cleave_hip_sub_bcast_f64_host": (i32, [vp, i64, vp, i32, vp, i64, vp, i32, vp, i64]),
    "cleave_hip_mul_bcast_f64_host": (i32, [vp, i64, vp, i32, vp, i64, vp, i32, vp, i64]),
    "cleave_hip_div_bcast_f64_host": (i32, [vp, i64, vp, i32, vp, i64, vp, i32, vp, i64]),
    "cleave_hip_sum_to_shape_f64_host": (i32, [vp, i64, vp, i32, vp, i64, vp, i32]),
    # memref-descriptor forms: every tensor argument is a pointer to an
    # unranked descriptor {int64 rank; void* ranked descriptor}
    "_mlir_ciface_cleave_hip_matmul_f32": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_matmul_bf16": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_add_f32": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_sub_f32": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_mul_f32": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_div_f32": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_neg_f32": (i32, [vp, vp]),
    "_mlir_ciface_cleave_hip_zero_f32": (i32, [vp]),
    "_mlir_ciface_cleave_hip_relu_f32": (i32, [vp, vp]),
    "_mlir_ciface_cleave_hip_sigmoid_f32": (i32, [vp, vp]),
    "_mlir_ciface_cleave_hip_tanh_f32": (i32, [vp, vp]),
    "_mlir_ciface_cleave_hip_sigmoid_bwd_f32": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_tanh_bwd_f32": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_relu_bwd_f32": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_div_bwd_f32": (i32, [vp, vp, vp, vp, vp]),
    "_mlir_ciface_cleave_hip_sgd_update_f32": (i32, [vp, vp, f32]),
    "_mlir_ciface_cleave_hip_add_row_bias_f32": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_sum_rows_f32": (i32, [vp, vp]),
    "_mlir_ciface_cleave_hip_add_bcast_f32": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_sub_bcast_f32": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_mul_bcast_f32": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_div_bcast_f32": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_add_bcast_f64": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_sub_bcast_f64": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_mul_bcast_f64": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_div_bcast_f64": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_sum_to_shape_f32": (i32, [vp, vp]),
    "_mlir_ciface_cleave_hip_sum_to_shape_f64": (i32, [vp, vp]),
    "_mlir_ciface_cleave_hip_sum_f32": (f32, [vp]),
    "_mlir_ciface_cleave_hip_mean_f32": (f32, [vp]),
    "_mlir_ciface_cleave_hip_max_of_f32": (f32, [vp]),
    "_mlir_ciface_cleave_hip_argmax_f32": (i64, [vp]),
    "_mlir_ciface_cleave_hip_sum_u32_u64": (u64, [vp]),
    "_mlir_ciface_cleave_hip_index_f32": (f32, [vp, vp]),
    "_mlir_ciface_cleave_hip_index_bwd_f32": (i32, [f32, vp, vp]),
    "_mlir_ciface_cleave_hip_mandelbrot_u32": (i32, [vp, f32, f32, f32, f32, i32]),
    "_mlir_ciface_cleave_hip_mlp_step_f32": (i32, [vp, vp, vp, vp, vp, vp, vp, f32]),
    "_mlir_ciface_cleave_hip_matmul_f64": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_add_f64": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_sub_f64": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_mul_f64": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_div_f64": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_neg_f64": (i32, [vp, vp]),
    "_mlir_ciface_cleave_hip_relu_f64": (i32, [vp, vp]),
    "_mlir_ciface_cleave_hip_sigmoid_f64": (i32, [vp, vp]),
    "_mlir_ciface_cleave_hip_tanh_f64": (i32, [vp, vp]),
    "_mlir_ciface_cleave_hip_sigmoid_bwd_f64": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_tanh_bwd_f64": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_relu_bwd_f64": (i32, [vp, vp, vp]),
    "_mlir_ciface_cleave_hip_sum_f64": (f64, [vp]),
    "_mlir_ciface_cleave_hip_mean_f64": (f64, [vp]),
    "_mlir_ciface_cleave_hip_max_of_f64": (f64, [vp]),
    "_mlir_ciface_cleave_hip_argmax_f64": (i64, [vp]),
    "_mlir_ciface_cleave_hip_index_f64": (f64, [vp, vp]),
    "_mlir_ciface_cleave_hip_index_bwd_f64": (i32, [f64, vp, vp]),
}

# Functions whose int32 return is a status code.
STATUS_FUNCS = {n for n, (r, _) in SIGNATURES.items() if r is i32 and n not in (
    "cleave_hip_device_available", "cleave_hip_last_error")}

_lib: C.CDLL | None = None


def load() -> C.CDLL:
    """Load libcleave_hip.so (once) and attach the signatures."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "(there is no CPU fallback)")
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    lib.cleave_hip_set_abort_on_error(0)
    _lib = lib
    return lib


def last_error() -> tuple[int, str]:
    lib = load()
    msg = lib.cleave_hip_last_error_message()
    return lib.cleave_hip_last_error(), (msg.decode() if msg else "")


def check(status: int) -> int:
    """Raise CleaveHipError for a negative status, return it otherwise."""
    if status < 0:
        code, msg = last_error()
        raise CleaveHipError(status, msg)
    return status


def call(name: str, *args):
    """Call an ABI function; status-returning ones raise on error."""
    out = getattr(load(), name)(*args)
    if name in STATUS_FUNCS:
        check(out)
    return out


def symbol_table() -> dict[str, int]:
    """cleave_hip_symbols() as {name: address}."""
    lib = load()
    n = C.c_int64(0)
    tab = lib.cleave_hip_symbols(C.byref(n))
    return {tab[i].name.decode(): tab[i].fn for i in range(n.value)}
