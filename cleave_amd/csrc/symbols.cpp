// symbols.cpp -- name -> function pointer table for a JIT host, the shape of
// register_cleave_rt_symbols (/root/reference/cleave/src/pipeline.rs:159-198),
// which registers every cleave-rt function by pointer.  A host that JITs
// `extern(cleave_hip_...)` calls walks this table once instead of keeping its
// own list.  Every function declared in include/cleave_hip.h and
// include/cleave_hip_memref.h appears here.
#include "../../include/cleave_hip_memref.h"

#define CH_SYM(f) {#f, reinterpret_cast<void*>(&f)}

namespace {
const cleave_hip_symbol kSymbols[] = {
    CH_SYM(cleave_hip_init),
    CH_SYM(cleave_hip_device_available),
    CH_SYM(cleave_hip_buf_alloc),
    CH_SYM(cleave_hip_buf_free),
    CH_SYM(cleave_hip_upload),
    CH_SYM(cleave_hip_download),
    CH_SYM(cleave_hip_sync),
    CH_SYM(cleave_hip_set_abort_on_error),
    CH_SYM(cleave_hip_last_error),
    CH_SYM(cleave_hip_last_error_message),
    CH_SYM(cleave_hip_event_create),
    CH_SYM(cleave_hip_event_record),
    CH_SYM(cleave_hip_event_elapsed_ms),
    CH_SYM(cleave_hip_event_destroy),
    CH_SYM(cleave_hip_symbols),
    CH_SYM(cleave_hip_fill_uniform_f32),
    CH_SYM(cleave_hip_fill_normal_f32),
    CH_SYM(cleave_hip_fill_bernoulli_f32),
    CH_SYM(cleave_hip_cast_f32_bf16),
    CH_SYM(cleave_hip_matmul_f32),
    CH_SYM(cleave_hip_matmul_batched_f32),
    CH_SYM(cleave_hip_matmul_bf16),
    CH_SYM(cleave_hip_matmul_batched_bf16),
    CH_SYM(cleave_hip_add_f32),
    CH_SYM(cleave_hip_sub_f32),
    CH_SYM(cleave_hip_mul_f32),
    CH_SYM(cleave_hip_div_f32),
    CH_SYM(cleave_hip_neg_f32),
    CH_SYM(cleave_hip_zero_f32),
    CH_SYM(cleave_hip_relu_f32),
    CH_SYM(cleave_hip_sigmoid_f32),
    CH_SYM(cleave_hip_tanh_f32),
    CH_SYM(cleave_hip_sigmoid_bwd_f32),
    CH_SYM(cleave_hip_tanh_bwd_f32),
    CH_SYM(cleave_hip_relu_bwd_f32),
    CH_SYM(cleave_hip_div_bwd_f32),
    CH_SYM(cleave_hip_sgd_update_f32),
    CH_SYM(cleave_hip_reduce_sum_f32),
    CH_SYM(cleave_hip_reduce_max_f32),
    CH_SYM(cleave_hip_reduce_sum_u32_u64),
    CH_SYM(cleave_hip_sum_f32),
    CH_SYM(cleave_hip_mean_f32),
    CH_SYM(cleave_hip_max_of_f32),
    CH_SYM(cleave_hip_argmax_f32),
    CH_SYM(cleave_hip_sum_u32_u64),
    CH_SYM(cleave_hip_index_f32),
    CH_SYM(cleave_hip_index_bwd_f32),
    CH_SYM(cleave_hip_mandelbrot_u32),
    CH_SYM(cleave_hip_mlp_step_f32),
    CH_SYM(_mlir_ciface_cleave_hip_matmul_f32),
    CH_SYM(_mlir_ciface_cleave_hip_matmul_bf16),
    CH_SYM(_mlir_ciface_cleave_hip_add_f32),
    CH_SYM(_mlir_ciface_cleave_hip_sub_f32),
    CH_SYM(_mlir_ciface_cleave_hip_mul_f32),
    CH_SYM(_mlir_ciface_cleave_hip_div_f32),
    CH_SYM(_mlir_ciface_cleave_hip_neg_f32),
    CH_SYM(_mlir_ciface_cleave_hip_zero_f32),
    CH_SYM(_mlir_ciface_cleave_hip_relu_f32),
    CH_SYM(_mlir_ciface_cleave_hip_sigmoid_f32),
    CH_SYM(_mlir_ciface_cleave_hip_tanh_f32),
    CH_SYM(_mlir_ciface_cleave_hip_sigmoid_bwd_f32),
    CH_SYM(_mlir_ciface_cleave_hip_tanh_bwd_f32),
    CH_SYM(_mlir_ciface_cleave_hip_relu_bwd_f32),
    CH_SYM(_mlir_ciface_cleave_hip_div_bwd_f32),
    CH_SYM(_mlir_ciface_cleave_hip_sgd_update_f32),
    CH_SYM(_mlir_ciface_cleave_hip_sum_f32),
    CH_SYM(_mlir_ciface_cleave_hip_mean_f32),
    CH_SYM(_mlir_ciface_cleave_hip_max_of_f32),
    CH_SYM(_mlir_ciface_cleave_hip_argmax_f32),
    CH_SYM(_mlir_ciface_cleave_hip_sum_u32_u64),
    CH_SYM(_mlir_ciface_cleave_hip_index_f32),
    CH_SYM(_mlir_ciface_cleave_hip_index_bwd_f32),
    CH_SYM(_mlir_ciface_cleave_hip_mandelbrot_u32),
    CH_SYM(_mlir_ciface_cleave_hip_mlp_step_f32),
};
}  // namespace

extern "C" const cleave_hip_symbol* cleave_hip_symbols(int64_t* count) {
    if (count) *count = (int64_t)(sizeof(kSymbols) / sizeof(kSymbols[0]));
    return kSymbols;
}
