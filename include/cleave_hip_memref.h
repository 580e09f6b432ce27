/*
 * cleave_hip_memref.h -- the tensor operators of cleave_hip.h taking MLIR
 * memref descriptors, for a lowering that passes cleave Tensors across an
 * `extern` call as memrefs.
 *
 * After one-shot-bufferize a cleave Tensor is a memref
 * (/root/reference/cleave/src/main.rs:551-565), but today only arrays cross
 * an extern call, as an (aligned pointer, i64 length) pair
 * (cleave/src/mlir_lower.rs:1096-1114, :1702-1713).  A function declared with
 * the `llvm.emit_c_interface` attribute is instead called through
 * `_mlir_ciface_<name>` with pointers to memref descriptors -- MLIR's
 * C-compatible wrapper ABI:
 *
 *   ranked   memref<d0 x .. x T>: { T* allocated; T* aligned; int64_t offset;
 *                                    int64_t sizes[rank]; int64_t strides[rank]; }
 *   unranked memref<* x T>:        { int64_t rank; void* descriptor; }
 *
 * Every entry point below takes UNRANKED descriptors, so one symbol serves
 * every rank: the caller casts (`memref.cast %t : memref<4x5xf32> to
 * memref<*xf32>`) before the call.  The element address is
 * aligned + offset * sizeof(T); tensor data are device pointers from
 * cleave_hip_buf_alloc.  Index arrays (memref<K x i32>) are host memory, as an
 * [i32; K] is in the reference.
 *
 * Layout rules, checked on the host before any device work:
 *   - element-wise operands, reduction inputs and every output: row-major
 *     contiguous (stride of dim i = product of the sizes after it; a dim of
 *     size 1 may carry any stride), with identical sizes (no broadcasting,
 *     as in the reference), except in the _bcast maps and sum_to_shape,
 *     whose operands keep their own sizes;
 *   - matmul operands: rank 2 [M x K], [K x N] (rank 3 with a leading batch
 *     for the batched forms), each either row-major or the transpose of a
 *     row-major buffer (strides {1, M} for A).  A transposed operand becomes
 *     trans_a / trans_b of the pointer form, so A^T B and A B^T -- the
 *     reverse-mode halves of the product rule -- need no copy.
 *
 * Status and error behaviour are those of the pointer forms in cleave_hip.h
 * (abort by default, negative status after cleave_hip_set_abort_on_error(0)).
 * The scalar-returning reductions return NaN / -1 after an error.
 *
 * These entry points have no counterpart in cleave-rt.  They are the library
 * side of passing Tensors across extern as memrefs.  The reference's lowering
 * passes an extern's arrays as a bare aligned pointer plus a length instead,
 * because MLIR's default conversion turns a memref argument into its
 * descriptor fields, which no hand-written extern matched
 * (cleave/src/mlir_lower.rs:1700-1716).  With `llvm.emit_c_interface` on the
 * declaration the descriptor arrives by pointer, in the layout above.
 */
#ifndef CLEAVE_HIP_MEMREF_H
#define CLEAVE_HIP_MEMREF_H

#include "cleave_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* memref<* x T>: rank, then a pointer to the ranked descriptor. */
typedef struct cleave_hip_memref {
    int64_t rank;
    void* descriptor;
} cleave_hip_memref;

typedef const cleave_hip_memref* cleave_hip_mr;

/* MatMul (stdlib/linalg/matrix.cleave:22-61): C = op(A) op(B), C overwritten.
 * Rank 2, or rank 3 for `batch` independent products (batched bf16: A and B
 * row-major only). */
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_matmul_f32(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr c);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_matmul_bf16(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr c);

/* Ring<Tensor> (stdlib/linalg/tensor.cleave:66-80). */
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_add_f32(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_sub_f32(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_mul_f32(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_div_f32(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_neg_f32(cleave_hip_mr a, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_zero_f32(cleave_hip_mr out);

/* Activation<Tensor> (stdlib/nn/nn.cleave:82-95). */
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_relu_f32(cleave_hip_mr x, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_sigmoid_f32(cleave_hip_mr x, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_tanh_f32(cleave_hip_mr x, cleave_hip_mr out);

/* Reverse-mode rules (stdlib/num/num.cleave:123-136, :222-223) and SGD. */
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_sigmoid_bwd_f32(cleave_hip_mr s, cleave_hip_mr g, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_tanh_bwd_f32(cleave_hip_mr t, cleave_hip_mr g, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_relu_bwd_f32(cleave_hip_mr x, cleave_hip_mr g, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_div_bwd_f32(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr g,
                                                          cleave_hip_mr da, cleave_hip_mr db);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_sgd_update_f32(cleave_hip_mr w, cleave_hip_mr g, float lr);

/* Row-broadcast bias: a, out [rows x cols], bias [cols] (or [1 x cols]);
 * its reverse rule sums g [rows x cols] over the rows into out [cols]. */
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_add_row_bias_f32(cleave_hip_mr a, cleave_hip_mr bias, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_sum_rows_f32(cleave_hip_mr g, cleave_hip_mr out);
/* Broadcasting maps (extension): out = a op b under numpy's broadcasting of
 * a's and b's sizes; out's sizes must be the broadcast shape.  Ranks 0 .. 8. */
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_add_bcast_f32(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_sub_bcast_f32(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_mul_bcast_f32(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_div_bcast_f32(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_add_bcast_f64(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_sub_bcast_f64(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_mul_bcast_f64(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_div_bcast_f64(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out);
/* Their reverse rule: out (sizes broadcasting to g's) = g summed over the
 * stretched dimensions. */
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_sum_to_shape_f32(cleave_hip_mr g, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_sum_to_shape_f64(cleave_hip_mr g, cleave_hip_mr out);

/* Sum / Mean / Max (stdlib/nn/nn.cleave:111-149), host-returning. */
CLEAVE_HIP_API float _mlir_ciface_cleave_hip_sum_f32(cleave_hip_mr x);
CLEAVE_HIP_API float _mlir_ciface_cleave_hip_mean_f32(cleave_hip_mr x);
CLEAVE_HIP_API float _mlir_ciface_cleave_hip_max_of_f32(cleave_hip_mr x);
CLEAVE_HIP_API int64_t _mlir_ciface_cleave_hip_argmax_f32(cleave_hip_mr x);
CLEAVE_HIP_API uint64_t _mlir_ciface_cleave_hip_sum_u32_u64(cleave_hip_mr x);

/* Index<Tensor> (stdlib/linalg/tensor.cleave:113-133): idx is a host
 * memref<K x i32> with K = rank of t. */
CLEAVE_HIP_API float _mlir_ciface_cleave_hip_index_f32(cleave_hip_mr t, cleave_hip_mr idx);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_index_bwd_f32(float g, cleave_hip_mr dt, cleave_hip_mr idx);

/* escape_count map (examples/mandelbrot.cleave:14-26): out is
 * memref<height x width x i32> of counts (u32 values). */
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_mandelbrot_u32(cleave_hip_mr out, float x0, float y0, float dx,
                                                             float dy, int32_t max_iter);

/* MLP step (style of examples/xor_tensor.cleave:38-92): x [B x D], y [B],
 * w1 [D x Hd], w2 [Hd]; dw1, dw2 and loss (one element) may be null. */
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_mlp_step_f32(cleave_hip_mr x, cleave_hip_mr y, cleave_hip_mr w1,
                                                           cleave_hip_mr w2, cleave_hip_mr dw1, cleave_hip_mr dw2,
                                                           cleave_hip_mr loss, float lr);

/* Tensor<f64, ...> forms of the above (memref<... x f64>), same rules. */
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_matmul_f64(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr c);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_add_f64(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_sub_f64(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_mul_f64(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_div_f64(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_neg_f64(cleave_hip_mr a, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_relu_f64(cleave_hip_mr x, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_sigmoid_f64(cleave_hip_mr x, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_tanh_f64(cleave_hip_mr x, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_sigmoid_bwd_f64(cleave_hip_mr s, cleave_hip_mr g, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_tanh_bwd_f64(cleave_hip_mr t, cleave_hip_mr g, cleave_hip_mr out);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_relu_bwd_f64(cleave_hip_mr x, cleave_hip_mr g, cleave_hip_mr out);
CLEAVE_HIP_API double _mlir_ciface_cleave_hip_sum_f64(cleave_hip_mr x);
CLEAVE_HIP_API double _mlir_ciface_cleave_hip_mean_f64(cleave_hip_mr x);
CLEAVE_HIP_API double _mlir_ciface_cleave_hip_max_of_f64(cleave_hip_mr x);
CLEAVE_HIP_API int64_t _mlir_ciface_cleave_hip_argmax_f64(cleave_hip_mr x);
CLEAVE_HIP_API double _mlir_ciface_cleave_hip_index_f64(cleave_hip_mr t, cleave_hip_mr idx);
CLEAVE_HIP_API int32_t _mlir_ciface_cleave_hip_index_bwd_f64(double g, cleave_hip_mr dt, cleave_hip_mr idx);

#ifdef __cplusplus
}
#endif

#endif /* CLEAVE_HIP_MEMREF_H */
