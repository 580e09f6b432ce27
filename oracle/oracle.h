/*
 * oracle.h -- CPU restatement of cleave's tensor hot path (TEST INFRASTRUCTURE).
 *
 * This library is the checker, never the product.  Only tests/, the smoke()
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py may load
 * it.  The product path (libcleave_hip.so) never links or calls it.
 *
 * Every function restates what the reference's CPU pipeline computes for one
 * stdlib tensor operation after MLIR lowers it to scalar loops
 * (convert-linalg-to-loops -> LLVM O2, no fast-math, no FP contraction;
 * /root/reference/cleave/src/main.rs:544-607).  It is compiled with
 * -O2 -ffp-contract=off so gcc keeps the same IEEE f32 operation order.
 *
 * Parity status per function (how each one is pinned) is listed next to the
 * declaration; the checks themselves live in tests/test_oracle.py.
 */
#ifndef CLEAVE_ORACLE_H
#define CLEAVE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- synthetic-input generators (build-defined; the reference has no RNG) ---- */

/* i-th output (0-based) of a splitmix64 stream seeded with `seed`.
 * Pinned: known-answer vector of splitmix64 seeded with 0. */
uint64_t or_splitmix64_at(uint64_t seed, uint64_t i);
/* U[lo,hi) in f32: u = (x>>40) * 2^-24 in [0,1), exact; out = lo + (hi-lo)*u.
 * For lo=-1, hi=1 the result is exact (2u - 1). */
void or_fill_uniform_f32(float* out, int64_t n, uint64_t seed, float lo, float hi);
/* N(mean, std) via Box-Muller (cos branch) on draws 2i, 2i+1, computed in
 * double and rounded to f32.  Pinned: sample mean/variance/normality. */
void or_fill_normal_f32(float* out, int64_t n, uint64_t seed, float mean, float std);
/* f32 -> bf16 round-to-nearest-even (NaN kept quiet). Pinned: hand-made vectors. */
uint16_t or_f32_to_bf16(float x);
float or_bf16_to_f32(uint16_t h);
void or_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n);

/* ---- MatMul (stdlib/linalg/matrix.cleave:27-61; region mlir_lower.rs:2089-2120) ----
 * C = 0; for i, j, k ascending: C[i,j] = C[i,j] + a(i,k) * b(k,j).
 * trans_a: A is stored K x M (C = A^T B); trans_b: B is stored N x K (C = A B^T).
 * rows [row0,row1) only, so a row band can be timed or checked.
 * Pinned: reference golden vectors (2x3*3x2, 2x2*2x2, A*0 = 0), f64 brute force. */
void or_matmul_f32_rows(const float* A, const float* B, float* C, int32_t M, int32_t N,
                        int32_t K, int32_t trans_a, int32_t trans_b, int32_t row0,
                        int32_t row1);
void or_matmul_f32(const float* A, const float* B, float* C, int32_t M, int32_t N,
                   int32_t K, int32_t trans_a, int32_t trans_b);
/* Same loop, rows split across `threads` OpenMP threads (each C[i,j] is an
 * independent sequential k-sum, so the bits are identical). */
void or_matmul_f32_mt(const float* A, const float* B, float* C, int32_t M, int32_t N,
                      int32_t K, int32_t trans_a, int32_t trans_b, int32_t threads);
/* Selected entries only: out[e] = C[ii[e], jj[e]], and absout[e] = sum_k |a||b|
 * (the denominator of the GEMM tolerance). */
void or_matmul_f32_entries(const float* A, const float* B, int32_t M, int32_t N, int32_t K,
                           int32_t trans_a, int32_t trans_b, const int32_t* ii,
                           const int32_t* jj, int64_t n, float* out, float* absout);
/* bf16 inputs upcast exactly to f32, then the same f32 loop. */
void or_matmul_bf16_entries(const uint16_t* A, const uint16_t* B, int32_t M, int32_t N,
                            int32_t K, int32_t trans_a, int32_t trans_b, const int32_t* ii,
                            const int32_t* jj, int64_t n, float* out, float* absout);
void or_matmul_bf16_rows(const uint16_t* A, const uint16_t* B, float* C, int32_t M,
                         int32_t N, int32_t K, int32_t row0, int32_t row1);

/* ---- Ring<Tensor> elementwise (stdlib/linalg/tensor.cleave:66-71) and
 *      Activation<Tensor> (stdlib/nn/nn.cleave:82-95) ---- */
void or_add_f32(const float* a, const float* b, float* out, int64_t n);
void or_sub_f32(const float* a, const float* b, float* out, int64_t n);
void or_mul_f32(const float* a, const float* b, float* out, int64_t n);
void or_div_f32(const float* a, const float* b, float* out, int64_t n);
void or_neg_f32(const float* a, float* out, int64_t n);
/* arith.maximumf(x, 0): IEEE-754-2019 maximum -- NaN propagates, max(-0,+0)=+0. */
void or_relu_f32(const float* a, float* out, int64_t n);
/* negf, math.exp (libm expf), addf(1,.), divf(1,.) in that order. */
void or_sigmoid_f32(const float* a, float* out, int64_t n);
void or_tanh_f32(const float* a, float* out, int64_t n);
float or_sigmoid_scalar(float x);

/* ---- derivative rules used by backward ops (stdlib/num/num.cleave:123-136, :222-223;
 *      stdlib/nn/nn.cleave:87-93 via the quotient + exp rules) ---- */
/* out = g * s * (1 - s), s = sigmoid(x) already computed. */
void or_sigmoid_bwd_f32(const float* s, const float* g, float* out, int64_t n);
/* out = g * (1 - t*t), t = tanh(x). */
void or_tanh_bwd_f32(const float* t, const float* g, float* out, int64_t n);
/* out = x > 0 ? g : 0 (maximumf subgradient, 0 at x == 0). */
void or_relu_bwd_f32(const float* x, const float* g, float* out, int64_t n);
/* div: da = g / b, db = -(g * a) / (b * b). */
void or_div_bwd_f32(const float* a, const float* b, const float* g, float* da, float* db,
                    int64_t n);

/* ---- a bias shared by every row (batched form of examples/xor_tensor.cleave:44-49) ---- */

/* out[i][j] = a[i][j] + bias[j].  Pinned: numpy broadcasting bit for bit; one
 * row is the reference's same-shape Ring add (or_add_f32). */
void or_add_row_bias_f32(const float* a, const float* bias, float* out, int32_t rows, int32_t cols);
/* out[j] = left fold of g[i][j] over i from row 0.  Pinned: exact integer
 * sums, a fold-order case that cancels differently, float64 bound. */
void or_sum_rows_f32(const float* g, float* out, int32_t rows, int32_t cols);

/* ---- broadcasting maps and their reverse rule (extension) ---- */

/* out = a op b (op: 0 add, 1 sub, 2 mul, 3 div) under numpy's broadcasting of
 * shapes ash (rank ar) and bsh (rank br), ranks 0 .. 8; -1 when they do not
 * broadcast.  Pinned: numpy's broadcast arithmetic bit for bit (one IEEE
 * operation per element), and equal shapes reduce to the same-shape maps. */
int32_t or_bcast_f32(int32_t op, const float* a, const int32_t* ash, int32_t ar, const float* b, const int32_t* bsh,
                     int32_t br, float* out);
int32_t or_bcast_f64(int32_t op, const double* a, const int32_t* ash, int32_t ar, const double* b,
                     const int32_t* bsh, int32_t br, double* out);
/* out (shape osh) = g (shape gsh) summed over the dimensions osh stretches,
 * each output's terms in row-major order from zero; -1 when osh does not
 * broadcast to gsh.  Pinned: numpy sums in float64 under the sum bound, exact
 * integer-valued cases, and [rows, cols] -> [cols] against or_sum_rows. */
int32_t or_sum_to_shape_f32(const float* g, const int32_t* gsh, int32_t gr, float* out, const int32_t* osh,
                            int32_t orank);
int32_t or_sum_to_shape_f64(const double* g, const int32_t* gsh, int32_t gr, double* out, const int32_t* osh,
                            int32_t orank);

/* ---- Index (stdlib/linalg/tensor.cleave:113-133) ---- */

/* tensor.extract over the row-major buffer (cleave/src/mlir_lower.rs:1968-2002):
 * element at offset sum_d idx[d] * prod_{e>d} dims[e].  Returns 0 with the
 * element in *out, or -1 for an index outside dims (undefined in the reference).
 * Pinned: numpy C-order indexing on random shapes of rank 1-4, and the
 * reference's constructed-tensor gradient (cleave/tests/mlir_lower.rs:2738-2757). */
int32_t or_index_f32(const float* t, const int32_t* dims, int32_t ndims, const int32_t* idx,
                     float* out);
/* Reverse form of `derivative index(c, idx): index(d(c), idx)`: dt[idx] += g.
 * Returns -1 for an index outside dims.  Pinned as above. */
int32_t or_index_bwd_f32(float g, float* dt, const int32_t* dims, int32_t ndims,
                         const int32_t* idx);

/* ---- Sum / Mean / Max (stdlib/nn/nn.cleave:111-149) ---- */
/* acc = v[0]; for i in 1..N: acc = acc + v[i]. */
float or_sum_f32(const float* v, int64_t n);
/* sum(v) / sitofp(N) (computed as f32 division). */
float or_mean_f32(const float* v, int64_t n);
/* acc = v[0]; for i in 1..N: if v[i] > acc (cmpf ogt) then acc = v[i]. */
float or_max_of_f32(const float* v, int64_t n);
/* index of the element the max_of fold returns (first occurrence; extension). */
int64_t or_argmax_f32(const float* v, int64_t n);
/* exact u64 sum of u32 counts. */
uint64_t or_sum_u32_u64(const uint32_t* v, int64_t n);

/* ---- escape_count (examples/mandelbrot.cleave:14-26 over
 *      stdlib/complex/complex.cleave:24-32, :54), f32 ---- */
/* z = 0; for n in 0..max_iter: z = z*z + c; first n with |z|^2 > 4, else max_iter.
 * Early exit after the first escape (the reference latches and keeps
 * iterating; the result is identical). */
uint32_t or_escape_count_f32(float cr, float ci, int32_t max_iter);
/* Literal latch form (no early exit) for small-grid equivalence checks. */
uint32_t or_escape_count_latch_f32(float cr, float ci, int32_t max_iter);
/* Grid: c = (x0 + col*dx, y0 + row*dy), rows [row0,row1), out row-major width wide. */
void or_mandelbrot_rows(uint32_t* out, int32_t width, int32_t height, float x0, float y0,
                        float dx, float dy, int32_t max_iter, int32_t row0, int32_t row1);
void or_mandelbrot_mt(uint32_t* out, int32_t width, int32_t height, float x0, float y0,
                      float dx, float dy, int32_t max_iter, int32_t threads);
/* Rows [row0,row1) only, split across threads (bit-identical to the rows form). */
void or_mandelbrot_rows_mt(uint32_t* out, int32_t width, int32_t height, float x0, float y0,
                           float dx, float dy, int32_t max_iter, int32_t row0, int32_t row1,
                           int32_t threads);

/* ---- 2-layer MLP step (style of examples/xor_tensor.cleave:38-92) ----
 * H = sigmoid(X W1); yhat = sigmoid(H W2); L = mean((yhat - y)^2);
 * backward by the reference's derivative rules; SGD W -= lr dW.
 * Row-major X [B x D], W1 [D x Hd], W2 [Hd], y [B].
 * Outputs loss, dW1 [D x Hd], dW2 [Hd]; when lr != 0, W1/W2 are updated in place.
 * Scratch: H [B x Hd] and delta [B] are allocated internally. */
float or_mlp_step_f32(const float* X, const float* y, float* W1, float* W2, int32_t B,
                      int32_t D, int32_t Hd, float lr, float* dW1, float* dW2,
                      int32_t threads);
/* Selected entries of that step's gradients (dW1[k1[e], n1[e]], dW2[n2[e]])
 * and its loss, with the forward pass computed as above; for full-size checks.
 * abs1/abs2 receive sum |x||d1| and sum |h||d2| (tolerance denominators).
 * Pinned: bitwise equal to or_mlp_step_f32's entries on small shapes. */
float or_mlp_grad_entries(const float* X, const float* y, const float* W1, const float* W2,
                          int32_t B, int32_t D, int32_t Hd, const int32_t* k1, const int32_t* n1,
                          int64_t e1, float* dw1, float* abs1, const int32_t* n2, int64_t e2,
                          float* dw2, float* abs2, int32_t threads);
/* Loss only, in double (for finite-difference gradient checks). */
double or_mlp_loss_f64(const float* X, const float* y, const float* W1, const float* W2,
                       int32_t B, int32_t D, int32_t Hd);

/* ---- examples/xor_tensor.cleave:38-92 restated: 2-2-1 sigmoid network with
 * biases, per-example loss (pred - y)^2, SGD over the 4 XOR rows in order
 * (i = step mod 4), init examples/xor_tensor.cleave:69-74.  Gradients by the
 * reverse-mode form of the same derivative rules.  Writes the 4 trained
 * predictions (forward of rows 00, 01, 10, 11).  Pinned: doc/backlog.md:142. */
void or_xor_tensor_train(int32_t steps, float lr, float* preds4);


/* f64: the same operators on Tensor<f64, ...> (every tensor impl is generic
 * over T: Float, and Float covers f64, stdlib/num/num.cleave:50-51).
 * Pinned: the reference's golden vectors in f64, exact identities (A*0 = 0,
 * A*I = A, transpose forms against explicit transposes), brute force in
 * long double, libm closed forms and special values, bitwise order checks. */
void or_matmul_f64_rows(const double* A, const double* B, double* C, int32_t M, int32_t N, int32_t K,
                        int32_t trans_a, int32_t trans_b, int32_t row0, int32_t row1);
void or_matmul_f64_mt(const double* A, const double* B, double* C, int32_t M, int32_t N, int32_t K,
                      int32_t trans_a, int32_t trans_b, int32_t threads);
void or_add_f64(const double* a, const double* b, double* out, int64_t n);
void or_sub_f64(const double* a, const double* b, double* out, int64_t n);
void or_mul_f64(const double* a, const double* b, double* out, int64_t n);
void or_div_f64(const double* a, const double* b, double* out, int64_t n);
void or_neg_f64(const double* a, double* out, int64_t n);
void or_relu_f64(const double* a, double* out, int64_t n);
double or_sigmoid_f64_scalar(double x);
void or_sigmoid_f64(const double* a, double* out, int64_t n);
void or_tanh_f64(const double* a, double* out, int64_t n);
void or_sigmoid_bwd_f64(const double* s, const double* g, double* out, int64_t n);
void or_tanh_bwd_f64(const double* t, const double* g, double* out, int64_t n);
void or_relu_bwd_f64(const double* x, const double* g, double* out, int64_t n);
void or_div_bwd_f64(const double* a, const double* b, const double* g, double* da, double* db, int64_t n);
void or_add_row_bias_f64(const double* a, const double* bias, double* out, int32_t rows, int32_t cols);
void or_sum_rows_f64(const double* g, double* out, int32_t rows, int32_t cols);
int32_t or_index_f64(const double* t, const int32_t* dims, int32_t ndims, const int32_t* idx, double* out);
int32_t or_index_bwd_f64(double g, double* dt, const int32_t* dims, int32_t ndims, const int32_t* idx);
double or_sum_f64(const double* v, int64_t n);
double or_mean_f64(const double* v, int64_t n);
double or_max_of_f64(const double* v, int64_t n);
int64_t or_argmax_f64(const double* v, int64_t n);

#ifdef __cplusplus
}
#endif

#endif /* CLEAVE_ORACLE_H */
