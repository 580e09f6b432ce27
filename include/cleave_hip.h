/*
 * cleave_hip.h -- C ABI of libcleave_hip.so, the MI355X (gfx950) backend for
 * cleave's tensor operator surface.
 *
 * Conventions follow cleave-rt, the reference's only native boundary
 * (/root/reference/cleave-rt/src/lib.rs:13-213):
 *   - plain `extern "C"` symbols, no C++ mangling (lib.rs:13-21);
 *   - scalars by value: int32_t dims, int64_t lengths, float scalars
 *     (cleave/src/rust_bindings.rs:21-35);
 *   - every array operand is a pair (pointer, int64_t element count), the
 *     form mlir_lower.rs emits for an array crossing an extern call
 *     (cleave/src/mlir_lower.rs:1096-1114, :1720-1751; sum_bytes,
 *     cleave-rt/src/lib.rs:86-90);
 *   - arrays are never returned: outputs are caller-allocated (ptr, len)
 *     pairs (cleave/src/mlir_lower.rs:1062-1075);
 *   - device buffers are opaque handles, like stdlib's RawBuf
 *     (stdlib/dynarray/dynarray.cleave:29), allocated by cleave_hip_buf_alloc;
 *   - errors: cleave-rt panics (lib.rs:69, :120, :148).  Here every call
 *     validates its arguments on the host before any launch; by default an
 *     error prints a message to stderr and aborts (same observable
 *     behaviour); cleave_hip_set_abort_on_error(0) switches to returning a
 *     negative status with the message kept for cleave_hip_last_error_message().
 *
 * Threading/sync: one thread, one HIP stream owned by the library
 * (cleave/src/main.rs:607 runs JIT code on the calling thread).  Calls that
 * return host-visible data (downloads, scalar-returning reductions)
 * synchronise the stream before returning; calls that only write device
 * buffers are queued on the stream and return immediately.
 *
 * Two pointer kinds, two sets of entry points:
 *   - the device entry points (cleave_hip_matmul_f32, ...) take device
 *     buffers (cleave_hip_buf_alloc, or any hipMalloc'd memory) and check on
 *     the host that every tensor operand is device memory whose allocation
 *     covers its length; anything else is CLEAVE_HIP_ERR_ARG, never a launch;
 *   - the host entry points (cleave_hip_matmul_f32_host, ...; end of this
 *     file) take host arrays, as cleave's extern lowering passes them, stage
 *     them through library memory in HBM and synchronise before returning.
 */
#ifndef CLEAVE_HIP_H
#define CLEAVE_HIP_H

#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define CLEAVE_HIP_API __attribute__((visibility("default")))
#else
#define CLEAVE_HIP_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define CLEAVE_HIP_OK 0
#define CLEAVE_HIP_ERR_RUNTIME (-1) /* HIP runtime error or no device */
#define CLEAVE_HIP_ERR_ARG (-2)     /* length/shape/flag validation failed */
#define CLEAVE_HIP_ERR_OOM (-3)     /* device allocation failed */

/* ---------------------------------------------------------------------- */
/* runtime (replaces cleave-rt's allocation and registration surface)     */
/* ---------------------------------------------------------------------- */

/* Selects device 0 and creates the library stream.  Idempotent.  Every other
 * entry point calls it implicitly.  (No reference counterpart: the reference
 * runs on the CPU with no device to open.) */
CLEAVE_HIP_API int32_t cleave_hip_init(void);
/* 1 when a device is usable, 0 otherwise (never aborts). */
CLEAVE_HIP_API int32_t cleave_hip_device_available(void);

/* Device allocation, 256-byte aligned.  Mirrors cleave_alloc
 * (cleave-rt/src/lib.rs:56-71; that one is 16-byte aligned and never freed);
 * here the library owns the memory and cleave_hip_buf_free releases it: into
 * a cache of free blocks that later allocations of the same size reuse
 * without a device synchronisation (work on the library stream is ordered).
 * The cache holds at most 32 GiB and is returned to the device when an
 * allocation (a buffer, or library scratch) would otherwise fail.  A device
 * entry point refuses an operand that runs past the bytes its buffer was
 * allocated with, and a pointer into a freed block still in the cache. */
CLEAVE_HIP_API void* cleave_hip_buf_alloc(int64_t bytes);
CLEAVE_HIP_API void cleave_hip_buf_free(void* buf);
/* Returns every cached free block to the device (after the library stream
 * drains) and the bytes released, for a host that needs the memory for
 * something outside this library.  The library's own allocations (buffers
 * and scratch) already do this before they fail.  (No reference
 * counterpart: cleave_alloc never frees, cleave-rt/src/lib.rs:56-71.) */
CLEAVE_HIP_API int64_t cleave_hip_buf_trim(void);
/* Bytes held by the cache of freed blocks. */
CLEAVE_HIP_API int64_t cleave_hip_buf_cached_bytes(void);
/* Host <-> device copies on the library stream; both return the byte count
 * (like print_bytes' "returns len", cleave-rt/src/lib.rs:114-122) after the
 * stream has drained, so the host buffer may be reused at once. */
CLEAVE_HIP_API int64_t cleave_hip_upload(void* dst_dev, const void* src_host, int64_t bytes);
CLEAVE_HIP_API int64_t cleave_hip_download(void* dst_host, const void* src_dev, int64_t bytes);
/* Waits for all queued work. */
CLEAVE_HIP_API int32_t cleave_hip_sync(void);

/* Error channel. */
CLEAVE_HIP_API void cleave_hip_set_abort_on_error(int32_t on);
CLEAVE_HIP_API int32_t cleave_hip_last_error(void);
CLEAVE_HIP_API const char* cleave_hip_last_error_message(void);

/* Events on the library stream (timing of queued work). */
CLEAVE_HIP_API void* cleave_hip_event_create(void);
CLEAVE_HIP_API int32_t cleave_hip_event_record(void* ev);
CLEAVE_HIP_API float cleave_hip_event_elapsed_ms(void* start, void* stop); /* syncs on stop */
CLEAVE_HIP_API void cleave_hip_event_destroy(void* ev);

/* Symbol table for a JIT host: name -> function pointer, the same shape as
 * register_cleave_rt_symbols (cleave/src/pipeline.rs:159-198).  Returns the
 * table and writes its length to *count. */
typedef struct cleave_hip_symbol {
    const char* name;
    void* fn;
} cleave_hip_symbol;
CLEAVE_HIP_API const cleave_hip_symbol* cleave_hip_symbols(int64_t* count);

/* ---------------------------------------------------------------------- */
/* synthetic inputs (the reference has no RNG; generator is build-defined) */
/* ---------------------------------------------------------------------- */

/* out[i] = lo + (hi-lo) * u_i, u_i = (splitmix64_i(seed) >> 40) * 2^-24. */
CLEAVE_HIP_API int32_t cleave_hip_fill_uniform_f32(float* out, int64_t len, uint64_t seed, float lo, float hi);
/* Box-Muller on draws 2i and 2i+1 (cos branch), mean + std * z. */
CLEAVE_HIP_API int32_t cleave_hip_fill_normal_f32(float* out, int64_t len, uint64_t seed, float mean, float std);
/* out[i] = (u_i < p) ? 1 : 0. */
CLEAVE_HIP_API int32_t cleave_hip_fill_bernoulli_f32(float* out, int64_t len, uint64_t seed, float p);
/* f32 -> bf16 round-to-nearest-even; bf16 stored as uint16_t. */
CLEAVE_HIP_API int32_t cleave_hip_cast_f32_bf16(const float* in, int64_t inlen, uint16_t* out, int64_t outlen);

/* ---------------------------------------------------------------------- */
/* MatMul (stdlib/linalg/matrix.cleave:22-61)                               */
/* ---------------------------------------------------------------------- */

/* C[M x N] = op(A) * op(B), fp32 accumulate, C overwritten (the reference
 * zero-fills its accumulator, stdlib/linalg/matrix.cleave:59).
 * trans_a = 0: A stored M x K row-major; 1: A stored K x M (C = A^T B).
 * trans_b = 0: B stored K x N row-major; 1: B stored N x K (C = A B^T).
 * The A^T B / A B^T forms are the reverse-mode halves of the product rule
 * add(matmul(d(a),b), matmul(a,d(b))) (stdlib/linalg/matrix.cleave:24).
 * Requires alen == M*K, blen == K*N, clen == M*N. */
CLEAVE_HIP_API int32_t cleave_hip_matmul_f32(const float* a, int64_t alen, const float* b, int64_t blen,
                              float* c, int64_t clen, int32_t M, int32_t N, int32_t K,
                              int32_t trans_a, int32_t trans_b);
/* batch independent f32 matmuls, operands packed back to back. */
CLEAVE_HIP_API int32_t cleave_hip_matmul_batched_f32(const float* a, int64_t alen, const float* b,
                                      int64_t blen, float* c, int64_t clen, int32_t batch,
                                      int32_t M, int32_t N, int32_t K, int32_t trans_a,
                                      int32_t trans_b);
/* bf16 inputs (uint16_t storage), fp32 accumulate and fp32 output.
 * Extension of the same operator (the reference is f32/f64 only). */
CLEAVE_HIP_API int32_t cleave_hip_matmul_bf16(const uint16_t* a, int64_t alen, const uint16_t* b,
                               int64_t blen, float* c, int64_t clen, int32_t M, int32_t N,
                               int32_t K, int32_t trans_a, int32_t trans_b);
/* batch independent bf16 matmuls, operands packed back to back, with the
 * same trans flags as the single product (each batch entry stored K x M for
 * trans_a, N x K for trans_b): the batched halves of the product rule. */
CLEAVE_HIP_API int32_t cleave_hip_matmul_batched_bf16(const uint16_t* a, int64_t alen, const uint16_t* b,
                                       int64_t blen, float* c, int64_t clen, int32_t batch,
                                       int32_t M, int32_t N, int32_t K, int32_t trans_a,
                                       int32_t trans_b);

/* ---------------------------------------------------------------------- */
/* Ring<Tensor> elementwise (stdlib/linalg/tensor.cleave:66-80)             */
/* Same-shape operands, no broadcasting (as in the reference).              */
/* ---------------------------------------------------------------------- */

CLEAVE_HIP_API int32_t cleave_hip_add_f32(const float* a, int64_t alen, const float* b, int64_t blen,
                           float* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_sub_f32(const float* a, int64_t alen, const float* b, int64_t blen,
                           float* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_mul_f32(const float* a, int64_t alen, const float* b, int64_t blen,
                           float* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_div_f32(const float* a, int64_t alen, const float* b, int64_t blen,
                           float* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_neg_f32(const float* a, int64_t alen, float* out, int64_t outlen);
/* Ring::zero (stdlib/linalg/tensor.cleave:79). */
CLEAVE_HIP_API int32_t cleave_hip_zero_f32(float* out, int64_t outlen);

/* ---------------------------------------------------------------------- */
/* Activation<Tensor> (stdlib/nn/nn.cleave:82-95)                           */
/* ---------------------------------------------------------------------- */

/* arith.maximumf(x, 0): NaN propagates, max(-0,+0) = +0 (nn.cleave:83-85). */
CLEAVE_HIP_API int32_t cleave_hip_relu_f32(const float* x, int64_t xlen, float* out, int64_t outlen);
/* 1 / (1 + exp(-x)) (nn.cleave:87-93). */
CLEAVE_HIP_API int32_t cleave_hip_sigmoid_f32(const float* x, int64_t xlen, float* out, int64_t outlen);
/* math.tanh (nn.cleave:94). */
CLEAVE_HIP_API int32_t cleave_hip_tanh_f32(const float* x, int64_t xlen, float* out, int64_t outlen);

/* ---------------------------------------------------------------------- */
/* backward ops: reverse-mode forms of the reference's derivative rules     */
/* (stdlib/num/num.cleave:123-136, :222-223; stdlib/linalg/tensor.cleave:126)*/
/* ---------------------------------------------------------------------- */

/* out = g * s * (1 - s), s = sigmoid(x) from the forward pass. */
CLEAVE_HIP_API int32_t cleave_hip_sigmoid_bwd_f32(const float* s, int64_t slen, const float* g, int64_t glen,
                                   float* out, int64_t outlen);
/* out = g * (1 - t*t), t = tanh(x) (num.cleave:223). */
CLEAVE_HIP_API int32_t cleave_hip_tanh_bwd_f32(const float* t, int64_t tlen, const float* g, int64_t glen,
                                float* out, int64_t outlen);
/* out = x > 0 ? g : 0. */
CLEAVE_HIP_API int32_t cleave_hip_relu_bwd_f32(const float* x, int64_t xlen, const float* g, int64_t glen,
                                float* out, int64_t outlen);
/* quotient rule (num.cleave:132-134): da = g / b, db = -(g*a) / (b*b). */
CLEAVE_HIP_API int32_t cleave_hip_div_bwd_f32(const float* a, int64_t alen, const float* b, int64_t blen,
                               const float* g, int64_t glen, float* da, int64_t dalen,
                               float* db, int64_t dblen);
/* SGD update in place: w = w - lr * g (examples/xor_tensor.cleave:86-90). */
CLEAVE_HIP_API int32_t cleave_hip_sgd_update_f32(float* w, int64_t wlen, const float* g, int64_t glen,
                                  float lr);

/* ---------------------------------------------------------------------- */
/* A bias shared by every row of a batch (extension: the reference's add    */
/* needs equal shapes, stdlib/linalg/tensor.cleave:66-71, and adds a         */
/* same-shape bias one example at a time, examples/xor_tensor.cleave:44-49) */
/* ---------------------------------------------------------------------- */

/* out[i*cols + j] = a[i*cols + j] + bias[j] for a row-major [rows x cols] a.
 * Requires alen == outlen == rows*cols and blen == cols. */
CLEAVE_HIP_API int32_t cleave_hip_add_row_bias_f32(const float* a, int64_t alen, const float* bias, int64_t blen,
                                                   float* out, int64_t outlen, int32_t rows, int32_t cols);
/* Reverse rule of that broadcast: out[j] = sum over i of g[i*cols + j]
 * (device order: ascending rows within fixed row groups, then the groups in
 * order).  Requires rows >= 1, glen == rows*cols, outlen == cols. */
CLEAVE_HIP_API int32_t cleave_hip_sum_rows_f32(const float* g, int64_t glen, float* out, int64_t outlen,
                                               int32_t rows, int32_t cols);

/* ---------------------------------------------------------------------- */
/* Broadcasting maps (extension: the reference's Ring<Tensor> maps need     */
/* equal shapes, stdlib/linalg/tensor.cleave:66-71, and Activation<Tensor>  */
/* is rank 1, stdlib/nn/nn.cleave:82)                                       */
/* ---------------------------------------------------------------------- */

/* out = a op b with numpy's broadcasting: the shapes (host arrays of rank
 * 0 .. 8, dimensions >= 0) align at their last dimension, a missing leading
 * dimension is 1, and a dimension of 1 stretches to the other operand's.
 * Each output element is one IEEE operation, as in the same-shape maps.
 * Requires alen and blen to match the shapes and outlen the broadcast shape;
 * shapes that do not broadcast are CLEAVE_HIP_ERR_ARG. */
CLEAVE_HIP_API int32_t cleave_hip_add_bcast_f32(const float* a, int64_t alen, const int32_t* ashape, int32_t arank,
                                                const float* b, int64_t blen, const int32_t* bshape, int32_t brank,
                                                float* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_sub_bcast_f32(const float* a, int64_t alen, const int32_t* ashape, int32_t arank,
                                                const float* b, int64_t blen, const int32_t* bshape, int32_t brank,
                                                float* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_mul_bcast_f32(const float* a, int64_t alen, const int32_t* ashape, int32_t arank,
                                                const float* b, int64_t blen, const int32_t* bshape, int32_t brank,
                                                float* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_div_bcast_f32(const float* a, int64_t alen, const int32_t* ashape, int32_t arank,
                                                const float* b, int64_t blen, const int32_t* bshape, int32_t brank,
                                                float* out, int64_t outlen);
/* Reverse rule of a broadcast: out (shape oshape, which broadcasts to
 * gshape) = g summed over the dimensions that broadcasting stretched, in an
 * order fixed by the shapes.  Requires orank <= grank <= 8. */
CLEAVE_HIP_API int32_t cleave_hip_sum_to_shape_f32(const float* g, int64_t glen, const int32_t* gshape,
                                                   int32_t grank, float* out, int64_t outlen,
                                                   const int32_t* oshape, int32_t orank);

/* ---------------------------------------------------------------------- */
/* Sum / Mean / Max (stdlib/nn/nn.cleave:111-149)                           */
/* ---------------------------------------------------------------------- */

/* Device-result forms (queued; result written to a device scalar). */
CLEAVE_HIP_API int32_t cleave_hip_reduce_sum_f32(const float* x, int64_t len, float* out_dev);
CLEAVE_HIP_API int32_t cleave_hip_reduce_max_f32(const float* x, int64_t len, float* max_dev,
                                  int64_t* argmax_dev);
CLEAVE_HIP_API int32_t cleave_hip_reduce_sum_u32_u64(const uint32_t* x, int64_t len, uint64_t* out_dev);
/* Exact i64 sum of an i32 array: the escape counts as cleave's i32 type holds
 * them (escape_count returns i32, examples/mandelbrot.cleave:14).  Extension:
 * the reference's Sum is over Float elements (stdlib/nn/nn.cleave:111-117). */
CLEAVE_HIP_API int32_t cleave_hip_reduce_sum_i32_i64(const int32_t* x, int64_t len, int64_t* out_dev);
/* cleave_hip_reduce_sum_f32 that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same kernels, grid and result as cleave_hip_reduce_sum_f32;
 * its partial sums live in a static 64 KiB device workspace (16384 floats,
 * one per stage-1 block; a call needing more is CLEAVE_HIP_ERR_ARG) whose
 * address the library's init resolves, so call cleave_hip_init() first if
 * the first call must not initialise.  Every call on a device shares that
 * workspace: calls that overlap on one device race. */
CLEAVE_HIP_API int32_t cleave_hip_reduce_sum_f32_noalloc(const float* x, int64_t len, float* out_dev);
/* Host-returning forms, like the stdlib functions (synchronise). */
CLEAVE_HIP_API float cleave_hip_sum_f32(const float* x, int64_t len);
CLEAVE_HIP_API float cleave_hip_mean_f32(const float* x, int64_t len);
CLEAVE_HIP_API float cleave_hip_max_of_f32(const float* x, int64_t len);
/* First index of the value max_of returns (extension; the reference has no argmax). */
CLEAVE_HIP_API int64_t cleave_hip_argmax_f32(const float* x, int64_t len);
CLEAVE_HIP_API uint64_t cleave_hip_sum_u32_u64(const uint32_t* x, int64_t len);
CLEAVE_HIP_API int64_t cleave_hip_sum_i32_i64(const int32_t* x, int64_t len); /* 0 after an error */

/* ---------------------------------------------------------------------- */
/* Index<Tensor> (stdlib/linalg/tensor.cleave:113-133)                      */
/* ---------------------------------------------------------------------- */

/* t[idx] of a row-major tensor with extents dims (tensor.extract).  dims and
 * idx are host int32 arrays of equal length (an [i32; K] across an extern
 * call); every index is checked against its extent and prod(dims) against
 * len.  Returns the element (synchronises); NaN after an error. */
CLEAVE_HIP_API float cleave_hip_index_f32(const float* t, int64_t len, const int32_t* dims, int64_t ndims,
                                          const int32_t* idx, int64_t nidx);
/* Reverse-mode form of `derivative index(c, idx): index(d(c), idx)`
 * (tensor.cleave:126): dt[idx] += g on the library stream. */
CLEAVE_HIP_API int32_t cleave_hip_index_bwd_f32(float g, float* dt, int64_t len, const int32_t* dims,
                                                int64_t ndims, const int32_t* idx, int64_t nidx);

/* ---------------------------------------------------------------------- */
/* escape_count map (examples/mandelbrot.cleave:14-26) in f32                */
/* ---------------------------------------------------------------------- */

/* out[row*width + col] = escape count of c = (x0 + col*dx, y0 + row*dy),
 * max_iter if it never escapes.  Requires outlen == width*height. */
CLEAVE_HIP_API int32_t cleave_hip_mandelbrot_u32(uint32_t* out, int64_t outlen, int32_t width, int32_t height,
                                  float x0, float y0, float dx, float dy, int32_t max_iter);

/* ---------------------------------------------------------------------- */
/* 2-layer MLP step (style of examples/xor_tensor.cleave:38-92)             */
/* ---------------------------------------------------------------------- */

/* H = sigmoid(X W1), yhat = sigmoid(H W2), loss = mean((yhat - y)^2),
 * reverse-mode gradients, then W -= lr * dW in place (lr = 0 skips the
 * update).  X [B x D], y [B], W1 [D x Hd], W2 [Hd].  dW1/dW2 receive the
 * gradients when non-null (lengths D*Hd and Hd).  loss_dev receives the
 * loss (device scalar) when non-null.  Scratch (B*Hd + 2*B floats) is
 * allocated by the library on first use and kept. */
CLEAVE_HIP_API int32_t cleave_hip_mlp_step_f32(const float* x, int64_t xlen, const float* y, int64_t ylen,
                                float* w1, int64_t w1len, float* w2, int64_t w2len,
                                float* dw1, int64_t dw1len, float* dw2, int64_t dw2len,
                                float* loss_dev, int32_t B, int32_t D, int32_t Hd, float lr);

/* The hidden layer of that step as its own forward and reverse rule, for a
 * host that meets the subgraph z = sigmoid(X W1) w2 (w2 a column) in a
 * program, such as a reverse-mode tape: the step's fused kernels (sigmoid and
 * the partial products with w2 in the GEMM's epilogue; d1 formed while the
 * dW1 GEMM reads H) whenever B, D and Hd are multiples of 256, the separate
 * kernels otherwise.  Reverse rules applied: the MatMul product rule
 * (stdlib/linalg/matrix.cleave:24) and sigmoid's s(1 - s)
 * (stdlib/num/num.cleave:132-134, :222).
 * Forward: H = sigmoid(X W1) [B x Hd], z = H w2 [B]; w2 and h 16-byte aligned.
 * Backward: given H and g = dL/dz [B], d1 = (g w2^T) * H(1 - H);
 * dW1 = X^T d1 [D x Hd], dW2 = H^T g [Hd]; either output may be null. */
CLEAVE_HIP_API int32_t cleave_hip_sigmoid_hidden_fwd_f32(const float* x, int64_t xlen, const float* w1,
                                                         int64_t w1len, const float* w2, int64_t w2len, float* h,
                                                         int64_t hlen, float* z, int64_t zlen, int32_t B,
                                                         int32_t D, int32_t Hd);
CLEAVE_HIP_API int32_t cleave_hip_sigmoid_hidden_bwd_f32(const float* x, int64_t xlen, const float* h,
                                                         int64_t hlen, const float* w2, int64_t w2len,
                                                         const float* g, int64_t glen, float* dw1, int64_t dw1len,
                                                         float* dw2, int64_t dw2len, int32_t B, int32_t D,
                                                         int32_t Hd);

/* ---------------------------------------------------------------------- */
/* Tensor<f64, ...>                                                         */
/* ---------------------------------------------------------------------- */
/* Every tensor impl of the stdlib is generic over T: Float
 * (stdlib/linalg/tensor.cleave:40, :66-71; stdlib/nn/nn.cleave:82, :111,
 * :119, :141; stdlib/linalg/matrix.cleave:27), and Float covers f64
 * (stdlib/num/num.cleave:50-51, Ring<f64> :189-196).  These are the f32
 * operators above on double operands, with the same argument meaning,
 * lengths in elements, checks and error behaviour; they compute in double
 * throughout (math.exp / math.tanh are the device's double exp / tanh). */

/* C = op(A) op(B) in f64 on the f64 matrix cores (v_mfma_f64_16x16x4f64). */
CLEAVE_HIP_API int32_t cleave_hip_matmul_f64(const double* a, int64_t alen, const double* b, int64_t blen,
                                             double* c, int64_t clen, int32_t M, int32_t N, int32_t K,
                                             int32_t trans_a, int32_t trans_b);
CLEAVE_HIP_API int32_t cleave_hip_matmul_batched_f64(const double* a, int64_t alen, const double* b,
                                                     int64_t blen, double* c, int64_t clen, int32_t batch,
                                                     int32_t M, int32_t N, int32_t K, int32_t trans_a,
                                                     int32_t trans_b);
CLEAVE_HIP_API int32_t cleave_hip_add_f64(const double* a, int64_t alen, const double* b, int64_t blen,
                                          double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_sub_f64(const double* a, int64_t alen, const double* b, int64_t blen,
                                          double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_mul_f64(const double* a, int64_t alen, const double* b, int64_t blen,
                                          double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_div_f64(const double* a, int64_t alen, const double* b, int64_t blen,
                                          double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_neg_f64(const double* a, int64_t alen, double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_zero_f64(double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_relu_f64(const double* x, int64_t xlen, double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_sigmoid_f64(const double* x, int64_t xlen, double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_tanh_f64(const double* x, int64_t xlen, double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_sigmoid_bwd_f64(const double* s, int64_t slen, const double* g, int64_t glen,
                                                  double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_tanh_bwd_f64(const double* t, int64_t tlen, const double* g, int64_t glen,
                                               double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_relu_bwd_f64(const double* x, int64_t xlen, const double* g, int64_t glen,
                                               double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_div_bwd_f64(const double* a, int64_t alen, const double* b, int64_t blen,
                                              const double* g, int64_t glen, double* da, int64_t dalen,
                                              double* db, int64_t dblen);
CLEAVE_HIP_API int32_t cleave_hip_sgd_update_f64(double* w, int64_t wlen, const double* g, int64_t glen,
                                                 double lr);
CLEAVE_HIP_API int32_t cleave_hip_add_row_bias_f64(const double* a, int64_t alen, const double* bias, int64_t blen,
                                                   double* out, int64_t outlen, int32_t rows, int32_t cols);
CLEAVE_HIP_API int32_t cleave_hip_sum_rows_f64(const double* g, int64_t glen, double* out, int64_t outlen,
                                               int32_t rows, int32_t cols);
CLEAVE_HIP_API int32_t cleave_hip_add_bcast_f64(const double* a, int64_t alen, const int32_t* ashape,
                                                int32_t arank, const double* b, int64_t blen, const int32_t* bshape,
                                                int32_t brank, double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_sub_bcast_f64(const double* a, int64_t alen, const int32_t* ashape,
                                                int32_t arank, const double* b, int64_t blen, const int32_t* bshape,
                                                int32_t brank, double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_mul_bcast_f64(const double* a, int64_t alen, const int32_t* ashape,
                                                int32_t arank, const double* b, int64_t blen, const int32_t* bshape,
                                                int32_t brank, double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_div_bcast_f64(const double* a, int64_t alen, const int32_t* ashape,
                                                int32_t arank, const double* b, int64_t blen, const int32_t* bshape,
                                                int32_t brank, double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_sum_to_shape_f64(const double* g, int64_t glen, const int32_t* gshape,
                                                   int32_t grank, double* out, int64_t outlen,
                                                   const int32_t* oshape, int32_t orank);
CLEAVE_HIP_API int32_t cleave_hip_reduce_sum_f64(const double* x, int64_t len, double* out_dev);
CLEAVE_HIP_API int32_t cleave_hip_reduce_max_f64(const double* x, int64_t len, double* max_dev,
                                                 int64_t* argmax_dev);
CLEAVE_HIP_API double cleave_hip_sum_f64(const double* x, int64_t len);
CLEAVE_HIP_API double cleave_hip_mean_f64(const double* x, int64_t len);
CLEAVE_HIP_API double cleave_hip_max_of_f64(const double* x, int64_t len);
CLEAVE_HIP_API int64_t cleave_hip_argmax_f64(const double* x, int64_t len);
CLEAVE_HIP_API double cleave_hip_index_f64(const double* t, int64_t len, const int32_t* dims, int64_t ndims,
                                           const int32_t* idx, int64_t nidx);
CLEAVE_HIP_API int32_t cleave_hip_index_bwd_f64(double g, double* dt, int64_t len, const int32_t* dims,
                                                int64_t ndims, const int32_t* idx, int64_t nidx);

/* ---------------------------------------------------------------------- */
/* Host-array forms                                                         */
/* ---------------------------------------------------------------------- */
/* cleave's extern lowering passes an [T; N] argument as the aligned pointer
 * of a HOST memref and its element count (cleave/src/mlir_lower.rs:1720-1751),
 * and cleave-rt's natives read that memory on the host (sum_bytes,
 * cleave-rt/src/lib.rs:86-90).  Each `_host` entry point below has the
 * signature and argument meaning of the device entry point of the same name
 * without the suffix, but every tensor operand is a borrowed host array
 * (pageable or pinned, valid only during the call).  The call copies the
 * inputs into library staging memory in HBM, runs the same kernels, copies
 * the outputs back and synchronises the library stream before it returns;
 * on error no output array is written.  In-out arrays (w of the SGD update,
 * w1/w2 of the MLP step, dt of index_bwd) are copied both ways.
 * Binding these is the drop-in for an `extern(...)` declaration. */

/* MatMul (stdlib/linalg/matrix.cleave:22-61, product rule :24). */
CLEAVE_HIP_API int32_t cleave_hip_matmul_f32_host(const float* a, int64_t alen, const float* b, int64_t blen,
                                                  float* c, int64_t clen, int32_t M, int32_t N, int32_t K,
                                                  int32_t trans_a, int32_t trans_b);
CLEAVE_HIP_API int32_t cleave_hip_matmul_batched_f32_host(const float* a, int64_t alen, const float* b,
                                                          int64_t blen, float* c, int64_t clen, int32_t batch,
                                                          int32_t M, int32_t N, int32_t K, int32_t trans_a,
                                                          int32_t trans_b);
CLEAVE_HIP_API int32_t cleave_hip_matmul_bf16_host(const uint16_t* a, int64_t alen, const uint16_t* b,
                                                   int64_t blen, float* c, int64_t clen, int32_t M, int32_t N,
                                                   int32_t K, int32_t trans_a, int32_t trans_b);
CLEAVE_HIP_API int32_t cleave_hip_matmul_batched_bf16_host(const uint16_t* a, int64_t alen, const uint16_t* b,
                                                           int64_t blen, float* c, int64_t clen, int32_t batch,
                                                           int32_t M, int32_t N, int32_t K, int32_t trans_a,
                                                           int32_t trans_b);

/* Ring<Tensor> and Activation<Tensor> (stdlib/linalg/tensor.cleave:66-80,
 * stdlib/nn/nn.cleave:82-95). */
CLEAVE_HIP_API int32_t cleave_hip_add_f32_host(const float* a, int64_t alen, const float* b, int64_t blen,
                                               float* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_sub_f32_host(const float* a, int64_t alen, const float* b, int64_t blen,
                                               float* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_mul_f32_host(const float* a, int64_t alen, const float* b, int64_t blen,
                                               float* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_div_f32_host(const float* a, int64_t alen, const float* b, int64_t blen,
                                               float* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_neg_f32_host(const float* a, int64_t alen, float* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_zero_f32_host(float* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_relu_f32_host(const float* x, int64_t xlen, float* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_sigmoid_f32_host(const float* x, int64_t xlen, float* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_tanh_f32_host(const float* x, int64_t xlen, float* out, int64_t outlen);

/* Backward maps (stdlib/num/num.cleave:123-136, :222-223). */
CLEAVE_HIP_API int32_t cleave_hip_sigmoid_bwd_f32_host(const float* s, int64_t slen, const float* g, int64_t glen,
                                                       float* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_tanh_bwd_f32_host(const float* t, int64_t tlen, const float* g, int64_t glen,
                                                    float* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_relu_bwd_f32_host(const float* x, int64_t xlen, const float* g, int64_t glen,
                                                    float* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_div_bwd_f32_host(const float* a, int64_t alen, const float* b, int64_t blen,
                                                   const float* g, int64_t glen, float* da, int64_t dalen,
                                                   float* db, int64_t dblen);
CLEAVE_HIP_API int32_t cleave_hip_sgd_update_f32_host(float* w, int64_t wlen, const float* g, int64_t glen,
                                                      float lr);
CLEAVE_HIP_API int32_t cleave_hip_add_row_bias_f32_host(const float* a, int64_t alen, const float* bias,
                                                        int64_t blen, float* out, int64_t outlen, int32_t rows,
                                                        int32_t cols);
CLEAVE_HIP_API int32_t cleave_hip_sum_rows_f32_host(const float* g, int64_t glen, float* out, int64_t outlen,
                                                    int32_t rows, int32_t cols);
CLEAVE_HIP_API int32_t cleave_hip_add_bcast_f32_host(const float* a, int64_t alen, const int32_t* ashape,
                                                     int32_t arank, const float* b, int64_t blen,
                                                     const int32_t* bshape, int32_t brank, float* out,
                                                     int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_sub_bcast_f32_host(const float* a, int64_t alen, const int32_t* ashape,
                                                     int32_t arank, const float* b, int64_t blen,
                                                     const int32_t* bshape, int32_t brank, float* out,
                                                     int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_mul_bcast_f32_host(const float* a, int64_t alen, const int32_t* ashape,
                                                     int32_t arank, const float* b, int64_t blen,
                                                     const int32_t* bshape, int32_t brank, float* out,
                                                     int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_div_bcast_f32_host(const float* a, int64_t alen, const int32_t* ashape,
                                                     int32_t arank, const float* b, int64_t blen,
                                                     const int32_t* bshape, int32_t brank, float* out,
                                                     int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_sum_to_shape_f32_host(const float* g, int64_t glen, const int32_t* gshape,
                                                        int32_t grank, float* out, int64_t outlen,
                                                        const int32_t* oshape, int32_t orank);

/* Sum / Mean / Max (stdlib/nn/nn.cleave:111-149): the value is returned, as
 * by the stdlib functions; NaN (argmax -1, u64 sum 0) after an error. */
CLEAVE_HIP_API float cleave_hip_sum_f32_host(const float* x, int64_t len);
CLEAVE_HIP_API float cleave_hip_mean_f32_host(const float* x, int64_t len);
CLEAVE_HIP_API float cleave_hip_max_of_f32_host(const float* x, int64_t len);
CLEAVE_HIP_API int64_t cleave_hip_argmax_f32_host(const float* x, int64_t len);
CLEAVE_HIP_API uint64_t cleave_hip_sum_u32_u64_host(const uint32_t* x, int64_t len);
CLEAVE_HIP_API int64_t cleave_hip_sum_i32_i64_host(const int32_t* x, int64_t len);

/* Index<Tensor> (stdlib/linalg/tensor.cleave:113-133). */
CLEAVE_HIP_API float cleave_hip_index_f32_host(const float* t, int64_t len, const int32_t* dims, int64_t ndims,
                                               const int32_t* idx, int64_t nidx);
CLEAVE_HIP_API int32_t cleave_hip_index_bwd_f32_host(float g, float* dt, int64_t len, const int32_t* dims,
                                                     int64_t ndims, const int32_t* idx, int64_t nidx);

/* Tensor<f64, ...> operators on host arrays. */
CLEAVE_HIP_API int32_t cleave_hip_matmul_f64_host(const double* a, int64_t alen, const double* b, int64_t blen,
                                                  double* c, int64_t clen, int32_t M, int32_t N, int32_t K,
                                                  int32_t trans_a, int32_t trans_b);
CLEAVE_HIP_API int32_t cleave_hip_matmul_batched_f64_host(const double* a, int64_t alen, const double* b,
                                                          int64_t blen, double* c, int64_t clen, int32_t batch,
                                                          int32_t M, int32_t N, int32_t K, int32_t trans_a,
                                                          int32_t trans_b);
CLEAVE_HIP_API int32_t cleave_hip_add_f64_host(const double* a, int64_t alen, const double* b, int64_t blen,
                                               double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_sub_f64_host(const double* a, int64_t alen, const double* b, int64_t blen,
                                               double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_mul_f64_host(const double* a, int64_t alen, const double* b, int64_t blen,
                                               double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_div_f64_host(const double* a, int64_t alen, const double* b, int64_t blen,
                                               double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_neg_f64_host(const double* a, int64_t alen, double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_zero_f64_host(double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_relu_f64_host(const double* x, int64_t xlen, double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_sigmoid_f64_host(const double* x, int64_t xlen, double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_tanh_f64_host(const double* x, int64_t xlen, double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_sigmoid_bwd_f64_host(const double* s, int64_t slen, const double* g,
                                                       int64_t glen, double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_tanh_bwd_f64_host(const double* t, int64_t tlen, const double* g, int64_t glen,
                                                    double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_relu_bwd_f64_host(const double* x, int64_t xlen, const double* g, int64_t glen,
                                                    double* out, int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_div_bwd_f64_host(const double* a, int64_t alen, const double* b, int64_t blen,
                                                   const double* g, int64_t glen, double* da, int64_t dalen,
                                                   double* db, int64_t dblen);
CLEAVE_HIP_API int32_t cleave_hip_sgd_update_f64_host(double* w, int64_t wlen, const double* g, int64_t glen,
                                                      double lr);
CLEAVE_HIP_API int32_t cleave_hip_add_row_bias_f64_host(const double* a, int64_t alen, const double* bias,
                                                        int64_t blen, double* out, int64_t outlen, int32_t rows,
                                                        int32_t cols);
CLEAVE_HIP_API int32_t cleave_hip_sum_rows_f64_host(const double* g, int64_t glen, double* out, int64_t outlen,
                                                    int32_t rows, int32_t cols);
CLEAVE_HIP_API int32_t cleave_hip_add_bcast_f64_host(const double* a, int64_t alen, const int32_t* ashape,
                                                     int32_t arank, const double* b, int64_t blen,
                                                     const int32_t* bshape, int32_t brank, double* out,
                                                     int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_sub_bcast_f64_host(const double* a, int64_t alen, const int32_t* ashape,
                                                     int32_t arank, const double* b, int64_t blen,
                                                     const int32_t* bshape, int32_t brank, double* out,
                                                     int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_mul_bcast_f64_host(const double* a, int64_t alen, const int32_t* ashape,
                                                     int32_t arank, const double* b, int64_t blen,
                                                     const int32_t* bshape, int32_t brank, double* out,
                                                     int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_div_bcast_f64_host(const double* a, int64_t alen, const int32_t* ashape,
                                                     int32_t arank, const double* b, int64_t blen,
                                                     const int32_t* bshape, int32_t brank, double* out,
                                                     int64_t outlen);
CLEAVE_HIP_API int32_t cleave_hip_sum_to_shape_f64_host(const double* g, int64_t glen, const int32_t* gshape,
                                                        int32_t grank, double* out, int64_t outlen,
                                                        const int32_t* oshape, int32_t orank);
CLEAVE_HIP_API double cleave_hip_sum_f64_host(const double* x, int64_t len);
CLEAVE_HIP_API double cleave_hip_mean_f64_host(const double* x, int64_t len);
CLEAVE_HIP_API double cleave_hip_max_of_f64_host(const double* x, int64_t len);
CLEAVE_HIP_API int64_t cleave_hip_argmax_f64_host(const double* x, int64_t len);
CLEAVE_HIP_API double cleave_hip_index_f64_host(const double* t, int64_t len, const int32_t* dims, int64_t ndims,
                                                const int32_t* idx, int64_t nidx);
CLEAVE_HIP_API int32_t cleave_hip_index_bwd_f64_host(double g, double* dt, int64_t len, const int32_t* dims,
                                                     int64_t ndims, const int32_t* idx, int64_t nidx);

/* escape_count map (examples/mandelbrot.cleave:14-26). */
CLEAVE_HIP_API int32_t cleave_hip_mandelbrot_u32_host(uint32_t* out, int64_t outlen, int32_t width,
                                                      int32_t height, float x0, float y0, float dx, float dy,
                                                      int32_t max_iter);

/* MLP step (examples/xor_tensor.cleave:38-92 style); `loss` is a host float
 * (one element) when non-null. */
CLEAVE_HIP_API int32_t cleave_hip_mlp_step_f32_host(const float* x, int64_t xlen, const float* y, int64_t ylen,
                                                    float* w1, int64_t w1len, float* w2, int64_t w2len,
                                                    float* dw1, int64_t dw1len, float* dw2, int64_t dw2len,
                                                    float* loss, int32_t B, int32_t D, int32_t Hd, float lr);

/* ---------------------------------------------------------------------- */
/* Output-first forms, for cleave's array-return identity                   */
/* ---------------------------------------------------------------------- */
/* A cleave `extern` whose result type is an array is declared at the C level
 * as returning i64, and the call's cleave result is its FIRST array argument
 * (cleave/src/mlir_lower.rs:1062-1075, :1123-1124; print_bytes,
 * stdlib/io/io.cleave:35).  So an extern that fills an array takes that array
 * first: each `_into` form below is the `_host` form of the same operator
 * with the output array moved to the front and an int64_t result, the output
 * length on success or the `_host` call's negative status.  All arrays are
 * host arrays, as for the `_host` forms; the output is written in place, so
 * the cleave result (the same array) holds it. */

/* c = op(a) * op(b) (stdlib/linalg/matrix.cleave:22-61). */
CLEAVE_HIP_API int64_t cleave_hip_matmul_f32_into(float* c, int64_t clen, const float* a, int64_t alen,
                                                  const float* b, int64_t blen, int32_t M, int32_t N, int32_t K,
                                                  int32_t trans_a, int32_t trans_b);
/* Ring<Tensor> (stdlib/linalg/tensor.cleave:66-71). */
CLEAVE_HIP_API int64_t cleave_hip_add_f32_into(float* out, int64_t outlen, const float* a, int64_t alen,
                                               const float* b, int64_t blen);
CLEAVE_HIP_API int64_t cleave_hip_sub_f32_into(float* out, int64_t outlen, const float* a, int64_t alen,
                                               const float* b, int64_t blen);
CLEAVE_HIP_API int64_t cleave_hip_mul_f32_into(float* out, int64_t outlen, const float* a, int64_t alen,
                                               const float* b, int64_t blen);
CLEAVE_HIP_API int64_t cleave_hip_div_f32_into(float* out, int64_t outlen, const float* a, int64_t alen,
                                               const float* b, int64_t blen);
CLEAVE_HIP_API int64_t cleave_hip_neg_f32_into(float* out, int64_t outlen, const float* x, int64_t xlen);
/* Activation<Tensor> (stdlib/nn/nn.cleave:82-95). */
CLEAVE_HIP_API int64_t cleave_hip_relu_f32_into(float* out, int64_t outlen, const float* x, int64_t xlen);
CLEAVE_HIP_API int64_t cleave_hip_sigmoid_f32_into(float* out, int64_t outlen, const float* x, int64_t xlen);
CLEAVE_HIP_API int64_t cleave_hip_tanh_f32_into(float* out, int64_t outlen, const float* x, int64_t xlen);
/* Backward maps (stdlib/num/num.cleave:123-136, :222-223). */
CLEAVE_HIP_API int64_t cleave_hip_sigmoid_bwd_f32_into(float* out, int64_t outlen, const float* s, int64_t slen,
                                                       const float* g, int64_t glen);
CLEAVE_HIP_API int64_t cleave_hip_tanh_bwd_f32_into(float* out, int64_t outlen, const float* t, int64_t tlen,
                                                    const float* g, int64_t glen);
CLEAVE_HIP_API int64_t cleave_hip_relu_bwd_f32_into(float* out, int64_t outlen, const float* x, int64_t xlen,
                                                    const float* g, int64_t glen);
/* The same on f64 arrays. */
CLEAVE_HIP_API int64_t cleave_hip_matmul_f64_into(double* c, int64_t clen, const double* a, int64_t alen,
                                                  const double* b, int64_t blen, int32_t M, int32_t N, int32_t K,
                                                  int32_t trans_a, int32_t trans_b);
CLEAVE_HIP_API int64_t cleave_hip_add_f64_into(double* out, int64_t outlen, const double* a, int64_t alen,
                                               const double* b, int64_t blen);
CLEAVE_HIP_API int64_t cleave_hip_sub_f64_into(double* out, int64_t outlen, const double* a, int64_t alen,
                                               const double* b, int64_t blen);
CLEAVE_HIP_API int64_t cleave_hip_mul_f64_into(double* out, int64_t outlen, const double* a, int64_t alen,
                                               const double* b, int64_t blen);
CLEAVE_HIP_API int64_t cleave_hip_div_f64_into(double* out, int64_t outlen, const double* a, int64_t alen,
                                               const double* b, int64_t blen);
CLEAVE_HIP_API int64_t cleave_hip_neg_f64_into(double* out, int64_t outlen, const double* x, int64_t xlen);
CLEAVE_HIP_API int64_t cleave_hip_relu_f64_into(double* out, int64_t outlen, const double* x, int64_t xlen);
CLEAVE_HIP_API int64_t cleave_hip_sigmoid_f64_into(double* out, int64_t outlen, const double* x, int64_t xlen);
CLEAVE_HIP_API int64_t cleave_hip_tanh_f64_into(double* out, int64_t outlen, const double* x, int64_t xlen);
CLEAVE_HIP_API int64_t cleave_hip_sigmoid_bwd_f64_into(double* out, int64_t outlen, const double* s, int64_t slen,
                                                       const double* g, int64_t glen);
CLEAVE_HIP_API int64_t cleave_hip_tanh_bwd_f64_into(double* out, int64_t outlen, const double* t, int64_t tlen,
                                                    const double* g, int64_t glen);
CLEAVE_HIP_API int64_t cleave_hip_relu_bwd_f64_into(double* out, int64_t outlen, const double* x, int64_t xlen,
                                                    const double* g, int64_t glen);
/* escape_count over a grid (examples/mandelbrot.cleave:14-26) as i32 counts,
 * escape_count's own return type: the counts of cleave_hip_mandelbrot_u32,
 * which never exceed max_iter, so the bits are the same. */
CLEAVE_HIP_API int64_t cleave_hip_escape_grid_i32(int32_t* out, int64_t outlen, int32_t width, int32_t height,
                                                  float x0, float y0, float dx, float dy, int32_t max_iter);

#ifdef __cplusplus
}
#endif

#endif /* CLEAVE_HIP_H */
