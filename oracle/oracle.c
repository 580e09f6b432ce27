/*
 * oracle.c -- CPU restatement of cleave's tensor hot path (TEST INFRASTRUCTURE).
 *
 * Checker only: loaded by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg, never by the product library.  Build: oracle/Makefile
 * (gcc -O2 -ffp-contract=off -fopenmp).  Each function cites the reference
 * source whose lowered semantics it restates.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* generators                                                               */
/* ------------------------------------------------------------------------ */

static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

/* splitmix64 (Steele, Lea, Flood 2014): state += golden; out = mix(state).
 * The i-th output of a stream seeded with s is mix(s + (i+1)*golden). */
uint64_t or_splitmix64_at(uint64_t seed, uint64_t i) {
    return mix64(seed + (i + 1) * 0x9E3779B97F4A7C15ULL);
}

static float unit24(uint64_t x) { /* [0,1) with 2^-24 spacing, exact in f32 */
    return (float)(x >> 40) * 5.9604644775390625e-08f;
}

void or_fill_uniform_f32(float* out, int64_t n, uint64_t seed, float lo, float hi) {
    const float w = hi - lo;
    for (int64_t i = 0; i < n; ++i) out[i] = lo + w * unit24(or_splitmix64_at(seed, (uint64_t)i));
}

void or_fill_normal_f32(float* out, int64_t n, uint64_t seed, float mean, float std) {
    for (int64_t i = 0; i < n; ++i) {
        uint64_t a = or_splitmix64_at(seed, 2 * (uint64_t)i);
        uint64_t b = or_splitmix64_at(seed, 2 * (uint64_t)i + 1);
        double u1 = ((double)(a >> 11) + 1.0) * 0x1.0p-53; /* (0,1] */
        double u2 = (double)(b >> 11) * 0x1.0p-53;         /* [0,1) */
        double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        out[i] = (float)((double)mean + (double)std * z);
    }
}

uint16_t or_f32_to_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float or_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void or_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = or_f32_to_bf16(in[i]);
}

/* ------------------------------------------------------------------------ */
/* MatMul: linalg.matmul lowered by convert-linalg-to-loops.                */
/* stdlib/linalg/matrix.cleave:59-60 zero-fills C (Ring::zero) and the      */
/* region at cleave/src/mlir_lower.rs:2089-2120 is mulf(in0,in1) then       */
/* addf(out, .), with k the innermost ascending loop.                       */
/* ------------------------------------------------------------------------ */

static inline float a_at(const float* A, int32_t M, int32_t K, int32_t ta, int32_t i, int32_t k) {
    return ta ? A[(int64_t)k * M + i] : A[(int64_t)i * K + k];
}
static inline float b_at(const float* B, int32_t N, int32_t K, int32_t tb, int32_t k, int32_t j) {
    return tb ? B[(int64_t)j * K + k] : B[(int64_t)k * N + j];
}

void or_matmul_f32_rows(const float* A, const float* B, float* C, int32_t M, int32_t N,
                        int32_t K, int32_t trans_a, int32_t trans_b, int32_t row0,
                        int32_t row1) {
    for (int32_t i = row0; i < row1; ++i) {
        for (int32_t j = 0; j < N; ++j) {
            float* c = &C[(int64_t)i * N + j];
            *c = 0.0f;
            for (int32_t k = 0; k < K; ++k) {
                float p = a_at(A, M, K, trans_a, i, k) * b_at(B, N, K, trans_b, k, j);
                *c = *c + p;
            }
        }
    }
}

void or_matmul_f32(const float* A, const float* B, float* C, int32_t M, int32_t N,
                   int32_t K, int32_t trans_a, int32_t trans_b) {
    or_matmul_f32_rows(A, B, C, M, N, K, trans_a, trans_b, 0, M);
}

void or_matmul_f32_mt(const float* A, const float* B, float* C, int32_t M, int32_t N,
                      int32_t K, int32_t trans_a, int32_t trans_b, int32_t threads) {
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
#endif
    for (int32_t i = 0; i < M; ++i)
        or_matmul_f32_rows(A, B, C, M, N, K, trans_a, trans_b, i, i + 1);
    (void)threads;
}

void or_matmul_f32_entries(const float* A, const float* B, int32_t M, int32_t N, int32_t K,
                           int32_t trans_a, int32_t trans_b, const int32_t* ii,
                           const int32_t* jj, int64_t n, float* out, float* absout) {
    for (int64_t e = 0; e < n; ++e) {
        float c = 0.0f;
        double s = 0.0;
        for (int32_t k = 0; k < K; ++k) {
            float a = a_at(A, M, K, trans_a, ii[e], k);
            float b = b_at(B, N, K, trans_b, k, jj[e]);
            c = c + a * b;
            s += fabs((double)a) * fabs((double)b);
        }
        out[e] = c;
        if (absout) absout[e] = (float)s;
    }
}

static inline float bf_at(const uint16_t* X, int64_t idx) { return or_bf16_to_f32(X[idx]); }

void or_matmul_bf16_entries(const uint16_t* A, const uint16_t* B, int32_t M, int32_t N,
                            int32_t K, int32_t trans_a, int32_t trans_b, const int32_t* ii,
                            const int32_t* jj, int64_t n, float* out, float* absout) {
    for (int64_t e = 0; e < n; ++e) {
        float c = 0.0f;
        double s = 0.0;
        for (int32_t k = 0; k < K; ++k) {
            int32_t i = ii[e], j = jj[e];
            float a = trans_a ? bf_at(A, (int64_t)k * M + i) : bf_at(A, (int64_t)i * K + k);
            float b = trans_b ? bf_at(B, (int64_t)j * K + k) : bf_at(B, (int64_t)k * N + j);
            c = c + a * b;
            s += fabs((double)a) * fabs((double)b);
        }
        out[e] = c;
        if (absout) absout[e] = (float)s;
    }
}

void or_matmul_bf16_rows(const uint16_t* A, const uint16_t* B, float* C, int32_t M,
                         int32_t N, int32_t K, int32_t row0, int32_t row1) {
    (void)M;
    for (int32_t i = row0; i < row1; ++i)
        for (int32_t j = 0; j < N; ++j) {
            float* c = &C[(int64_t)i * N + j];
            *c = 0.0f;
            for (int32_t k = 0; k < K; ++k)
                *c = *c + bf_at(A, (int64_t)i * K + k) * bf_at(B, (int64_t)k * N + j);
        }
}

/* ------------------------------------------------------------------------ */
/* Ring<Tensor> (stdlib/linalg/tensor.cleave:66-71): arith.{add,sub,mul,div,neg}f */
/* applied elementwise after elementwise-to-linalg + linalg-to-loops.       */
/* ------------------------------------------------------------------------ */

void or_add_f32(const float* a, const float* b, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}
void or_sub_f32(const float* a, const float* b, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = a[i] - b[i];
}
void or_mul_f32(const float* a, const float* b, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = a[i] * b[i];
}
void or_div_f32(const float* a, const float* b, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = a[i] / b[i];
}
void or_neg_f32(const float* a, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = -a[i];
}

/* arith.maximumf (stdlib/nn/nn.cleave:83-85): IEEE 754-2019 maximum. */
static inline float ieee_maximum(float x, float y) {
    if (isnan(x) || isnan(y)) return x + y; /* propagates a quiet NaN */
    if (x == y) return signbit(x) ? y : x;  /* max(-0,+0) = +0 */
    return x > y ? x : y;
}
void or_relu_f32(const float* a, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = ieee_maximum(a[i], 0.0f);
}

/* stdlib/nn/nn.cleave:87-93: negf, math.exp, addf(one, e), divf(one, denom). */
float or_sigmoid_scalar(float x) {
    float negx = -x;
    float e = expf(negx);
    float denom = 1.0f + e;
    return 1.0f / denom;
}
void or_sigmoid_f32(const float* a, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = or_sigmoid_scalar(a[i]);
}
/* stdlib/nn/nn.cleave:94: math.tanh -> libm tanhf. */
void or_tanh_f32(const float* a, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = tanhf(a[i]);
}

/* ------------------------------------------------------------------------ */
/* backward ops: the reference's derivative rules, in reverse mode.         */
/* sigmoid: d(1/(1+e^-x)) via quotient + exp rules (stdlib/num/num.cleave   */
/* :132-134, :222) = e^-x/(1+e^-x)^2 = s(1-s).                               */
/* tanh: stdlib/num/num.cleave:223, 1 - t^2.                                 */
/* ------------------------------------------------------------------------ */

void or_sigmoid_bwd_f32(const float* s, const float* g, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = g[i] * s[i] * (1.0f - s[i]);
}
void or_tanh_bwd_f32(const float* t, const float* g, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = g[i] * (1.0f - t[i] * t[i]);
}
void or_relu_bwd_f32(const float* x, const float* g, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = x[i] > 0.0f ? g[i] : 0.0f;
}
/* quotient rule, stdlib/num/num.cleave:132-134: d(a/b) = (da*b - a*db)/(b*b). */
void or_div_bwd_f32(const float* a, const float* b, const float* g, float* da, float* db,
                    int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        da[i] = g[i] / b[i];
        db[i] = -(g[i] * a[i]) / (b[i] * b[i]);
    }
}

/* ------------------------------------------------------------------------ */
/* A bias shared by every row: the batched form of the reference's          */
/* same-shape `matmul(x, w) + b1` (examples/xor_tensor.cleave:44-49), and    */
/* its reverse rule (the cotangent summed over the broadcast rows).         */
/* ------------------------------------------------------------------------ */

void or_add_row_bias_f32(const float* a, const float* bias, float* out, int32_t rows, int32_t cols) {
    for (int64_t i = 0; i < rows; ++i)
        for (int64_t j = 0; j < cols; ++j) out[i * cols + j] = a[i * cols + j] + bias[j];
}
/* Left fold down each column from row 0, like Sum (stdlib/nn/nn.cleave:111-117). */
void or_sum_rows_f32(const float* g, float* out, int32_t rows, int32_t cols) {
    for (int64_t j = 0; j < cols; ++j) {
        float acc = g[j];
        for (int64_t i = 1; i < rows; ++i) acc = acc + g[i * cols + j];
        out[j] = acc;
    }
}

/* ------------------------------------------------------------------------ */
/* Broadcasting maps and their reverse rule (extension: the reference's      */
/* Ring<Tensor> maps need equal shapes, stdlib/linalg/tensor.cleave:66-71,   */
/* and Activation<Tensor> is rank 1, stdlib/nn/nn.cleave:82).  numpy's rule: */
/* shapes aligned at their last dimension, a missing leading dimension is 1, */
/* a dimension of 1 stretches to the other operand's.                        */
/* ------------------------------------------------------------------------ */

/* Right-aligns a rank-r shape into R dimensions. */
static void or_align(const int32_t* sh, int32_t r, int R, int64_t* d) {
    for (int i = 0; i < R; ++i) d[i] = i < R - r ? 1 : sh[i - (R - r)];
}

/* The output shape of a broadcast: its rank, or -1 when the shapes do not
 * broadcast (or a rank is outside 0 .. 8). */
static int or_bcast_shape(const int32_t* ash, int32_t ar, const int32_t* bsh, int32_t br, int64_t* da, int64_t* db,
                          int64_t* dn) {
    if (ar < 0 || ar > 8 || br < 0 || br > 8) return -1;
    const int R = ar > br ? (ar > 0 ? ar : 1) : (br > 0 ? br : 1);
    or_align(ash, ar, R, da);
    or_align(bsh, br, R, db);
    for (int i = 0; i < R; ++i) {
        if (da[i] != db[i] && da[i] != 1 && db[i] != 1) return -1;
        dn[i] = da[i] == 1 ? db[i] : da[i];
    }
    return R;
}

/* out = a op b (op 0 add, 1 sub, 2 mul, 3 div), output elements in row-major
 * order, each one IEEE operation on the elements its index maps to.  Returns
 * -1 when the shapes do not broadcast. */
#define OR_BCAST(T, sfx)                                                                                         \
    int32_t or_bcast_##sfx(int32_t op, const T* a, const int32_t* ash, int32_t ar, const T* b,                   \
                           const int32_t* bsh, int32_t br, T* out) {                                             \
        int64_t da[8], db[8], dn[8], idx[8] = {0};                                                               \
        const int R = or_bcast_shape(ash, ar, bsh, br, da, db, dn);                                              \
        if (R < 0) return -1;                                                                                    \
        int64_t total = 1;                                                                                       \
        for (int i = 0; i < R; ++i) total *= dn[i];                                                              \
        for (int64_t o = 0; o < total; ++o) {                                                                    \
            int64_t oa = 0, ob = 0, sa = 1, sb = 1;                                                              \
            for (int i = R - 1; i >= 0; --i) {                                                                   \
                oa += (da[i] == 1 ? 0 : idx[i]) * sa;                                                            \
                ob += (db[i] == 1 ? 0 : idx[i]) * sb;                                                            \
                sa *= da[i];                                                                                     \
                sb *= db[i];                                                                                     \
            }                                                                                                    \
            const T x = a[oa], y = b[ob];                                                                        \
            out[o] = op == 0 ? x + y : op == 1 ? x - y : op == 2 ? x * y : x / y;                                \
            for (int i = R - 1; i >= 0; --i) {                                                                   \
                if (++idx[i] < dn[i]) break;                                                                     \
                idx[i] = 0;                                                                                      \
            }                                                                                                    \
        }                                                                                                        \
        return 0;                                                                                                \
    }
OR_BCAST(float, f32)
OR_BCAST(double, f64)
#undef OR_BCAST

/* out (shape osh, broadcasting to gsh) = g summed over the stretched
 * dimensions: out starts at zero and every element of g, in row-major order,
 * is added into the element its index maps to -- for each output element,
 * its terms in row-major order of the stretched dimensions.  Returns -1 when
 * osh does not broadcast to gsh. */
#define OR_SUM_TO_SHAPE(T, sfx)                                                                                  \
    int32_t or_sum_to_shape_##sfx(const T* g, const int32_t* gsh, int32_t gr, T* out, const int32_t* osh,        \
                                  int32_t orank) {                                                               \
        if (gr < 0 || gr > 8 || orank < 0 || orank > gr) return -1;                                              \
        const int R = gr > 0 ? gr : 1;                                                                           \
        int64_t dg[8], dout[8], so[8], idx[8] = {0};                                                             \
        or_align(gsh, gr, R, dg);                                                                                \
        or_align(osh, orank, R, dout);                                                                           \
        int64_t gtotal = 1, ototal = 1;                                                                          \
        for (int i = R - 1; i >= 0; --i) {                                                                       \
            if (dout[i] != dg[i] && dout[i] != 1) return -1;                                                     \
            so[i] = ototal;                                                                                      \
            ototal *= dout[i];                                                                                   \
            gtotal *= dg[i];                                                                                     \
        }                                                                                                        \
        for (int64_t o = 0; o < ototal; ++o) out[o] = 0;                                                         \
        for (int64_t e = 0; e < gtotal; ++e) {                                                                   \
            int64_t oo = 0;                                                                                      \
            for (int i = 0; i < R; ++i) oo += (dout[i] == 1 ? 0 : idx[i]) * so[i];                               \
            out[oo] = out[oo] + g[e];                                                                            \
            for (int i = R - 1; i >= 0; --i) {                                                                   \
                if (++idx[i] < dg[i]) break;                                                                     \
                idx[i] = 0;                                                                                      \
            }                                                                                                    \
        }                                                                                                        \
        return 0;                                                                                                \
    }
OR_SUM_TO_SHAPE(float, f32)
OR_SUM_TO_SHAPE(double, f64)
#undef OR_SUM_TO_SHAPE

/* ------------------------------------------------------------------------ */
/* Index (stdlib/linalg/tensor.cleave:113-133): tensor.extract over the     */
/* row-major buffer (cleave/src/mlir_lower.rs:1968-2002).                   */
/* ------------------------------------------------------------------------ */

static int64_t or_flat_offset(const int32_t* dims, int32_t ndims, const int32_t* idx) {
    int64_t off = 0;
    for (int32_t d = 0; d < ndims; ++d) {
        if (dims[d] <= 0 || idx[d] < 0 || idx[d] >= dims[d]) return -1;
        off = off * dims[d] + idx[d];
    }
    return off;
}
int32_t or_index_f32(const float* t, const int32_t* dims, int32_t ndims, const int32_t* idx,
                     float* out) {
    const int64_t off = or_flat_offset(dims, ndims, idx);
    if (off < 0) return -1;
    *out = t[off];
    return 0;
}
/* `derivative index(c, idx): index(d(c), idx)` in reverse form: the cotangent
 * of c gains g at idx; repeated reads of one element accumulate. */
int32_t or_index_bwd_f32(float g, float* dt, const int32_t* dims, int32_t ndims,
                         const int32_t* idx) {
    const int64_t off = or_flat_offset(dims, ndims, idx);
    if (off < 0) return -1;
    dt[off] = dt[off] + g;
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Sum / Mean / Max (stdlib/nn/nn.cleave:111-149).                          */
/* ------------------------------------------------------------------------ */

float or_sum_f32(const float* v, int64_t n) {
    float acc = v[0];
    for (int64_t i = 1; i < n; ++i) acc = acc + v[i];
    return acc;
}
float or_mean_f32(const float* v, int64_t n) { return or_sum_f32(v, n) / (float)n; }
float or_max_of_f32(const float* v, int64_t n) {
    float acc = v[0];
    for (int64_t i = 1; i < n; ++i)
        if (v[i] > acc) acc = v[i]; /* cmpf ogt: false when either side is NaN */
    return acc;
}
int64_t or_argmax_f32(const float* v, int64_t n) {
    float acc = v[0];
    int64_t idx = 0;
    for (int64_t i = 1; i < n; ++i)
        if (v[i] > acc) {
            acc = v[i];
            idx = i;
        }
    return idx;
}
uint64_t or_sum_u32_u64(const uint32_t* v, int64_t n) {
    uint64_t s = 0;
    for (int64_t i = 0; i < n; ++i) s += v[i];
    return s;
}

/* ------------------------------------------------------------------------ */
/* escape_count (examples/mandelbrot.cleave:14-26) with Complex mul/add     */
/* (stdlib/complex/complex.cleave:25-32) and magnitude_sq (:54), in f32.    */
/* ------------------------------------------------------------------------ */

uint32_t or_escape_count_f32(float cr, float ci, int32_t max_iter) {
    float zr = 0.0f, zi = 0.0f;
    for (int32_t n = 0; n < max_iter; ++n) {
        float re = zr * zr - zi * zi; /* x.real*y.real - x.imag*y.imag */
        float im = zr * zi + zi * zr; /* x.real*y.imag + x.imag*y.real */
        zr = re + cr;
        zi = im + ci;
        if (zr * zr + zi * zi > 4.0f) return (uint32_t)n;
    }
    return (uint32_t)max_iter;
}

uint32_t or_escape_count_latch_f32(float cr, float ci, int32_t max_iter) {
    float zr = 0.0f, zi = 0.0f;
    int32_t count = max_iter, escaped = 0;
    for (int32_t n = 0; n < max_iter; ++n) {
        float re = zr * zr - zi * zi;
        float im = zr * zi + zi * zr;
        zr = re + cr;
        zi = im + ci;
        if (!escaped && (zr * zr + zi * zi > 4.0f)) {
            escaped = 1;
            count = n;
        }
    }
    return (uint32_t)count;
}

void or_mandelbrot_rows(uint32_t* out, int32_t width, int32_t height, float x0, float y0,
                        float dx, float dy, int32_t max_iter, int32_t row0, int32_t row1) {
    (void)height;
    for (int32_t r = row0; r < row1; ++r) {
        float ci = y0 + (float)r * dy;
        for (int32_t c = 0; c < width; ++c) {
            float cr = x0 + (float)c * dx;
            out[(int64_t)r * width + c] = or_escape_count_f32(cr, ci, max_iter);
        }
    }
}

void or_mandelbrot_rows_mt(uint32_t* out, int32_t width, int32_t height, float x0, float y0,
                           float dx, float dy, int32_t max_iter, int32_t row0, int32_t row1,
                           int32_t threads) {
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
#endif
    for (int32_t r = row0; r < row1; ++r)
        or_mandelbrot_rows(out, width, height, x0, y0, dx, dy, max_iter, r, r + 1);
    (void)threads;
}

void or_mandelbrot_mt(uint32_t* out, int32_t width, int32_t height, float x0, float y0,
                      float dx, float dy, int32_t max_iter, int32_t threads) {
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
#endif
    for (int32_t r = 0; r < height; ++r)
        or_mandelbrot_rows(out, width, height, x0, y0, dx, dy, max_iter, r, r + 1);
    (void)threads;
}

/* ------------------------------------------------------------------------ */
/* 2-layer MLP step in the style of examples/xor_tensor.cleave:38-92 with   */
/* the config's batch mean and no biases.  Forward ops follow the stdlib    */
/* bodies above; the backward applies the reference's derivative rules     */
/* (matmul product rule stdlib/linalg/matrix.cleave:24 in reverse mode,     */
/* d(e*e) = de*e + e*de, sigmoid' = s(1-s), d(sum/N) = d(sum)/N).           */
/* ------------------------------------------------------------------------ */

float or_mlp_step_f32(const float* X, const float* y, float* W1, float* W2, int32_t B,
                      int32_t D, int32_t Hd, float lr, float* dW1, float* dW2,
                      int32_t threads) {
    if (threads < 1) threads = 1;
    float* H = (float*)malloc(sizeof(float) * (size_t)B * (size_t)Hd);
    float* d2 = (float*)malloc(sizeof(float) * (size_t)B);
    /* H = sigmoid(X W1) */
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(threads)
#endif
    for (int32_t m = 0; m < B; ++m) {
        float* h = &H[(int64_t)m * Hd];
        for (int32_t n = 0; n < Hd; ++n) h[n] = 0.0f;
        for (int32_t k = 0; k < D; ++k) {
            float x = X[(int64_t)m * D + k];
            const float* w = &W1[(int64_t)k * Hd];
            for (int32_t n = 0; n < Hd; ++n) h[n] = h[n] + x * w[n]; /* k ascending per (m,n) */
        }
        for (int32_t n = 0; n < Hd; ++n) h[n] = or_sigmoid_scalar(h[n]);
    }
    /* yhat = sigmoid(H W2); e = yhat - y; loss = mean(e*e) */
    float acc = 0.0f;
    for (int32_t m = 0; m < B; ++m) {
        const float* h = &H[(int64_t)m * Hd];
        float z = 0.0f;
        for (int32_t n = 0; n < Hd; ++n) z = z + h[n] * W2[n];
        float yh = or_sigmoid_scalar(z);
        float e = yh - y[m];
        float sq = e * e;
        acc = (m == 0) ? sq : acc + sq;
        float gy = (e + e) / (float)B;     /* d(e*e)/dyhat = e + e; mean divides by N */
        d2[m] = gy * yh * (1.0f - yh);     /* sigmoid' = s(1-s) */
    }
    float loss = acc / (float)B;
    /* dW2 = H^T d2 (m ascending) */
    for (int32_t n = 0; n < Hd; ++n) dW2[n] = 0.0f;
    for (int32_t m = 0; m < B; ++m) {
        const float* h = &H[(int64_t)m * Hd];
        for (int32_t n = 0; n < Hd; ++n) dW2[n] = dW2[n] + h[n] * d2[m];
    }
    /* d1 = (d2 W2^T) * H(1-H), written over H; dW1 = X^T d1 (m ascending) */
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(threads)
#endif
    for (int32_t m = 0; m < B; ++m) {
        float* h = &H[(int64_t)m * Hd];
        for (int32_t n = 0; n < Hd; ++n) {
            float g = d2[m] * W2[n];
            h[n] = g * h[n] * (1.0f - h[n]);
        }
    }
    /* Blocks of 32 rows of dW1 per task, m outermost inside a block: every
       entry dW1[k][n] is still its m-ascending chain of unfused mul/add, but
       a block's 32 rows stay in cache while the d1 rows stream past once per
       block (one k at a time re-read all of d1 for every k). */
    const int32_t KB = 32;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(threads)
#endif
    for (int32_t kb = 0; kb < D; kb += KB) {
        const int32_t ke = kb + KB < D ? kb + KB : D;
        for (int32_t k = kb; k < ke; ++k)
            for (int32_t n = 0; n < Hd; ++n) dW1[(int64_t)k * Hd + n] = 0.0f;
        for (int32_t m = 0; m < B; ++m) {
            const float* d1 = &H[(int64_t)m * Hd];
            for (int32_t k = kb; k < ke; ++k) {
                float x = X[(int64_t)m * D + k];
                float* dw = &dW1[(int64_t)k * Hd];
                for (int32_t n = 0; n < Hd; ++n) dw[n] = dw[n] + x * d1[n];
            }
        }
    }
    if (lr != 0.0f) {
        for (int64_t i = 0; i < (int64_t)D * Hd; ++i) W1[i] = W1[i] - lr * dW1[i];
        for (int32_t n = 0; n < Hd; ++n) W2[n] = W2[n] - lr * dW2[n];
    }
    free(H);
    free(d2);
    return loss;
}

/* Selected gradient entries of the step above, for checks at sizes where
 * the whole step is too slow.  The forward pass, d2 and the loss are computed
 * exactly as in or_mlp_step_f32 (rows split over threads; the row products
 * run 4 columns per vector instruction, each column still one k-ascending
 * chain of unfused mul/add, so the bits are those of the scalar loop).  Then
 * dW2[n2[e]] = sum_m h[m,n] d2[m] and dW1[k1[e], n1[e]] = sum_m x[m,k] d1[m,n],
 * d1 = (d2[m] W2[n]) h (1 - h), each m-ascending as in or_mlp_step_f32.
 * abs1/abs2 receive the sums of |operand products| (the GEMM tolerance's
 * denominators).  Returns the loss, or NaN when Hd % 4 != 0. */
typedef float or_v4f __attribute__((vector_size(16)));

float or_mlp_grad_entries(const float* X, const float* y, const float* W1, const float* W2,
                          int32_t B, int32_t D, int32_t Hd, const int32_t* k1, const int32_t* n1,
                          int64_t e1, float* dw1, float* abs1, const int32_t* n2, int64_t e2,
                          float* dw2, float* abs2, int32_t threads) {
    if (threads < 1) threads = 1;
    if (Hd % 4 != 0) return NAN;
    /* columns of H the sampled entries read, in one list */
    int32_t* col_of = (int32_t*)malloc(sizeof(int32_t) * (size_t)Hd);
    for (int32_t n = 0; n < Hd; ++n) col_of[n] = -1;
    int32_t ncols = 0;
    for (int64_t e = 0; e < e1; ++e)
        if (col_of[n1[e]] < 0) col_of[n1[e]] = ncols++;
    for (int64_t e = 0; e < e2; ++e)
        if (col_of[n2[e]] < 0) col_of[n2[e]] = ncols++;
    int32_t* cols = (int32_t*)malloc(sizeof(int32_t) * (size_t)(ncols > 0 ? ncols : 1));
    for (int32_t n = 0; n < Hd; ++n)
        if (col_of[n] >= 0) cols[col_of[n]] = n;
    float* Hs = (float*)malloc(sizeof(float) * (size_t)B * (size_t)(ncols > 0 ? ncols : 1));
    float* d2 = (float*)malloc(sizeof(float) * (size_t)B);
    float* sq = (float*)malloc(sizeof(float) * (size_t)B);
#ifdef _OPENMP
#pragma omp parallel num_threads(threads)
#endif
    {
        float* h = (float*)malloc(sizeof(float) * (size_t)Hd);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int32_t m = 0; m < B; ++m) {
            for (int32_t n = 0; n < Hd; ++n) h[n] = 0.0f;
            for (int32_t k = 0; k < D; ++k) {
                const float x = X[(int64_t)m * D + k];
                const or_v4f xv = {x, x, x, x};
                const float* w = &W1[(int64_t)k * Hd];
                for (int32_t n = 0; n < Hd; n += 4) {
                    or_v4f hv, wv;
                    memcpy(&hv, &h[n], sizeof hv);
                    memcpy(&wv, &w[n], sizeof wv);
                    hv = hv + xv * wv; /* per column: h = h + x*w, k ascending */
                    memcpy(&h[n], &hv, sizeof hv);
                }
            }
            for (int32_t n = 0; n < Hd; ++n) h[n] = or_sigmoid_scalar(h[n]);
            float z = 0.0f;
            for (int32_t n = 0; n < Hd; ++n) z = z + h[n] * W2[n];
            const float yh = or_sigmoid_scalar(z);
            const float e = yh - y[m];
            sq[m] = e * e;
            const float gy = (e + e) / (float)B;
            d2[m] = gy * yh * (1.0f - yh);
            for (int32_t c = 0; c < ncols; ++c) Hs[(int64_t)m * ncols + c] = h[cols[c]];
        }
        free(h);
    }
    float acc = 0.0f;
    for (int32_t m = 0; m < B; ++m) acc = (m == 0) ? sq[m] : acc + sq[m];
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
#endif
    for (int64_t e = 0; e < e2; ++e) {
        const int32_t c = col_of[n2[e]];
        float g = 0.0f;
        double a = 0.0;
        for (int32_t m = 0; m < B; ++m) {
            const float hv = Hs[(int64_t)m * ncols + c];
            g = g + hv * d2[m];
            a += fabs((double)hv) * fabs((double)d2[m]);
        }
        dw2[e] = g;
        if (abs2) abs2[e] = (float)a;
    }
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
#endif
    for (int64_t e = 0; e < e1; ++e) {
        const int32_t c = col_of[n1[e]], k = k1[e];
        const float w2 = W2[n1[e]];
        float g = 0.0f;
        double a = 0.0;
        for (int32_t m = 0; m < B; ++m) {
            const float hv = Hs[(int64_t)m * ncols + c];
            const float d1 = (d2[m] * w2) * hv * (1.0f - hv);
            const float x = X[(int64_t)m * D + k];
            g = g + x * d1;
            a += fabs((double)x) * fabs((double)d1);
        }
        dw1[e] = g;
        if (abs1) abs1[e] = (float)a;
    }
    free(col_of);
    free(cols);
    free(Hs);
    free(d2);
    free(sq);
    return acc / (float)B;
}

double or_mlp_loss_f64(const float* X, const float* y, const float* W1, const float* W2,
                       int32_t B, int32_t D, int32_t Hd) {
    double loss = 0.0;
    for (int32_t m = 0; m < B; ++m) {
        double z2 = 0.0;
        for (int32_t n = 0; n < Hd; ++n) {
            double z = 0.0;
            for (int32_t k = 0; k < D; ++k) z += (double)X[(int64_t)m * D + k] * W1[(int64_t)k * Hd + n];
            double h = 1.0 / (1.0 + exp(-z));
            z2 += h * W2[n];
        }
        double yh = 1.0 / (1.0 + exp(-z2));
        double e = yh - y[m];
        loss += e * e;
    }
    return loss / B;
}

/* ------------------------------------------------------------------------ */
/* examples/xor_tensor.cleave:38-92 (forward :47-56, loss :58-62, loop :81-92) */
/* ------------------------------------------------------------------------ */

typedef struct {
    float w[4], b1[2], w2[2], b2;
} xor_params;

static float xor_forward(const xor_params* p, float x1, float x2, float* h0, float* h1) {
    /* z = matmul(x, w) + b1: k-ascending matmul, then the Ring add */
    float z0 = 0.0f, z1 = 0.0f;
    z0 = z0 + x1 * p->w[0];
    z0 = z0 + x2 * p->w[2];
    z1 = z1 + x1 * p->w[1];
    z1 = z1 + x2 * p->w[3];
    z0 = z0 + p->b1[0];
    z1 = z1 + p->b1[1];
    *h0 = or_sigmoid_scalar(z0);
    *h1 = or_sigmoid_scalar(z1);
    float o = 0.0f;
    o = o + *h0 * p->w2[0];
    o = o + *h1 * p->w2[1];
    o = o + p->b2;
    return or_sigmoid_scalar(o);
}

void or_xor_tensor_train(int32_t steps, float lr, float* preds4) {
    xor_params p = {{0.5f, 0.5f, 0.5f, -0.5f}, {-0.2f, -0.2f}, {1.0f, -1.0f}, 0.0f};
    const float xs1[4] = {0.0f, 0.0f, 1.0f, 1.0f}, xs2[4] = {0.0f, 1.0f, 0.0f, 1.0f};
    const float ys[4] = {0.0f, 1.0f, 1.0f, 0.0f};
    for (int32_t step = 0; step < steps; ++step) {
        int i = step % 4;
        float h0, h1;
        float pred = xor_forward(&p, xs1[i], xs2[i], &h0, &h1);
        float e = pred - ys[i];
        float dpred = e + e;                          /* d(e*e) = de*e + e*de */
        float dout = dpred * pred * (1.0f - pred);    /* sigmoid' = s(1-s) */
        float dh0 = dout * p.w2[0], dh1 = dout * p.w2[1];
        float dz0 = dh0 * h0 * (1.0f - h0), dz1 = dh1 * h1 * (1.0f - h1);
        float g_w[4] = {dz0 * xs1[i], dz1 * xs1[i], dz0 * xs2[i], dz1 * xs2[i]};
        float g_w2[2] = {dout * h0, dout * h1};
        for (int k = 0; k < 4; ++k) p.w[k] = p.w[k] - lr * g_w[k];
        p.b1[0] = p.b1[0] - lr * dz0;
        p.b1[1] = p.b1[1] - lr * dz1;
        p.w2[0] = p.w2[0] - lr * g_w2[0];
        p.w2[1] = p.w2[1] - lr * g_w2[1];
        p.b2 = p.b2 - lr * dout;
    }
    for (int r = 0; r < 4; ++r) {
        float h0, h1;
        preds4[r] = xor_forward(&p, xs1[r], xs2[r], &h0, &h1);
    }
}

/* ======================================================================== */
/* f64: the same operators on Tensor<f64, ...>.  Every tensor impl is       */
/* generic over T: Float (stdlib/linalg/tensor.cleave:40, :66-71;           */
/* stdlib/nn/nn.cleave:82, :111, :119, :141; stdlib/linalg/matrix.cleave:27) */
/* and Float covers f64 (stdlib/num/num.cleave:50-51, Ring<f64> :189-196),  */
/* so the lowered ops are the f32 ones above in double: addf/mulf/... on    */
/* f64, math.exp / math.tanh through libm's exp / tanh.                     */
/* ======================================================================== */

static inline double a_at64(const double* A, int32_t M, int32_t K, int32_t ta, int32_t i, int32_t k) {
    return ta ? A[(int64_t)k * M + i] : A[(int64_t)i * K + k];
}
static inline double b_at64(const double* B, int32_t N, int32_t K, int32_t tb, int32_t k, int32_t j) {
    return tb ? B[(int64_t)j * K + k] : B[(int64_t)k * N + j];
}

/* linalg.matmul on f64 (matrix.cleave:59-60, region mlir_lower.rs:2089-2120):
 * C = 0, then for k ascending C = C + (a * b), each op rounded. */
void or_matmul_f64_rows(const double* A, const double* B, double* C, int32_t M, int32_t N, int32_t K,
                        int32_t trans_a, int32_t trans_b, int32_t row0, int32_t row1) {
    for (int32_t i = row0; i < row1; ++i)
        for (int32_t j = 0; j < N; ++j) {
            double c = 0.0;
            for (int32_t k = 0; k < K; ++k) {
                double p = a_at64(A, M, K, trans_a, i, k) * b_at64(B, N, K, trans_b, k, j);
                c = c + p;
            }
            C[(int64_t)i * N + j] = c;
        }
}

void or_matmul_f64_mt(const double* A, const double* B, double* C, int32_t M, int32_t N, int32_t K,
                      int32_t trans_a, int32_t trans_b, int32_t threads) {
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
#endif
    for (int32_t i = 0; i < M; ++i) or_matmul_f64_rows(A, B, C, M, N, K, trans_a, trans_b, i, i + 1);
    (void)threads;
}

void or_add_f64(const double* a, const double* b, double* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}
void or_sub_f64(const double* a, const double* b, double* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = a[i] - b[i];
}
void or_mul_f64(const double* a, const double* b, double* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = a[i] * b[i];
}
void or_div_f64(const double* a, const double* b, double* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = a[i] / b[i];
}
void or_neg_f64(const double* a, double* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = -a[i];
}
/* arith.maximumf on f64 (nn.cleave:83-85). */
static inline double ieee_maximum64(double x, double y) {
    if (isnan(x) || isnan(y)) return x + y;
    if (x == y) return signbit(x) ? y : x;
    return x > y ? x : y;
}
void or_relu_f64(const double* a, double* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = ieee_maximum64(a[i], 0.0);
}
/* nn.cleave:87-93 on f64: negf, math.exp (libm exp), addf(1, e), divf(1, .). */
double or_sigmoid_f64_scalar(double x) {
    double e = exp(-x);
    double denom = 1.0 + e;
    return 1.0 / denom;
}
void or_sigmoid_f64(const double* a, double* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = or_sigmoid_f64_scalar(a[i]);
}
void or_tanh_f64(const double* a, double* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = tanh(a[i]);
}
void or_sigmoid_bwd_f64(const double* s, const double* g, double* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = g[i] * s[i] * (1.0 - s[i]);
}
void or_tanh_bwd_f64(const double* t, const double* g, double* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = g[i] * (1.0 - t[i] * t[i]);
}
void or_relu_bwd_f64(const double* x, const double* g, double* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = x[i] > 0.0 ? g[i] : 0.0;
}
void or_div_bwd_f64(const double* a, const double* b, const double* g, double* da, double* db, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        da[i] = g[i] / b[i];
        db[i] = -(g[i] * a[i]) / (b[i] * b[i]);
    }
}
void or_add_row_bias_f64(const double* a, const double* bias, double* out, int32_t rows, int32_t cols) {
    for (int64_t i = 0; i < rows; ++i)
        for (int64_t j = 0; j < cols; ++j) out[i * cols + j] = a[i * cols + j] + bias[j];
}
void or_sum_rows_f64(const double* g, double* out, int32_t rows, int32_t cols) {
    for (int64_t j = 0; j < cols; ++j) {
        double acc = g[j];
        for (int64_t i = 1; i < rows; ++i) acc = acc + g[i * cols + j];
        out[j] = acc;
    }
}
int32_t or_index_f64(const double* t, const int32_t* dims, int32_t ndims, const int32_t* idx, double* out) {
    const int64_t off = or_flat_offset(dims, ndims, idx);
    if (off < 0) return -1;
    *out = t[off];
    return 0;
}
int32_t or_index_bwd_f64(double g, double* dt, const int32_t* dims, int32_t ndims, const int32_t* idx) {
    const int64_t off = or_flat_offset(dims, ndims, idx);
    if (off < 0) return -1;
    dt[off] = dt[off] + g;
    return 0;
}
/* Sum / Mean / Max on f64 (nn.cleave:111-149): left fold from v[0];
 * mean = sum / N.to() (sitofp to f64); strict-> first-wins max. */
double or_sum_f64(const double* v, int64_t n) {
    double acc = v[0];
    for (int64_t i = 1; i < n; ++i) acc = acc + v[i];
    return acc;
}
double or_mean_f64(const double* v, int64_t n) { return or_sum_f64(v, n) / (double)n; }
double or_max_of_f64(const double* v, int64_t n) {
    double acc = v[0];
    for (int64_t i = 1; i < n; ++i)
        if (v[i] > acc) acc = v[i];
    return acc;
}
int64_t or_argmax_f64(const double* v, int64_t n) {
    double acc = v[0];
    int64_t idx = 0;
    for (int64_t i = 1; i < n; ++i)
        if (v[i] > acc) {
            acc = v[i];
            idx = i;
        }
    return idx;
}
