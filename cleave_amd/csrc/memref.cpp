// memref.cpp -- the MLIR memref-descriptor forms of the tensor operators
// (include/cleave_hip_memref.h).  Each entry point reads its unranked
// descriptors, checks rank, shape and strides on the host, and calls the
// pointer form from cleave_hip.h, so kernels, validation of the pointer
// forms and the error contract are shared.
#include <cmath>
#include <cstdint>

#include "../../include/cleave_hip_memref.h"
#include "common.hpp"

namespace {

constexpr int kMaxRank = 8;

// One operand: element address and the ranked descriptor's sizes/strides.
struct View {
    char* data = nullptr;
    int64_t rank = 0;
    const int64_t* sizes = nullptr;
    const int64_t* strides = nullptr;
    int64_t count = 1;  // product of sizes
};

// Ranked descriptor layout: allocated, aligned, offset, sizes[rank], strides[rank].
int32_t read_view(cleave_hip_mr m, int esz, const char* fn, const char* arg, View* v) {
    CH_REQUIRE(m != nullptr && m->descriptor != nullptr, "%s: %s: null memref descriptor", fn, arg);
    CH_REQUIRE(m->rank >= 0 && m->rank <= kMaxRank, "%s: %s: rank %lld outside 0..%d", fn, arg,
               (long long)m->rank, kMaxRank);
    auto* words = static_cast<int64_t*>(m->descriptor);
    char* aligned = reinterpret_cast<char*>(static_cast<uintptr_t>(words[1]));
    const int64_t offset = words[2];
    v->rank = m->rank;
    v->sizes = words + 3;
    v->strides = words + 3 + m->rank;
    v->count = 1;
    for (int64_t i = 0; i < v->rank; ++i) {
        CH_REQUIRE(v->sizes[i] >= 0, "%s: %s: negative size %lld in dim %lld", fn, arg,
                   (long long)v->sizes[i], (long long)i);
        CH_REQUIRE(v->sizes[i] == 0 || v->count <= INT64_MAX / v->sizes[i],
                   "%s: %s: element count past int64 at dim %lld", fn, arg, (long long)i);
        v->count *= v->sizes[i];
    }
    CH_REQUIRE(offset >= 0, "%s: %s: negative offset %lld", fn, arg, (long long)offset);
    CH_REQUIRE(v->count == 0 || aligned != nullptr, "%s: %s: null data pointer", fn, arg);
    v->data = aligned + offset * esz;
    return CLEAVE_HIP_OK;
}

// Row-major contiguous: stride of dim i is the product of the sizes after it
// (a dim of size 1 may carry any stride).
bool row_major(const View& v, int64_t first = 0) {
    int64_t want = 1;
    for (int64_t i = v.rank - 1; i >= first; --i) {
        if (v.sizes[i] != 1 && v.strides[i] != want) return false;
        want *= v.sizes[i];
    }
    return true;
}

bool same_sizes(const View& a, const View& b) {
    if (a.rank != b.rank) return false;
    for (int64_t i = 0; i < a.rank; ++i)
        if (a.sizes[i] != b.sizes[i]) return false;
    return true;
}

// An element-wise operand: contiguous, and (when ref is given) shaped like ref.
int32_t flat_view(cleave_hip_mr m, int esz, const char* fn, const char* arg, const View* ref, View* v) {
    int32_t st = read_view(m, esz, fn, arg, v);
    if (st != CLEAVE_HIP_OK) return st;
    CH_REQUIRE(row_major(*v), "%s: %s: not row-major contiguous", fn, arg);
    if (ref) CH_REQUIRE(same_sizes(*ref, *v), "%s: %s: shape differs from the first operand (no broadcasting)", fn, arg);
    return CLEAVE_HIP_OK;
}

// A matmul operand of rank r = 2 or 3 (leading batch): logical [.., rows x cols],
// stored row-major (trans = 0) or as the transpose of a row-major buffer (trans = 1).
int32_t mat_view(cleave_hip_mr m, int esz, const char* fn, const char* arg, View* v, int* trans) {
    int32_t st = read_view(m, esz, fn, arg, v);
    if (st != CLEAVE_HIP_OK) return st;
    CH_REQUIRE(v->rank == 2 || v->rank == 3, "%s: %s: rank %lld, expected 2 (or 3 with a batch)", fn, arg,
               (long long)v->rank);
    const int64_t r = v->rank, rows = v->sizes[r - 2], cols = v->sizes[r - 1];
    const int64_t rs = v->strides[r - 2], cs = v->strides[r - 1];
    const bool batch_ok = r == 2 || v->sizes[0] == 1 || v->strides[0] == rows * cols;
    CH_REQUIRE(batch_ok, "%s: %s: batch entries are not packed back to back", fn, arg);
    if ((rows == 1 || rs == cols) && (cols == 1 || cs == 1)) {
        *trans = 0;
    } else if ((rows == 1 || rs == 1) && (cols == 1 || cs == rows)) {
        *trans = 1;
    } else {
        return ch::fail(CLEAVE_HIP_ERR_ARG, "%s: %s: strides {%lld, %lld} are neither row-major nor transposed",
                        fn, arg, (long long)rs, (long long)cs);
    }
    return CLEAVE_HIP_OK;
}

int32_t narrow(int64_t x, const char* fn, const char* what, int32_t* out) {
    CH_REQUIRE(x >= 0 && x <= INT32_MAX, "%s: %s %lld does not fit int32", fn, what, (long long)x);
    *out = (int32_t)x;
    return CLEAVE_HIP_OK;
}

#define CH_TRY(expr)                                  \
    do {                                              \
        int32_t _st = (expr);                         \
        if (_st != CLEAVE_HIP_OK) return _st;         \
    } while (0)

// Pointer forms of one product element type: the single and the batched one.
template <class TA, class TC>
struct MatmulFns {
    int32_t (*single)(const TA*, int64_t, const TA*, int64_t, TC*, int64_t, int32_t, int32_t, int32_t, int32_t,
                      int32_t);
    int32_t (*batched)(const TA*, int64_t, const TA*, int64_t, TC*, int64_t, int32_t, int32_t, int32_t, int32_t,
                       int32_t, int32_t);
};

template <class TA, class TC>
int32_t matmul_mr(MatmulFns<TA, TC> f, cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr c, const char* fn) {
    View A, B, C;
    int ta = 0, tb = 0, tc = 0;
    CH_TRY(mat_view(a, sizeof(TA), fn, "a", &A, &ta));
    CH_TRY(mat_view(b, sizeof(TA), fn, "b", &B, &tb));
    CH_TRY(mat_view(c, sizeof(TC), fn, "c", &C, &tc));
    CH_REQUIRE(A.rank == B.rank && B.rank == C.rank, "%s: operand ranks differ (%lld, %lld, %lld)", fn,
               (long long)A.rank, (long long)B.rank, (long long)C.rank);
    CH_REQUIRE(tc == 0, "%s: c must be row-major", fn);
    const int64_t r = A.rank;
    const int64_t M = A.sizes[r - 2], K = A.sizes[r - 1], N = B.sizes[r - 1];
    CH_REQUIRE(B.sizes[r - 2] == K && C.sizes[r - 2] == M && C.sizes[r - 1] == N,
               "%s: shapes [%lld x %lld] * [%lld x %lld] -> [%lld x %lld] do not chain", fn, (long long)M,
               (long long)K, (long long)B.sizes[r - 2], (long long)N, (long long)C.sizes[r - 2],
               (long long)C.sizes[r - 1]);
    int32_t m32, n32, k32;
    CH_TRY(narrow(M, fn, "M", &m32));
    CH_TRY(narrow(N, fn, "N", &n32));
    CH_TRY(narrow(K, fn, "K", &k32));
    const TA* ap = reinterpret_cast<const TA*>(A.data);
    const TA* bp = reinterpret_cast<const TA*>(B.data);
    TC* cp = reinterpret_cast<TC*>(C.data);
    if (r == 2) return f.single(ap, A.count, bp, B.count, cp, C.count, m32, n32, k32, ta, tb);
    CH_REQUIRE(A.sizes[0] == B.sizes[0] && B.sizes[0] == C.sizes[0], "%s: batch sizes differ", fn);
    int32_t batch;
    CH_TRY(narrow(A.sizes[0], fn, "batch", &batch));
    return f.batched(ap, A.count, bp, B.count, cp, C.count, batch, m32, n32, k32, ta, tb);
}

template <class T>
int32_t map1_mr(int32_t (*f)(const T*, int64_t, T*, int64_t), cleave_hip_mr x, cleave_hip_mr out, const char* fn) {
    View X, O;
    CH_TRY(flat_view(x, sizeof(T), fn, "x", nullptr, &X));
    CH_TRY(flat_view(out, sizeof(T), fn, "out", &X, &O));
    return f(reinterpret_cast<const T*>(X.data), X.count, reinterpret_cast<T*>(O.data), O.count);
}

template <class T>
int32_t map2_mr(int32_t (*f)(const T*, int64_t, const T*, int64_t, T*, int64_t), cleave_hip_mr a, cleave_hip_mr b,
                cleave_hip_mr out, const char* fn) {
    View A, B, O;
    CH_TRY(flat_view(a, sizeof(T), fn, "a", nullptr, &A));
    CH_TRY(flat_view(b, sizeof(T), fn, "b", &A, &B));
    CH_TRY(flat_view(out, sizeof(T), fn, "out", &A, &O));
    return f(reinterpret_cast<const T*>(A.data), A.count, reinterpret_cast<const T*>(B.data), B.count,
             reinterpret_cast<T*>(O.data), O.count);
}

// Sizes of a view as the int32 shape array the pointer forms take.
int32_t shape_i32(const View& v, const char* fn, int32_t* out) {
    for (int64_t d = 0; d < v.rank; ++d) CH_TRY(narrow(v.sizes[d], fn, "extent", &out[d]));
    return CLEAVE_HIP_OK;
}

// A broadcasting map: each operand row-major contiguous with its own sizes;
// out shaped as their broadcast (numpy's rule, checked by the pointer form;
// out's own sizes checked here).
template <class T>
int32_t bcast_mr(int32_t (*f)(const T*, int64_t, const int32_t*, int32_t, const T*, int64_t, const int32_t*, int32_t,
                              T*, int64_t),
                 cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out, const char* fn) {
    View A, B, O;
    CH_TRY(flat_view(a, sizeof(T), fn, "a", nullptr, &A));
    CH_TRY(flat_view(b, sizeof(T), fn, "b", nullptr, &B));
    CH_TRY(flat_view(out, sizeof(T), fn, "out", nullptr, &O));
    int32_t as[kMaxRank], bs[kMaxRank];
    CH_TRY(shape_i32(A, fn, as));
    CH_TRY(shape_i32(B, fn, bs));
    const int64_t R = A.rank > B.rank ? A.rank : B.rank;
    bool fits = O.rank == R;
    for (int64_t i = 0; fits && i < R; ++i) {
        const int64_t ja = i - (R - A.rank), jb = i - (R - B.rank);
        const int64_t da = ja < 0 ? 1 : A.sizes[ja], db = jb < 0 ? 1 : B.sizes[jb];
        if (da != db && da != 1 && db != 1) break;  // the pointer form reports it
        fits = O.sizes[i] == (da == 1 ? db : da);
    }
    CH_REQUIRE(fits, "%s: out's sizes are not the broadcast of a's and b's", fn);
    return f(reinterpret_cast<const T*>(A.data), A.count, as, (int32_t)A.rank, reinterpret_cast<const T*>(B.data),
             B.count, bs, (int32_t)B.rank, reinterpret_cast<T*>(O.data), O.count);
}

template <class T>
int32_t sum_to_shape_mr(int32_t (*f)(const T*, int64_t, const int32_t*, int32_t, T*, int64_t, const int32_t*, int32_t),
                        cleave_hip_mr g, cleave_hip_mr out, const char* fn) {
    View G, O;
    CH_TRY(flat_view(g, sizeof(T), fn, "g", nullptr, &G));
    CH_TRY(flat_view(out, sizeof(T), fn, "out", nullptr, &O));
    int32_t gs[kMaxRank], os[kMaxRank];
    CH_TRY(shape_i32(G, fn, gs));
    CH_TRY(shape_i32(O, fn, os));
    return f(reinterpret_cast<const T*>(G.data), G.count, gs, (int32_t)G.rank, reinterpret_cast<T*>(O.data), O.count,
             os, (int32_t)O.rank);
}

// A host-returning reduction over a contiguous operand; `bad` after an error.
template <class R, class T>
R reduce_mr(R (*f)(const T*, int64_t), cleave_hip_mr x, const char* fn, R bad) {
    View X;
    if (flat_view(x, sizeof(T), fn, "x", nullptr, &X) != CLEAVE_HIP_OK) return bad;
    return f(reinterpret_cast<const T*>(X.data), X.count);
}

// idx: host memref<K x i32>, K = rank of the tensor; copied to int32 arrays of dims/idx.
int32_t index_args(const View& t, cleave_hip_mr idx, const char* fn, int32_t* dims, int32_t* ix) {
    View I;
    CH_TRY(read_view(idx, 4, fn, "idx", &I));
    CH_REQUIRE(I.rank == 1 && I.sizes[0] == t.rank, "%s: idx must be memref<%lld x i32>", fn, (long long)t.rank);
    CH_REQUIRE(t.rank >= 1, "%s: a rank-0 tensor has no index", fn);
    const int32_t* ip = reinterpret_cast<const int32_t*>(I.data);
    for (int64_t d = 0; d < t.rank; ++d) {
        CH_TRY(narrow(t.sizes[d], fn, "extent", &dims[d]));
        ix[d] = ip[d * I.strides[0]];
    }
    return CLEAVE_HIP_OK;
}

}  // namespace

extern "C" {

int32_t _mlir_ciface_cleave_hip_matmul_f32(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr c) {
    return matmul_mr<float, float>({cleave_hip_matmul_f32, cleave_hip_matmul_batched_f32}, a, b, c,
                                   "_mlir_ciface_cleave_hip_matmul_f32");
}
int32_t _mlir_ciface_cleave_hip_matmul_bf16(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr c) {
    return matmul_mr<uint16_t, float>({cleave_hip_matmul_bf16, cleave_hip_matmul_batched_bf16}, a, b, c,
                                      "_mlir_ciface_cleave_hip_matmul_bf16");
}
int32_t _mlir_ciface_cleave_hip_matmul_f64(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr c) {
    return matmul_mr<double, double>({cleave_hip_matmul_f64, cleave_hip_matmul_batched_f64}, a, b, c,
                                     "_mlir_ciface_cleave_hip_matmul_f64");
}

#define CH_MAP2(name, T, sfx)                                                                                 \
    int32_t _mlir_ciface_cleave_hip_##name##_##sfx(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out) {   \
        return map2_mr<T>(cleave_hip_##name##_##sfx, a, b, out, "_mlir_ciface_cleave_hip_" #name "_" #sfx); \
    }
#define CH_MAP1(name, T, sfx)                                                                                 \
    int32_t _mlir_ciface_cleave_hip_##name##_##sfx(cleave_hip_mr x, cleave_hip_mr out) {                    \
        return map1_mr<T>(cleave_hip_##name##_##sfx, x, out, "_mlir_ciface_cleave_hip_" #name "_" #sfx);    \
    }
#define CH_MAPS(T, sfx)            \
    CH_MAP2(add, T, sfx)           \
    CH_MAP2(sub, T, sfx)           \
    CH_MAP2(mul, T, sfx)           \
    CH_MAP2(div, T, sfx)           \
    CH_MAP1(neg, T, sfx)           \
    CH_MAP1(relu, T, sfx)          \
    CH_MAP1(sigmoid, T, sfx)       \
    CH_MAP1(tanh, T, sfx)          \
    CH_MAP2(sigmoid_bwd, T, sfx)   \
    CH_MAP2(tanh_bwd, T, sfx)      \
    CH_MAP2(relu_bwd, T, sfx)
CH_MAPS(float, f32)
CH_MAPS(double, f64)

#define CH_BCAST_MR(name, T, sfx)                                                                               \
    int32_t _mlir_ciface_cleave_hip_##name##_bcast_##sfx(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr out) { \
        return bcast_mr<T>(cleave_hip_##name##_bcast_##sfx, a, b, out,                                           \
                           "_mlir_ciface_cleave_hip_" #name "_bcast_" #sfx);                                     \
    }
CH_BCAST_MR(add, float, f32)
CH_BCAST_MR(sub, float, f32)
CH_BCAST_MR(mul, float, f32)
CH_BCAST_MR(div, float, f32)
CH_BCAST_MR(add, double, f64)
CH_BCAST_MR(sub, double, f64)
CH_BCAST_MR(mul, double, f64)
CH_BCAST_MR(div, double, f64)
#undef CH_BCAST_MR

int32_t _mlir_ciface_cleave_hip_sum_to_shape_f32(cleave_hip_mr g, cleave_hip_mr out) {
    return sum_to_shape_mr<float>(cleave_hip_sum_to_shape_f32, g, out, "_mlir_ciface_cleave_hip_sum_to_shape_f32");
}
int32_t _mlir_ciface_cleave_hip_sum_to_shape_f64(cleave_hip_mr g, cleave_hip_mr out) {
    return sum_to_shape_mr<double>(cleave_hip_sum_to_shape_f64, g, out, "_mlir_ciface_cleave_hip_sum_to_shape_f64");
}

int32_t _mlir_ciface_cleave_hip_zero_f32(cleave_hip_mr out) {
    const char* fn = "_mlir_ciface_cleave_hip_zero_f32";
    View O;
    CH_TRY(flat_view(out, 4, fn, "out", nullptr, &O));
    return cleave_hip_zero_f32(reinterpret_cast<float*>(O.data), O.count);
}

int32_t _mlir_ciface_cleave_hip_div_bwd_f32(cleave_hip_mr a, cleave_hip_mr b, cleave_hip_mr g, cleave_hip_mr da,
                                           cleave_hip_mr db) {
    const char* fn = "_mlir_ciface_cleave_hip_div_bwd_f32";
    View A, B, G, DA, DB;
    CH_TRY(flat_view(a, 4, fn, "a", nullptr, &A));
    CH_TRY(flat_view(b, 4, fn, "b", &A, &B));
    CH_TRY(flat_view(g, 4, fn, "g", &A, &G));
    CH_TRY(flat_view(da, 4, fn, "da", &A, &DA));
    CH_TRY(flat_view(db, 4, fn, "db", &A, &DB));
    return cleave_hip_div_bwd_f32(reinterpret_cast<const float*>(A.data), A.count,
                                  reinterpret_cast<const float*>(B.data), B.count,
                                  reinterpret_cast<const float*>(G.data), G.count, reinterpret_cast<float*>(DA.data),
                                  DA.count, reinterpret_cast<float*>(DB.data), DB.count);
}

int32_t _mlir_ciface_cleave_hip_sgd_update_f32(cleave_hip_mr w, cleave_hip_mr g, float lr) {
    const char* fn = "_mlir_ciface_cleave_hip_sgd_update_f32";
    View W, G;
    CH_TRY(flat_view(w, 4, fn, "w", nullptr, &W));
    CH_TRY(flat_view(g, 4, fn, "g", &W, &G));
    return cleave_hip_sgd_update_f32(reinterpret_cast<float*>(W.data), W.count,
                                     reinterpret_cast<const float*>(G.data), G.count, lr);
}

int32_t _mlir_ciface_cleave_hip_add_row_bias_f32(cleave_hip_mr a, cleave_hip_mr bias, cleave_hip_mr out) {
    const char* fn = "_mlir_ciface_cleave_hip_add_row_bias_f32";
    View A, Bv, O;
    CH_TRY(flat_view(a, 4, fn, "a", nullptr, &A));
    CH_REQUIRE(A.rank == 2, "%s: a must be [rows x cols]", fn);
    CH_TRY(flat_view(bias, 4, fn, "bias", nullptr, &Bv));
    CH_REQUIRE(Bv.count == A.sizes[1] && (Bv.rank == 1 || (Bv.rank == 2 && Bv.sizes[0] == 1)),
               "%s: bias must be [cols] or [1 x cols]", fn);
    CH_TRY(flat_view(out, 4, fn, "out", &A, &O));
    int32_t rows, cols;
    CH_TRY(narrow(A.sizes[0], fn, "rows", &rows));
    CH_TRY(narrow(A.sizes[1], fn, "cols", &cols));
    return cleave_hip_add_row_bias_f32(reinterpret_cast<const float*>(A.data), A.count,
                                       reinterpret_cast<const float*>(Bv.data), Bv.count,
                                       reinterpret_cast<float*>(O.data), O.count, rows, cols);
}

int32_t _mlir_ciface_cleave_hip_sum_rows_f32(cleave_hip_mr g, cleave_hip_mr out) {
    const char* fn = "_mlir_ciface_cleave_hip_sum_rows_f32";
    View G, O;
    CH_TRY(flat_view(g, 4, fn, "g", nullptr, &G));
    CH_REQUIRE(G.rank == 2, "%s: g must be [rows x cols]", fn);
    CH_TRY(flat_view(out, 4, fn, "out", nullptr, &O));
    CH_REQUIRE(O.count == G.sizes[1], "%s: out must hold cols = %lld elements", fn, (long long)G.sizes[1]);
    int32_t rows, cols;
    CH_TRY(narrow(G.sizes[0], fn, "rows", &rows));
    CH_TRY(narrow(G.sizes[1], fn, "cols", &cols));
    return cleave_hip_sum_rows_f32(reinterpret_cast<const float*>(G.data), G.count,
                                   reinterpret_cast<float*>(O.data), O.count, rows, cols);
}

float _mlir_ciface_cleave_hip_sum_f32(cleave_hip_mr x) {
    return reduce_mr<float, float>(cleave_hip_sum_f32, x, "_mlir_ciface_cleave_hip_sum_f32", NAN);
}
float _mlir_ciface_cleave_hip_mean_f32(cleave_hip_mr x) {
    return reduce_mr<float, float>(cleave_hip_mean_f32, x, "_mlir_ciface_cleave_hip_mean_f32", NAN);
}
float _mlir_ciface_cleave_hip_max_of_f32(cleave_hip_mr x) {
    return reduce_mr<float, float>(cleave_hip_max_of_f32, x, "_mlir_ciface_cleave_hip_max_of_f32", NAN);
}
int64_t _mlir_ciface_cleave_hip_argmax_f32(cleave_hip_mr x) {
    return reduce_mr<int64_t, float>(cleave_hip_argmax_f32, x, "_mlir_ciface_cleave_hip_argmax_f32", -1);
}
uint64_t _mlir_ciface_cleave_hip_sum_u32_u64(cleave_hip_mr x) {
    return reduce_mr<uint64_t, uint32_t>(cleave_hip_sum_u32_u64, x, "_mlir_ciface_cleave_hip_sum_u32_u64", 0);
}
double _mlir_ciface_cleave_hip_sum_f64(cleave_hip_mr x) {
    return reduce_mr<double, double>(cleave_hip_sum_f64, x, "_mlir_ciface_cleave_hip_sum_f64", NAN);
}
double _mlir_ciface_cleave_hip_mean_f64(cleave_hip_mr x) {
    return reduce_mr<double, double>(cleave_hip_mean_f64, x, "_mlir_ciface_cleave_hip_mean_f64", NAN);
}
double _mlir_ciface_cleave_hip_max_of_f64(cleave_hip_mr x) {
    return reduce_mr<double, double>(cleave_hip_max_of_f64, x, "_mlir_ciface_cleave_hip_max_of_f64", NAN);
}
int64_t _mlir_ciface_cleave_hip_argmax_f64(cleave_hip_mr x) {
    return reduce_mr<int64_t, double>(cleave_hip_argmax_f64, x, "_mlir_ciface_cleave_hip_argmax_f64", -1);
}

float _mlir_ciface_cleave_hip_index_f32(cleave_hip_mr t, cleave_hip_mr idx) {
    const char* fn = "_mlir_ciface_cleave_hip_index_f32";
    View T;
    int32_t dims[kMaxRank], ix[kMaxRank];
    if (flat_view(t, 4, fn, "t", nullptr, &T) != CLEAVE_HIP_OK) return NAN;
    if (index_args(T, idx, fn, dims, ix) != CLEAVE_HIP_OK) return NAN;
    return cleave_hip_index_f32(reinterpret_cast<const float*>(T.data), T.count, dims, T.rank, ix, T.rank);
}
int32_t _mlir_ciface_cleave_hip_index_bwd_f32(float g, cleave_hip_mr dt, cleave_hip_mr idx) {
    const char* fn = "_mlir_ciface_cleave_hip_index_bwd_f32";
    View T;
    int32_t dims[kMaxRank], ix[kMaxRank];
    CH_TRY(flat_view(dt, 4, fn, "dt", nullptr, &T));
    CH_TRY(index_args(T, idx, fn, dims, ix));
    return cleave_hip_index_bwd_f32(g, reinterpret_cast<float*>(T.data), T.count, dims, T.rank, ix, T.rank);
}
double _mlir_ciface_cleave_hip_index_f64(cleave_hip_mr t, cleave_hip_mr idx) {
    const char* fn = "_mlir_ciface_cleave_hip_index_f64";
    View T;
    int32_t dims[kMaxRank], ix[kMaxRank];
    if (flat_view(t, 8, fn, "t", nullptr, &T) != CLEAVE_HIP_OK) return NAN;
    if (index_args(T, idx, fn, dims, ix) != CLEAVE_HIP_OK) return NAN;
    return cleave_hip_index_f64(reinterpret_cast<const double*>(T.data), T.count, dims, T.rank, ix, T.rank);
}
int32_t _mlir_ciface_cleave_hip_index_bwd_f64(double g, cleave_hip_mr dt, cleave_hip_mr idx) {
    const char* fn = "_mlir_ciface_cleave_hip_index_bwd_f64";
    View T;
    int32_t dims[kMaxRank], ix[kMaxRank];
    CH_TRY(flat_view(dt, 8, fn, "dt", nullptr, &T));
    CH_TRY(index_args(T, idx, fn, dims, ix));
    return cleave_hip_index_bwd_f64(g, reinterpret_cast<double*>(T.data), T.count, dims, T.rank, ix, T.rank);
}

int32_t _mlir_ciface_cleave_hip_mandelbrot_u32(cleave_hip_mr out, float x0, float y0, float dx, float dy,
                                              int32_t max_iter) {
    const char* fn = "_mlir_ciface_cleave_hip_mandelbrot_u32";
    View O;
    CH_TRY(flat_view(out, 4, fn, "out", nullptr, &O));
    CH_REQUIRE(O.rank == 2, "%s: out must be memref<height x width>", fn);
    int32_t h, w;
    CH_TRY(narrow(O.sizes[0], fn, "height", &h));
    CH_TRY(narrow(O.sizes[1], fn, "width", &w));
    return cleave_hip_mandelbrot_u32(reinterpret_cast<uint32_t*>(O.data), O.count, w, h, x0, y0, dx, dy, max_iter);
}

int32_t _mlir_ciface_cleave_hip_mlp_step_f32(cleave_hip_mr x, cleave_hip_mr y, cleave_hip_mr w1, cleave_hip_mr w2,
                                            cleave_hip_mr dw1, cleave_hip_mr dw2, cleave_hip_mr loss, float lr) {
    const char* fn = "_mlir_ciface_cleave_hip_mlp_step_f32";
    View X, Y, W1, W2, DW1, DW2, L;
    CH_TRY(flat_view(x, 4, fn, "x", nullptr, &X));
    CH_TRY(flat_view(y, 4, fn, "y", nullptr, &Y));
    CH_TRY(flat_view(w1, 4, fn, "w1", nullptr, &W1));
    CH_TRY(flat_view(w2, 4, fn, "w2", nullptr, &W2));
    CH_REQUIRE(X.rank == 2 && W1.rank == 2 && Y.count == X.sizes[0] && W1.sizes[0] == X.sizes[1] &&
                   W2.count == W1.sizes[1],
               "%s: expected x [B x D], y [B], w1 [D x Hd], w2 [Hd]", fn);
    float* dw1p = nullptr;
    float* dw2p = nullptr;
    float* lossp = nullptr;
    int64_t dw1n = 0, dw2n = 0;
    if (dw1) {
        CH_TRY(flat_view(dw1, 4, fn, "dw1", &W1, &DW1));
        dw1p = reinterpret_cast<float*>(DW1.data);
        dw1n = DW1.count;
    }
    if (dw2) {
        CH_TRY(flat_view(dw2, 4, fn, "dw2", nullptr, &DW2));
        CH_REQUIRE(DW2.count == W2.count, "%s: dw2 must have %lld elements", fn, (long long)W2.count);
        dw2p = reinterpret_cast<float*>(DW2.data);
        dw2n = DW2.count;
    }
    if (loss) {
        CH_TRY(flat_view(loss, 4, fn, "loss", nullptr, &L));
        CH_REQUIRE(L.count == 1, "%s: loss must hold one element", fn);
        lossp = reinterpret_cast<float*>(L.data);
    }
    int32_t B, D, Hd;
    CH_TRY(narrow(X.sizes[0], fn, "B", &B));
    CH_TRY(narrow(X.sizes[1], fn, "D", &D));
    CH_TRY(narrow(W1.sizes[1], fn, "Hd", &Hd));
    return cleave_hip_mlp_step_f32(reinterpret_cast<const float*>(X.data), X.count,
                                   reinterpret_cast<const float*>(Y.data), Y.count, reinterpret_cast<float*>(W1.data),
                                   W1.count, reinterpret_cast<float*>(W2.data), W2.count, dw1p, dw1n, dw2p, dw2n,
                                   lossp, B, D, Hd, lr);
}

}  // extern "C"
