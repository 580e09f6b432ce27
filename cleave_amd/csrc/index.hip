// index.hip -- Index<Tensor>::index (stdlib/linalg/tensor.cleave:113-133), f32 and f64, and
// the reverse-mode form of its derivative rule `index(d(c), idx)`.
//
// `idx` and the tensor's `dims` arrive as (pointer, length) pairs of host
// int32 arrays, the form an [i32; K] argument takes across an extern call
// (cleave/src/mlir_lower.rs:1720-1751).  The element offset is the row-major
// flattening of the reference's tensor<d0 x ... x T> (mlir_lower.rs:214-239).
// Every index is checked against its extent on the host before the device is
// touched (tensor.extract out of range is undefined in the reference; here it
// is an argument error).
#include "common.hpp"

namespace {

int32_t flat_offset(const char* fn, int64_t len, const int32_t* dims, int64_t ndims,
                    const int32_t* idx, int64_t nidx, int64_t* off) {
    CH_REQUIRE(ndims >= 1 && ndims == nidx, "%s: %lld indices for a rank-%lld tensor", fn,
               (long long)nidx, (long long)ndims);
    CH_REQUIRE(dims && idx, "%s: null dims or idx array", fn);
    int64_t o = 0, count = 1;
    for (int64_t d = 0; d < ndims; ++d) {
        CH_REQUIRE(dims[d] > 0, "%s: extent %d of dim %lld is not positive", fn, dims[d], (long long)d);
        CH_REQUIRE(idx[d] >= 0 && idx[d] < dims[d], "%s: index %d out of range [0, %d) in dim %lld", fn,
                   idx[d], dims[d], (long long)d);
        o = o * dims[d] + idx[d];
        count *= dims[d];
    }
    CH_REQUIRE(count == len, "%s: dims describe %lld elements, buffer holds %lld", fn, (long long)count,
               (long long)len);
    *off = o;
    return CLEAVE_HIP_OK;
}

template <class T>
__global__ void scatter_add_kernel(T* __restrict__ dt, int64_t off, T g) { dt[off] = dt[off] + g; }

template <class T>
T run_index(const char* fn, const T* t, int64_t len, const int32_t* dims, int64_t ndims, const int32_t* idx,
            int64_t nidx) {
    ch::clear_error();
    int64_t off = 0;
    if (!t) {
        ch::fail(CLEAVE_HIP_ERR_ARG, "%s: null tensor", fn);
        return NAN;
    }
    if (flat_offset(fn, len, dims, ndims, idx, nidx, &off) != CLEAVE_HIP_OK) return NAN;
    if (ch::ensure_init() != CLEAVE_HIP_OK) return NAN;
    if (ch::require_device(fn, "t", t, (uint64_t)len * sizeof(T)) != CLEAVE_HIP_OK) return NAN;
    T v = NAN;
    if (cleave_hip_download(&v, t + off, sizeof(T)) != (int64_t)sizeof(T)) return NAN;
    return v;
}

template <class T>
int32_t run_index_bwd(const char* fn, T g, T* dt, int64_t len, const int32_t* dims, int64_t ndims,
                      const int32_t* idx, int64_t nidx) {
    CH_REQUIRE(dt != nullptr, "%s: null gradient buffer", fn);
    int64_t off = 0;
    const int32_t st = flat_offset(fn, len, dims, ndims, idx, nidx, &off);
    if (st != CLEAVE_HIP_OK) return st;
    CH_INIT_OR_RETURN();
    CH_DEVICE(fn, dt, len * sizeof(T));
    scatter_add_kernel<T><<<1, 1, 0, ch::stream()>>>(dt, off, g);
    CH_LAUNCHED("scatter_add_kernel");
    return CLEAVE_HIP_OK;
}

}  // namespace

extern "C" {

float cleave_hip_index_f32(const float* t, int64_t len, const int32_t* dims, int64_t ndims,
                           const int32_t* idx, int64_t nidx) {
    return run_index<float>("cleave_hip_index_f32", t, len, dims, ndims, idx, nidx);
}

int32_t cleave_hip_index_bwd_f32(float g, float* dt, int64_t len, const int32_t* dims, int64_t ndims,
                                 const int32_t* idx, int64_t nidx) {
    return run_index_bwd<float>("cleave_hip_index_bwd_f32", g, dt, len, dims, ndims, idx, nidx);
}

double cleave_hip_index_f64(const double* t, int64_t len, const int32_t* dims, int64_t ndims,
                            const int32_t* idx, int64_t nidx) {
    return run_index<double>("cleave_hip_index_f64", t, len, dims, ndims, idx, nidx);
}

int32_t cleave_hip_index_bwd_f64(double g, double* dt, int64_t len, const int32_t* dims, int64_t ndims,
                                 const int32_t* idx, int64_t nidx) {
    return run_index_bwd<double>("cleave_hip_index_bwd_f64", g, dt, len, dims, ndims, idx, nidx);
}

}  // extern "C"
