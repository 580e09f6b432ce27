// index.hip -- Index<Tensor>::index (stdlib/linalg/tensor.cleave:113-133) and
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

__global__ void scatter_add_kernel(float* __restrict__ dt, int64_t off, float g) { dt[off] = dt[off] + g; }

}  // namespace

extern "C" {

float cleave_hip_index_f32(const float* t, int64_t len, const int32_t* dims, int64_t ndims,
                           const int32_t* idx, int64_t nidx) {
    ch::clear_error();
    int64_t off = 0;
    if (!t) {
        ch::fail(CLEAVE_HIP_ERR_ARG, "cleave_hip_index_f32: null tensor");
        return NAN;
    }
    if (flat_offset("cleave_hip_index_f32", len, dims, ndims, idx, nidx, &off) != CLEAVE_HIP_OK) return NAN;
    if (ch::ensure_init() != CLEAVE_HIP_OK) return NAN;
    if (ch::require_device("cleave_hip_index_f32", "t", t, (uint64_t)len * 4) != CLEAVE_HIP_OK) return NAN;
    float v = NAN;
    if (cleave_hip_download(&v, t + off, sizeof(float)) != (int64_t)sizeof(float)) return NAN;
    return v;
}

int32_t cleave_hip_index_bwd_f32(float g, float* dt, int64_t len, const int32_t* dims, int64_t ndims,
                                 const int32_t* idx, int64_t nidx) {
    CH_REQUIRE(dt != nullptr, "cleave_hip_index_bwd_f32: null gradient buffer");
    int64_t off = 0;
    const int32_t st = flat_offset("cleave_hip_index_bwd_f32", len, dims, ndims, idx, nidx, &off);
    if (st != CLEAVE_HIP_OK) return st;
    CH_INIT_OR_RETURN();
    CH_DEVICE("cleave_hip_index_bwd_f32", dt, len * 4);
    scatter_add_kernel<<<1, 1, 0, ch::stream()>>>(dt, off, g);
    CH_LAUNCHED("scatter_add_kernel");
    return CLEAVE_HIP_OK;
}

}  // extern "C"
