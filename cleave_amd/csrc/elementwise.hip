// elementwise.hip -- same-shape f32 maps: Ring<Tensor> (stdlib/linalg/tensor.cleave:66-80),
// Activation<Tensor> (stdlib/nn/nn.cleave:82-95) and the backward forms of the
// reference's derivative rules (stdlib/num/num.cleave:123-136, :222-223).
//
// HBM-bound: each thread moves one 16-byte vector per operand with
// non-temporal loads/stores, over a grid that covers the array.
// The library is compiled with -ffp-contract=off, so every op below rounds
// exactly where the reference's scalar loop does (add/sub/mul/div/neg/relu
// are bit-exact; exp/tanh come from the device math library).
#include "common.hpp"

namespace {

struct AddOp { __device__ float operator()(float a, float b) const { return a + b; } };
struct SubOp { __device__ float operator()(float a, float b) const { return a - b; } };
struct MulOp { __device__ float operator()(float a, float b) const { return a * b; } };
struct DivOp { __device__ float operator()(float a, float b) const { return a / b; } };
struct NegOp { __device__ float operator()(float a) const { return -a; } };
// arith.maximumf(x, 0): IEEE 754-2019 maximum; NaN propagates, max(-0,+0)=+0.
struct ReluOp {
    __device__ float operator()(float x) const { return x > 0.0f ? x : (x != x ? x + 0.0f : 0.0f); }
};
// negf, math.exp, addf(1,.), divf(1,.) -- stdlib/nn/nn.cleave:88-92.
struct SigmoidOp {
    __device__ float operator()(float x) const { return 1.0f / (1.0f + expf(-x)); }
};
struct TanhOp { __device__ float operator()(float x) const { return tanhf(x); } };
struct SigmoidBwdOp {  // g * s * (1 - s)
    __device__ float operator()(float s, float g) const { return g * s * (1.0f - s); }
};
struct TanhBwdOp {  // g * (1 - t*t)
    __device__ float operator()(float t, float g) const { return g * (1.0f - t * t); }
};
struct ReluBwdOp {  // x > 0 ? g : 0
    __device__ float operator()(float x, float g) const { return x > 0.0f ? g : 0.0f; }
};

constexpr int kThreads = 256;

typedef float f4 __attribute__((ext_vector_type(4)));

// One 16-byte vector per thread over a grid that covers the whole array (a
// grid-stride loop only past 2^31 blocks), with non-temporal loads and stores:
// streamed data is not kept in L2, which lifts a read+write stream from ~5.5
// to ~6.4 TB/s on MI355X.
unsigned grid_for(int64_t nvec) {
    int64_t want = (nvec + kThreads - 1) / kThreads;
    if (want > 0x7FFFFFFF) want = 0x7FFFFFFF;
    return (unsigned)(want < 1 ? 1 : want);
}

__device__ __forceinline__ f4 ld4(const float* p) { return __builtin_nontemporal_load(reinterpret_cast<const f4*>(p)); }
__device__ __forceinline__ void st4(float* p, f4 v) { __builtin_nontemporal_store(v, reinterpret_cast<f4*>(p)); }

template <class Op>
__global__ __launch_bounds__(kThreads) void map1_kernel(const float* __restrict__ a,
                                                        float* __restrict__ out, int64_t n) {
    Op op;
    const int64_t nv = n / 4;
    const int64_t step = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < nv; i += step) {
        const f4 x = ld4(a + 4 * i);
        st4(out + 4 * i, f4{op(x[0]), op(x[1]), op(x[2]), op(x[3])});
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
        int64_t i = nv * 4 + threadIdx.x;
        out[i] = op(a[i]);
    }
}

template <class Op>
__global__ __launch_bounds__(kThreads) void map2_kernel(const float* __restrict__ a,
                                                        const float* __restrict__ b,
                                                        float* __restrict__ out, int64_t n) {
    Op op;
    const int64_t nv = n / 4;
    const int64_t step = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < nv; i += step) {
        const f4 x = ld4(a + 4 * i), y = ld4(b + 4 * i);
        st4(out + 4 * i, f4{op(x[0], y[0]), op(x[1], y[1]), op(x[2], y[2]), op(x[3], y[3])});
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
        int64_t i = nv * 4 + threadIdx.x;
        out[i] = op(a[i], b[i]);
    }
}

// Scalar fallback for operands that are not 16-byte aligned.
template <class Op>
__global__ void map1_scalar_kernel(const float* a, float* out, int64_t n) {
    Op op;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = op(a[i]);
}
template <class Op>
__global__ void map2_scalar_kernel(const float* a, const float* b, float* out, int64_t n) {
    Op op;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = op(a[i], b[i]);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <class Op>
int32_t run1(const char* name, const float* a, int64_t alen, float* out, int64_t outlen) {
    CH_REQUIRE(alen >= 0 && alen == outlen, "%s: input length %lld != output length %lld", name,
               (long long)alen, (long long)outlen);
    if (alen == 0) return CLEAVE_HIP_OK;
    CH_REQUIRE(a && out, "%s: null buffer", name);
    CH_INIT_OR_RETURN();
    CH_DEVICE(name, a, alen * 4);
    CH_DEVICE(name, out, outlen * 4);
    if (aligned16(a) && aligned16(out))
        map1_kernel<Op><<<grid_for(alen / 4), kThreads, 0, ch::stream()>>>(a, out, alen);
    else
        map1_scalar_kernel<Op><<<grid_for(alen / 4 + 1), kThreads, 0, ch::stream()>>>(a, out, alen);
    CH_LAUNCHED(name);
    return CLEAVE_HIP_OK;
}

template <class Op>
int32_t run2(const char* name, const float* a, int64_t alen, const float* b, int64_t blen,
             float* out, int64_t outlen) {
    CH_REQUIRE(alen >= 0 && alen == blen && alen == outlen,
               "%s: operand lengths differ (%lld, %lld, out %lld); no broadcasting", name,
               (long long)alen, (long long)blen, (long long)outlen);
    if (alen == 0) return CLEAVE_HIP_OK;
    CH_REQUIRE(a && b && out, "%s: null buffer", name);
    CH_INIT_OR_RETURN();
    CH_DEVICE(name, a, alen * 4);
    CH_DEVICE(name, b, blen * 4);
    CH_DEVICE(name, out, outlen * 4);
    if (aligned16(a) && aligned16(b) && aligned16(out))
        map2_kernel<Op><<<grid_for(alen / 4), kThreads, 0, ch::stream()>>>(a, b, out, alen);
    else
        map2_scalar_kernel<Op><<<grid_for(alen / 4 + 1), kThreads, 0, ch::stream()>>>(a, b, out, alen);
    CH_LAUNCHED(name);
    return CLEAVE_HIP_OK;
}

__global__ void zero_kernel(float* out, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = 0.0f;
}

__global__ void div_bwd_kernel(const float* a, const float* b, const float* g, float* da,
                               float* db, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        float ai = a[i], bi = b[i], gi = g[i];
        da[i] = gi / bi;
        db[i] = -(gi * ai) / (bi * bi);
    }
}

__global__ void sgd_kernel(float* w, const float* g, float lr, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        w[i] = w[i] - lr * g[i];
}

}  // namespace

extern "C" {

int32_t cleave_hip_add_f32(const float* a, int64_t alen, const float* b, int64_t blen, float* out, int64_t outlen) {
    return run2<AddOp>("cleave_hip_add_f32", a, alen, b, blen, out, outlen);
}
int32_t cleave_hip_sub_f32(const float* a, int64_t alen, const float* b, int64_t blen, float* out, int64_t outlen) {
    return run2<SubOp>("cleave_hip_sub_f32", a, alen, b, blen, out, outlen);
}
int32_t cleave_hip_mul_f32(const float* a, int64_t alen, const float* b, int64_t blen, float* out, int64_t outlen) {
    return run2<MulOp>("cleave_hip_mul_f32", a, alen, b, blen, out, outlen);
}
int32_t cleave_hip_div_f32(const float* a, int64_t alen, const float* b, int64_t blen, float* out, int64_t outlen) {
    return run2<DivOp>("cleave_hip_div_f32", a, alen, b, blen, out, outlen);
}
int32_t cleave_hip_neg_f32(const float* a, int64_t alen, float* out, int64_t outlen) {
    return run1<NegOp>("cleave_hip_neg_f32", a, alen, out, outlen);
}
int32_t cleave_hip_relu_f32(const float* x, int64_t xlen, float* out, int64_t outlen) {
    return run1<ReluOp>("cleave_hip_relu_f32", x, xlen, out, outlen);
}
int32_t cleave_hip_sigmoid_f32(const float* x, int64_t xlen, float* out, int64_t outlen) {
    return run1<SigmoidOp>("cleave_hip_sigmoid_f32", x, xlen, out, outlen);
}
int32_t cleave_hip_tanh_f32(const float* x, int64_t xlen, float* out, int64_t outlen) {
    return run1<TanhOp>("cleave_hip_tanh_f32", x, xlen, out, outlen);
}
int32_t cleave_hip_sigmoid_bwd_f32(const float* s, int64_t slen, const float* g, int64_t glen, float* out, int64_t outlen) {
    return run2<SigmoidBwdOp>("cleave_hip_sigmoid_bwd_f32", s, slen, g, glen, out, outlen);
}
int32_t cleave_hip_tanh_bwd_f32(const float* t, int64_t tlen, const float* g, int64_t glen, float* out, int64_t outlen) {
    return run2<TanhBwdOp>("cleave_hip_tanh_bwd_f32", t, tlen, g, glen, out, outlen);
}
int32_t cleave_hip_relu_bwd_f32(const float* x, int64_t xlen, const float* g, int64_t glen, float* out, int64_t outlen) {
    return run2<ReluBwdOp>("cleave_hip_relu_bwd_f32", x, xlen, g, glen, out, outlen);
}

int32_t cleave_hip_zero_f32(float* out, int64_t outlen) {
    CH_REQUIRE(outlen >= 0, "cleave_hip_zero_f32: negative length");
    if (outlen == 0) return CLEAVE_HIP_OK;
    CH_REQUIRE(out != nullptr, "cleave_hip_zero_f32: null buffer");
    CH_INIT_OR_RETURN();
    CH_DEVICE("cleave_hip_zero_f32", out, outlen * 4);
    // A fill kernel rather than hipMemsetAsync, so the call can be captured in a graph.
    zero_kernel<<<grid_for(outlen / 4 + 1), kThreads, 0, ch::stream()>>>(out, outlen);
    CH_LAUNCHED("zero_kernel");
    return CLEAVE_HIP_OK;
}

int32_t cleave_hip_div_bwd_f32(const float* a, int64_t alen, const float* b, int64_t blen,
                               const float* g, int64_t glen, float* da, int64_t dalen, float* db,
                               int64_t dblen) {
    CH_REQUIRE(alen >= 0 && alen == blen && alen == glen && alen == dalen && alen == dblen,
               "cleave_hip_div_bwd_f32: operand lengths differ");
    if (alen == 0) return CLEAVE_HIP_OK;
    CH_REQUIRE(a && b && g && da && db, "cleave_hip_div_bwd_f32: null buffer");
    CH_INIT_OR_RETURN();
    const char* fn = "cleave_hip_div_bwd_f32";
    CH_DEVICE(fn, a, alen * 4);
    CH_DEVICE(fn, b, blen * 4);
    CH_DEVICE(fn, g, glen * 4);
    CH_DEVICE(fn, da, dalen * 4);
    CH_DEVICE(fn, db, dblen * 4);
    div_bwd_kernel<<<grid_for(alen / 4 + 1), kThreads, 0, ch::stream()>>>(a, b, g, da, db, alen);
    CH_LAUNCHED("div_bwd_kernel");
    return CLEAVE_HIP_OK;
}

int32_t cleave_hip_sgd_update_f32(float* w, int64_t wlen, const float* g, int64_t glen, float lr) {
    CH_REQUIRE(wlen >= 0 && wlen == glen, "cleave_hip_sgd_update_f32: wlen %lld != glen %lld",
               (long long)wlen, (long long)glen);
    if (wlen == 0) return CLEAVE_HIP_OK;
    CH_REQUIRE(w && g, "cleave_hip_sgd_update_f32: null buffer");
    CH_INIT_OR_RETURN();
    CH_DEVICE("cleave_hip_sgd_update_f32", w, wlen * 4);
    CH_DEVICE("cleave_hip_sgd_update_f32", g, glen * 4);
    sgd_kernel<<<grid_for(wlen / 4 + 1), kThreads, 0, ch::stream()>>>(w, g, lr, wlen);
    CH_LAUNCHED("sgd_kernel");
    return CLEAVE_HIP_OK;
}

}  // extern "C"
