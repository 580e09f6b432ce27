// elementwise.hip -- same-shape f32 and f64 maps: Ring<Tensor> (stdlib/linalg/tensor.cleave:66-80),
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

// Element math in the operand's own precision: f32 calls expf/tanhf, f64
// calls exp/tanh (math.exp / math.tanh on Tensor<f64>, num.cleave:218-228).
__device__ __forceinline__ float exp_t(float x) { return expf(x); }
__device__ __forceinline__ double exp_t(double x) { return exp(x); }
__device__ __forceinline__ float tanh_t(float x) { return tanhf(x); }
__device__ __forceinline__ double tanh_t(double x) { return tanh(x); }

struct AddOp { template <class T> __device__ T operator()(T a, T b) const { return a + b; } };
struct SubOp { template <class T> __device__ T operator()(T a, T b) const { return a - b; } };
struct MulOp { template <class T> __device__ T operator()(T a, T b) const { return a * b; } };
struct DivOp { template <class T> __device__ T operator()(T a, T b) const { return a / b; } };
struct NegOp { template <class T> __device__ T operator()(T a) const { return -a; } };
// arith.maximumf(x, 0): IEEE 754-2019 maximum; NaN propagates, max(-0,+0)=+0.
struct ReluOp {
    template <class T>
    __device__ T operator()(T x) const { return x > T(0) ? x : (x != x ? x + T(0) : T(0)); }
};
// negf, math.exp, addf(1,.), divf(1,.) -- stdlib/nn/nn.cleave:88-92.
struct SigmoidOp {
    template <class T>
    __device__ T operator()(T x) const { return T(1) / (T(1) + exp_t(-x)); }
};
struct TanhOp { template <class T> __device__ T operator()(T x) const { return tanh_t(x); } };
struct SigmoidBwdOp {  // g * s * (1 - s)
    template <class T>
    __device__ T operator()(T s, T g) const { return g * s * (T(1) - s); }
};
struct TanhBwdOp {  // g * (1 - t*t)
    template <class T>
    __device__ T operator()(T t, T g) const { return g * (T(1) - t * t); }
};
struct ReluBwdOp {  // x > 0 ? g : 0
    template <class T>
    __device__ T operator()(T x, T g) const { return x > T(0) ? g : T(0); }
};

constexpr int kThreads = 256;

// One 16-byte vector per lane: 4 floats or 2 doubles.
template <class T>
struct Vec16 {
    static constexpr int kN = 16 / sizeof(T);
    typedef T type __attribute__((ext_vector_type(kN)));
};

// One 16-byte vector per thread over a grid that covers the whole array (a
// grid-stride loop only past 2^31 blocks), with non-temporal loads and stores:
// streamed data is not kept in L2, which lifts a read+write stream from ~5.5
// to ~6.4 TB/s on MI355X.
unsigned grid_for(int64_t nvec) {
    int64_t want = (nvec + kThreads - 1) / kThreads;
    if (want > 0x7FFFFFFF) want = 0x7FFFFFFF;
    return (unsigned)(want < 1 ? 1 : want);
}

template <class T>
__device__ __forceinline__ typename Vec16<T>::type ldv(const T* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const typename Vec16<T>::type*>(p));
}
template <class T>
__device__ __forceinline__ void stv(T* p, typename Vec16<T>::type v) {
    __builtin_nontemporal_store(v, reinterpret_cast<typename Vec16<T>::type*>(p));
}

template <class Op, class T>
__global__ __launch_bounds__(kThreads) void map1_kernel(const T* __restrict__ a, T* __restrict__ out, int64_t n) {
    constexpr int V = Vec16<T>::kN;
    Op op;
    const int64_t nv = n / V;
    const int64_t step = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < nv; i += step) {
        const typename Vec16<T>::type x = ldv(a + V * i);
        typename Vec16<T>::type y;
#pragma unroll
        for (int e = 0; e < V; ++e) y[e] = op(x[e]);
        stv(out + V * i, y);
    }
    if (blockIdx.x == 0 && threadIdx.x < (n % V)) {
        int64_t i = nv * V + threadIdx.x;
        out[i] = op(a[i]);
    }
}

template <class Op, class T>
__global__ __launch_bounds__(kThreads) void map2_kernel(const T* __restrict__ a, const T* __restrict__ b,
                                                        T* __restrict__ out, int64_t n) {
    constexpr int V = Vec16<T>::kN;
    Op op;
    const int64_t nv = n / V;
    const int64_t step = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < nv; i += step) {
        const typename Vec16<T>::type x = ldv(a + V * i), y = ldv(b + V * i);
        typename Vec16<T>::type z;
#pragma unroll
        for (int e = 0; e < V; ++e) z[e] = op(x[e], y[e]);
        stv(out + V * i, z);
    }
    if (blockIdx.x == 0 && threadIdx.x < (n % V)) {
        int64_t i = nv * V + threadIdx.x;
        out[i] = op(a[i], b[i]);
    }
}

// Scalar fallback for operands that are not 16-byte aligned.
template <class Op, class T>
__global__ void map1_scalar_kernel(const T* a, T* out, int64_t n) {
    Op op;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = op(a[i]);
}
template <class Op, class T>
__global__ void map2_scalar_kernel(const T* a, const T* b, T* out, int64_t n) {
    Op op;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = op(a[i], b[i]);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <class Op, class T>
int32_t run1(const char* name, const T* a, int64_t alen, T* out, int64_t outlen) {
    constexpr int V = Vec16<T>::kN;
    CH_REQUIRE(alen >= 0 && alen == outlen, "%s: input length %lld != output length %lld", name,
               (long long)alen, (long long)outlen);
    if (alen == 0) return CLEAVE_HIP_OK;
    CH_REQUIRE(a && out, "%s: null buffer", name);
    CH_INIT_OR_RETURN();
    CH_DEVICE(name, a, alen * sizeof(T));
    CH_DEVICE(name, out, outlen * sizeof(T));
    if (aligned16(a) && aligned16(out))
        map1_kernel<Op, T><<<grid_for(alen / V), kThreads, 0, ch::stream()>>>(a, out, alen);
    else
        map1_scalar_kernel<Op, T><<<grid_for(alen / V + 1), kThreads, 0, ch::stream()>>>(a, out, alen);
    CH_LAUNCHED(name);
    return CLEAVE_HIP_OK;
}

template <class Op, class T>
int32_t run2(const char* name, const T* a, int64_t alen, const T* b, int64_t blen, T* out, int64_t outlen) {
    constexpr int V = Vec16<T>::kN;
    CH_REQUIRE(alen >= 0 && alen == blen && alen == outlen,
               "%s: operand lengths differ (%lld, %lld, out %lld); no broadcasting", name,
               (long long)alen, (long long)blen, (long long)outlen);
    if (alen == 0) return CLEAVE_HIP_OK;
    CH_REQUIRE(a && b && out, "%s: null buffer", name);
    CH_INIT_OR_RETURN();
    CH_DEVICE(name, a, alen * sizeof(T));
    CH_DEVICE(name, b, blen * sizeof(T));
    CH_DEVICE(name, out, outlen * sizeof(T));
    if (aligned16(a) && aligned16(b) && aligned16(out))
        map2_kernel<Op, T><<<grid_for(alen / V), kThreads, 0, ch::stream()>>>(a, b, out, alen);
    else
        map2_scalar_kernel<Op, T><<<grid_for(alen / V + 1), kThreads, 0, ch::stream()>>>(a, b, out, alen);
    CH_LAUNCHED(name);
    return CLEAVE_HIP_OK;
}

template <class T>
__global__ void zero_kernel(T* out, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = T(0);
}

template <class T>
__global__ void div_bwd_kernel(const T* a, const T* b, const T* g, T* da, T* db, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        T ai = a[i], bi = b[i], gi = g[i];
        da[i] = gi / bi;
        db[i] = -(gi * ai) / (bi * bi);
    }
}

template <class T>
__global__ void sgd_kernel(T* w, const T* g, T lr, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        w[i] = w[i] - lr * g[i];
}

template <class T>
int32_t run_zero(const char* fn, T* out, int64_t outlen) {
    CH_REQUIRE(outlen >= 0, "%s: negative length", fn);
    if (outlen == 0) return CLEAVE_HIP_OK;
    CH_REQUIRE(out != nullptr, "%s: null buffer", fn);
    CH_INIT_OR_RETURN();
    CH_DEVICE(fn, out, outlen * sizeof(T));
    // A fill kernel rather than hipMemsetAsync, so the call can be captured in a graph.
    zero_kernel<T><<<grid_for(outlen / 4 + 1), kThreads, 0, ch::stream()>>>(out, outlen);
    CH_LAUNCHED(fn);
    return CLEAVE_HIP_OK;
}

template <class T>
int32_t run_div_bwd(const char* fn, const T* a, int64_t alen, const T* b, int64_t blen, const T* g, int64_t glen,
                    T* da, int64_t dalen, T* db, int64_t dblen) {
    CH_REQUIRE(alen >= 0 && alen == blen && alen == glen && alen == dalen && alen == dblen,
               "%s: operand lengths differ", fn);
    if (alen == 0) return CLEAVE_HIP_OK;
    CH_REQUIRE(a && b && g && da && db, "%s: null buffer", fn);
    CH_INIT_OR_RETURN();
    CH_DEVICE(fn, a, alen * sizeof(T));
    CH_DEVICE(fn, b, blen * sizeof(T));
    CH_DEVICE(fn, g, glen * sizeof(T));
    CH_DEVICE(fn, da, dalen * sizeof(T));
    CH_DEVICE(fn, db, dblen * sizeof(T));
    div_bwd_kernel<T><<<grid_for(alen / 4 + 1), kThreads, 0, ch::stream()>>>(a, b, g, da, db, alen);
    CH_LAUNCHED(fn);
    return CLEAVE_HIP_OK;
}

template <class T>
int32_t run_sgd(const char* fn, T* w, int64_t wlen, const T* g, int64_t glen, T lr) {
    CH_REQUIRE(wlen >= 0 && wlen == glen, "%s: wlen %lld != glen %lld", fn, (long long)wlen, (long long)glen);
    if (wlen == 0) return CLEAVE_HIP_OK;
    CH_REQUIRE(w && g, "%s: null buffer", fn);
    CH_INIT_OR_RETURN();
    CH_DEVICE(fn, w, wlen * sizeof(T));
    CH_DEVICE(fn, g, glen * sizeof(T));
    sgd_kernel<T><<<grid_for(wlen / 4 + 1), kThreads, 0, ch::stream()>>>(w, g, lr, wlen);
    CH_LAUNCHED(fn);
    return CLEAVE_HIP_OK;
}

}  // namespace

extern "C" {

#define CH_MAP2_ENTRY(op, Op, T, sfx)                                                                    \
    int32_t cleave_hip_##op##_##sfx(const T* a, int64_t alen, const T* b, int64_t blen, T* out,         \
                                    int64_t outlen) {                                                    \
        return run2<Op, T>("cleave_hip_" #op "_" #sfx, a, alen, b, blen, out, outlen);                 \
    }
#define CH_MAP1_ENTRY(op, Op, T, sfx)                                                                    \
    int32_t cleave_hip_##op##_##sfx(const T* a, int64_t alen, T* out, int64_t outlen) {                \
        return run1<Op, T>("cleave_hip_" #op "_" #sfx, a, alen, out, outlen);                          \
    }
#define CH_MAP_ENTRIES(T, sfx)                                                                           \
    CH_MAP2_ENTRY(add, AddOp, T, sfx)                                                                    \
    CH_MAP2_ENTRY(sub, SubOp, T, sfx)                                                                    \
    CH_MAP2_ENTRY(mul, MulOp, T, sfx)                                                                    \
    CH_MAP2_ENTRY(div, DivOp, T, sfx)                                                                    \
    CH_MAP1_ENTRY(neg, NegOp, T, sfx)                                                                    \
    CH_MAP1_ENTRY(relu, ReluOp, T, sfx)                                                                  \
    CH_MAP1_ENTRY(sigmoid, SigmoidOp, T, sfx)                                                            \
    CH_MAP1_ENTRY(tanh, TanhOp, T, sfx)                                                                  \
    CH_MAP2_ENTRY(sigmoid_bwd, SigmoidBwdOp, T, sfx)                                                     \
    CH_MAP2_ENTRY(tanh_bwd, TanhBwdOp, T, sfx)                                                           \
    CH_MAP2_ENTRY(relu_bwd, ReluBwdOp, T, sfx)                                                           \
    int32_t cleave_hip_zero_##sfx(T* out, int64_t outlen) {                                              \
        return run_zero<T>("cleave_hip_zero_" #sfx, out, outlen);                                       \
    }                                                                                                    \
    int32_t cleave_hip_div_bwd_##sfx(const T* a, int64_t alen, const T* b, int64_t blen, const T* g,    \
                                     int64_t glen, T* da, int64_t dalen, T* db, int64_t dblen) {        \
        return run_div_bwd<T>("cleave_hip_div_bwd_" #sfx, a, alen, b, blen, g, glen, da, dalen, db, dblen); \
    }                                                                                                    \
    int32_t cleave_hip_sgd_update_##sfx(T* w, int64_t wlen, const T* g, int64_t glen, T lr) {          \
        return run_sgd<T>("cleave_hip_sgd_update_" #sfx, w, wlen, g, glen, lr);                         \
    }

CH_MAP_ENTRIES(float, f32)
CH_MAP_ENTRIES(double, f64)

}  // extern "C"
