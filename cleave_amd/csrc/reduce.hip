// reduce.hip -- Sum / Mean / Max (stdlib/nn/nn.cleave:111-149), the exact
// u64 sum of u32 escape counts, and the exact i64 sum of i32 arrays (the
// same counts as cleave's i32 type carries them).
//
// Two stages, both deterministic for a given length: stage 1 runs a fixed
// grid (a function of the length and the CU count only); each thread folds
// 16-byte vectors in registers, the wave combines lanes with cross-lane
// shuffles, LDS carries the 4 wave results to one block result.  Stage 2 is
// one block over the block results.
//
// Max semantics: the reference folds acc = v[0]; if v[i] > acc then acc = v[i]
// (cmpf ogt, stdlib/num/num.cleave:303).  A NaN at i > 0 never wins; a NaN at
// v[0] is the answer.  With v[0] not NaN the fold returns the first index of
// the largest non-NaN value, which is associative as (value desc, index asc)
// -- that is what the tree combines (-0 and +0 compare equal, so the earlier
// one is kept, as in the fold).
#include <cfloat>

#include "common.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

// Native clang vectors (register-promoted; HIP's float4/uint4 structs are not
// always) loaded with non-temporal hints: the data is streamed once.
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// Stage-1 grid: enough blocks for 16 per CU (a function of the length and the
// CU count only, so results are reproducible on a given device).
unsigned stage1_blocks(int64_t nvec) {
    int64_t want = (nvec + (int64_t)kThreads * kUnroll - 1) / ((int64_t)kThreads * kUnroll);
    int64_t cap = (int64_t)ch::num_cus() * 16;
    if (want > cap) want = cap;
    return (unsigned)(want < 1 ? 1 : want);
}

// ---- sum f32 / f64 ------------------------------------------------------------
// One 16-byte vector per load: 4 floats or 2 doubles.
template <class T>
struct Vec16 {
    static constexpr int kN = 16 / sizeof(T);
    typedef T type __attribute__((ext_vector_type(kN)));
};

template <class T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

template <class T>
__device__ T block_sum(T v) {
    __shared__ T part[kThreads / 64];
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
    __syncthreads();
    T r = T(0);
    if (threadIdx.x == 0)
        for (int w = 0; w < kThreads / 64; ++w) r += part[w];
    return r;  // valid in thread 0
}

// Each lane keeps one accumulator per vector element and adds them in a
// fixed tree at the end: (a0 + a1) + (a2 + a3) for f32, a0 + a1 for f64.
template <class T>
__global__ __launch_bounds__(kThreads) void sum_stage1(const T* __restrict__ x, int64_t n, T* __restrict__ partial,
                                                       int aligned) {
    constexpr int V = Vec16<T>::kN;
    typedef typename Vec16<T>::type VT;
    T acc[V];
#pragma unroll
    for (int e = 0; e < V; ++e) acc[e] = T(0);
    if (aligned) {
        const int64_t nv = n / V;
        const int64_t step = (int64_t)gridDim.x * kThreads * kUnroll;
        for (int64_t base = (int64_t)blockIdx.x * kThreads * kUnroll + threadIdx.x; base < nv; base += step) {
            VT v[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                int64_t i = base + (int64_t)u * kThreads;
                v[u] = i < nv ? __builtin_nontemporal_load(reinterpret_cast<const VT*>(x) + i) : VT(T(0));
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u)
#pragma unroll
                for (int e = 0; e < V; ++e) acc[e] += v[u][e];
        }
        if (blockIdx.x == 0 && threadIdx.x < (n % V)) acc[0] += x[nv * V + threadIdx.x];
    } else {
        for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
            acc[0] += x[i];
    }
    T lane;
    if constexpr (V == 4) lane = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    else lane = acc[0] + acc[1];
    T r = block_sum(lane);
    if (threadIdx.x == 0) partial[blockIdx.x] = r;
}

// Stage 2 folds thread t's partials t, t + 256, ... in that order.  The
// loads of a run of kStage2Loads go out together before the adds: one memory
// latency per run instead of one per partial (5.2 us -> ~1.5 us for 4096
// partials; the order, and so the result, is unchanged).
constexpr int kStage2Loads = 16;

template <class T>
__global__ __launch_bounds__(kThreads) void sum_stage2(const T* __restrict__ partial, int nparts, T* __restrict__ out) {
    T acc = T(0);
    for (int i0 = threadIdx.x; i0 < nparts; i0 += kThreads * kStage2Loads) {
        T v[kStage2Loads];
#pragma unroll
        for (int u = 0; u < kStage2Loads; ++u) {
            const int i = i0 + u * kThreads;
            v[u] = i < nparts ? partial[i] : T(0);
        }
#pragma unroll
        for (int u = 0; u < kStage2Loads; ++u)
            if (i0 + u * kThreads < nparts) acc += v[u];
    }
    T r = block_sum(acc);
    if (threadIdx.x == 0) *out = r;
}

// ---- max / argmax f32 / f64 -------------------------------------------------
template <class T>
struct Best {
    T v;
    int64_t i;
};
template <class T>
__device__ __forceinline__ void take_better(Best<T>& a, T v, int64_t i) {
    // Comparisons involving NaN are false, so a NaN candidate never wins.
    if (v > a.v || (v == a.v && i < a.i)) {
        a.v = v;
        a.i = i;
    }
}
template <class T>
__device__ __forceinline__ Best<T> wave_best(Best<T> b) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        T v = __shfl_xor(b.v, o);
        int64_t i = __shfl_xor(b.i, o);
        take_better(b, v, i);
    }
    return b;
}
template <class T>
__device__ Best<T> block_best(Best<T> b) {
    __shared__ T pv[kThreads / 64];
    __shared__ int64_t pi[kThreads / 64];
    b = wave_best(b);
    if ((threadIdx.x & 63) == 0) {
        pv[threadIdx.x >> 6] = b.v;
        pi[threadIdx.x >> 6] = b.i;
    }
    __syncthreads();
    Best<T> r{-INFINITY, INT64_MAX};
    if (threadIdx.x == 0)
        for (int w = 0; w < kThreads / 64; ++w) take_better(r, pv[w], pi[w]);
    return r;
}

template <class T>
__global__ __launch_bounds__(kThreads) void max_stage1(const T* __restrict__ x, int64_t n, T* __restrict__ pv,
                                                       int64_t* __restrict__ pi, int aligned) {
    constexpr int V = Vec16<T>::kN;
    typedef typename Vec16<T>::type VT;
    Best<T> b{-INFINITY, INT64_MAX};
    if (aligned) {
        const int64_t nv = n / V;
        const int64_t step = (int64_t)gridDim.x * kThreads * kUnroll;
        for (int64_t base = (int64_t)blockIdx.x * kThreads * kUnroll + threadIdx.x; base < nv; base += step) {
            VT v[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                int64_t i = base + (int64_t)u * kThreads;
                if (i < nv) v[u] = __builtin_nontemporal_load(reinterpret_cast<const VT*>(x) + i);
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                int64_t i = base + (int64_t)u * kThreads;
                if (i < nv) {
#pragma unroll
                    for (int e = 0; e < V; ++e) take_better(b, v[u][e], V * i + e);
                }
            }
        }
        if (blockIdx.x == 0 && threadIdx.x < (n % V)) take_better(b, x[nv * V + threadIdx.x], nv * V + threadIdx.x);
    } else {
        for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
            take_better(b, x[i], i);
    }
    Best<T> r = block_best(b);
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = r.v;
        pi[blockIdx.x] = r.i;
    }
}

template <class T>
__global__ __launch_bounds__(kThreads) void max_stage2(const T* __restrict__ x, const T* __restrict__ pv,
                                                       const int64_t* __restrict__ pi, int nparts,
                                                       T* __restrict__ out_v, int64_t* __restrict__ out_i) {
    Best<T> b{-INFINITY, INT64_MAX};
    for (int i0 = threadIdx.x; i0 < nparts; i0 += kThreads * kStage2Loads) {
        T v[kStage2Loads];
        int64_t ix[kStage2Loads];
#pragma unroll
        for (int u = 0; u < kStage2Loads; ++u) {
            const int i = i0 + u * kThreads;
            v[u] = i < nparts ? pv[i] : T(-INFINITY);
            ix[u] = i < nparts ? pi[i] : INT64_MAX;
        }
#pragma unroll
        for (int u = 0; u < kStage2Loads; ++u)
            if (i0 + u * kThreads < nparts) take_better(b, v[u], ix[u]);
    }
    Best<T> r = block_best(b);
    if (threadIdx.x == 0) {
        T x0 = x[0];
        if (x0 != x0) {  // nothing compares > NaN, so the fold keeps a NaN v[0]
            r.v = x0;
            r.i = 0;
        } else if (r.i == INT64_MAX) {  // every other element is NaN
            r.v = x0;
            r.i = 0;
        }
        if (out_v) *out_v = r.v;
        if (out_i) *out_i = r.i;
    }
}

// ---- u64 sum of u32 -----------------------------------------------------------
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ uint64_t block_sum_u64(uint64_t v) {
    __shared__ uint64_t part[kThreads / 64];
    v = wave_sum_u64(v);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
    __syncthreads();
    uint64_t r = 0;
    if (threadIdx.x == 0)
        for (int w = 0; w < kThreads / 64; ++w) r += part[w];
    return r;
}

// Signed: each element is sign-extended to 64 bits, so the u64 total is the
// two's-complement bits of the exact i64 sum (stage 2 is the same add).
template <bool Signed>
__device__ __forceinline__ uint64_t widen(uint32_t v) {
    return Signed ? (uint64_t)(int64_t)(int32_t)v : (uint64_t)v;
}

template <bool Signed>
__global__ __launch_bounds__(kThreads) void sum_u32_stage1(const uint32_t* __restrict__ x, int64_t n,
                                                           uint64_t* __restrict__ partial,
                                                           int aligned) {
    uint64_t acc = 0;
    if (aligned) {
        const int64_t nv = n / 4;
        const int64_t step = (int64_t)gridDim.x * kThreads * kUnroll;
        for (int64_t base = (int64_t)blockIdx.x * kThreads * kUnroll + threadIdx.x; base < nv; base += step) {
            u4 v[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                int64_t i = base + (int64_t)u * kThreads;
                v[u] = i < nv ? __builtin_nontemporal_load(reinterpret_cast<const u4*>(x) + i) : u4{0, 0, 0, 0};
            }
            // Add in 64 bits (mod 2^64, exact for both forms).
#pragma unroll
            for (int u = 0; u < kUnroll; ++u)
                acc += (widen<Signed>(v[u][0]) + widen<Signed>(v[u][1])) +
                       (widen<Signed>(v[u][2]) + widen<Signed>(v[u][3]));
        }
        if (blockIdx.x == 0 && threadIdx.x < (n & 3)) acc += widen<Signed>(x[nv * 4 + threadIdx.x]);
    } else {
        for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
            acc += widen<Signed>(x[i]);
    }
    uint64_t r = block_sum_u64(acc);
    if (threadIdx.x == 0) partial[blockIdx.x] = r;
}

__global__ __launch_bounds__(kThreads) void sum_u64_stage2(const uint64_t* __restrict__ partial,
                                                           int nparts, uint64_t* __restrict__ out) {
    uint64_t acc = 0;
    for (int i0 = threadIdx.x; i0 < nparts; i0 += kThreads * kStage2Loads) {
        uint64_t v[kStage2Loads];
#pragma unroll
        for (int u = 0; u < kStage2Loads; ++u) {
            const int i = i0 + u * kThreads;
            v[u] = i < nparts ? partial[i] : 0;
        }
#pragma unroll
        for (int u = 0; u < kStage2Loads; ++u) acc += v[u];
    }
    uint64_t r = block_sum_u64(acc);
    if (threadIdx.x == 0) *out = r;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Sum into a device scalar: stage-1 partials in scratch slot 0.
template <class T>
int32_t run_reduce_sum(const char* fn, const T* x, int64_t len, T* out_dev) {
    constexpr int V = Vec16<T>::kN;
    CH_REQUIRE(len >= 1, "%s: length must be >= 1 (sum reads v[0])", fn);
    CH_REQUIRE(x && out_dev, "%s: null buffer", fn);
    CH_INIT_OR_RETURN();
    CH_DEVICE(fn, x, len * sizeof(T));
    CH_DEVICE(fn, out_dev, sizeof(T));
    const int aligned = aligned16(x);
    unsigned blocks = stage1_blocks(aligned ? len / V + 1 : len / kUnroll + 1);
    T* part = (T*)ch::scratch(0, sizeof(T) * blocks);
    if (!part) return CLEAVE_HIP_ERR_OOM;
    sum_stage1<T><<<blocks, kThreads, 0, ch::stream()>>>(x, len, part, aligned);
    CH_LAUNCHED("sum_stage1");
    sum_stage2<T><<<1, kThreads, 0, ch::stream()>>>(part, (int)blocks, out_dev);
    CH_LAUNCHED("sum_stage2");
    return CLEAVE_HIP_OK;
}

// max_of / argmax into device scalars: partial indices then values in slot 1.
template <class T>
int32_t run_reduce_max(const char* fn, const T* x, int64_t len, T* max_dev, int64_t* argmax_dev) {
    constexpr int V = Vec16<T>::kN;
    CH_REQUIRE(len >= 1, "%s: length must be >= 1 (max_of reads v[0])", fn);
    CH_REQUIRE(x && (max_dev || argmax_dev), "%s: null buffer", fn);
    CH_INIT_OR_RETURN();
    CH_DEVICE(fn, x, len * sizeof(T));
    if (max_dev) CH_DEVICE(fn, max_dev, sizeof(T));
    if (argmax_dev) CH_DEVICE(fn, argmax_dev, 8);
    const int aligned = aligned16(x);
    unsigned blocks = stage1_blocks(aligned ? len / V + 1 : len / kUnroll + 1);
    char* base = (char*)ch::scratch(1, (sizeof(T) + sizeof(int64_t)) * blocks + 64);
    if (!base) return CLEAVE_HIP_ERR_OOM;
    int64_t* pi = (int64_t*)base;
    T* pv = (T*)(base + sizeof(int64_t) * blocks);
    max_stage1<T><<<blocks, kThreads, 0, ch::stream()>>>(x, len, pv, pi, aligned);
    CH_LAUNCHED("max_stage1");
    max_stage2<T><<<1, kThreads, 0, ch::stream()>>>(x, pv, pi, (int)blocks, max_dev, argmax_dev);
    CH_LAUNCHED("max_stage2");
    return CLEAVE_HIP_OK;
}

// Host-returning forms: queue the reduction into a library-owned device word,
// then copy it back (synchronising the stream).  `bad` comes back after an
// error (NaN, or -1 for an index).
template <class R, class Queue>
R reduce_to_host(Queue queue, R bad) {
    ch::clear_error();
    if (ch::ensure_init() != CLEAVE_HIP_OK) return bad;
    R* d = (R*)ch::scratch(3, 64);
    if (!d) return bad;
    if (queue(d) != CLEAVE_HIP_OK) return bad;
    R r = bad;
    if (cleave_hip_download(&r, d, sizeof(R)) != (int64_t)sizeof(R)) return bad;
    return r;
}

}  // namespace

extern "C" {

int32_t cleave_hip_reduce_sum_f32(const float* x, int64_t len, float* out_dev) {
    return run_reduce_sum<float>("cleave_hip_reduce_sum_f32", x, len, out_dev);
}

int32_t cleave_hip_reduce_sum_f64(const double* x, int64_t len, double* out_dev) {
    return run_reduce_sum<double>("cleave_hip_reduce_sum_f64", x, len, out_dev);
}

// cleave_hip_reduce_sum_f32 with its stage-1 partials in the library's static
// workspace instead of allocated scratch: the same kernels, grid and result,
// and no hipMalloc/hipFree on any call.  The partials are all written by
// stage 1 before stage 2 reads them, so nothing needs clearing between calls.
int32_t cleave_hip_reduce_sum_f32_noalloc(const float* x, int64_t len, float* out_dev) {
    const char* fn = "cleave_hip_reduce_sum_f32_noalloc";
    CH_REQUIRE(len >= 1, "%s: length must be >= 1 (sum reads v[0])", fn);
    CH_REQUIRE(x && out_dev, "%s: null buffer", fn);
    CH_INIT_OR_RETURN();
    CH_DEVICE(fn, x, len * 4);
    CH_DEVICE(fn, out_dev, 4);
    float* part = ch::noalloc_workspace();
    if (!part) return ch::fail(CLEAVE_HIP_ERR_RUNTIME, "%s: the static workspace has no device address", fn);
    const int aligned = aligned16(x);
    unsigned blocks = stage1_blocks(aligned ? len / 4 + 1 : len / kUnroll + 1);
    CH_REQUIRE(blocks <= (unsigned)ch::kNoAllocFloats,
               "%s: %u partial sums exceed the static workspace of %d floats", fn, blocks, ch::kNoAllocFloats);
    sum_stage1<float><<<blocks, kThreads, 0, ch::stream()>>>(x, len, part, aligned);
    CH_LAUNCHED("sum_stage1");
    sum_stage2<float><<<1, kThreads, 0, ch::stream()>>>(part, (int)blocks, out_dev);
    CH_LAUNCHED("sum_stage2");
    return CLEAVE_HIP_OK;
}

int32_t cleave_hip_reduce_max_f32(const float* x, int64_t len, float* max_dev, int64_t* argmax_dev) {
    return run_reduce_max<float>("cleave_hip_reduce_max_f32", x, len, max_dev, argmax_dev);
}

int32_t cleave_hip_reduce_max_f64(const double* x, int64_t len, double* max_dev, int64_t* argmax_dev) {
    return run_reduce_max<double>("cleave_hip_reduce_max_f64", x, len, max_dev, argmax_dev);
}

int32_t cleave_hip_reduce_sum_u32_u64(const uint32_t* x, int64_t len, uint64_t* out_dev) {
    CH_REQUIRE(len >= 0, "cleave_hip_reduce_sum_u32_u64: negative length");
    CH_REQUIRE(x && out_dev, "cleave_hip_reduce_sum_u32_u64: null buffer");
    CH_INIT_OR_RETURN();
    CH_DEVICE("cleave_hip_reduce_sum_u32_u64", x, len * 4);
    CH_DEVICE("cleave_hip_reduce_sum_u32_u64", out_dev, 8);
    const int aligned = aligned16(x);
    unsigned blocks = stage1_blocks(aligned ? len / 4 + 1 : len / kUnroll + 1);
    uint64_t* part = (uint64_t*)ch::scratch(2, sizeof(uint64_t) * blocks);
    if (!part) return CLEAVE_HIP_ERR_OOM;
    sum_u32_stage1<false><<<blocks, kThreads, 0, ch::stream()>>>(x, len, part, aligned);
    CH_LAUNCHED("sum_u32_stage1");
    sum_u64_stage2<<<1, kThreads, 0, ch::stream()>>>(part, (int)blocks, out_dev);
    CH_LAUNCHED("sum_u64_stage2");
    return CLEAVE_HIP_OK;
}

int32_t cleave_hip_reduce_sum_i32_i64(const int32_t* x, int64_t len, int64_t* out_dev) {
    const char* fn = "cleave_hip_reduce_sum_i32_i64";
    CH_REQUIRE(len >= 0, "%s: negative length", fn);
    CH_REQUIRE(x && out_dev, "%s: null buffer", fn);
    CH_INIT_OR_RETURN();
    CH_DEVICE(fn, x, len * 4);
    CH_DEVICE(fn, out_dev, 8);
    const int aligned = aligned16(x);
    unsigned blocks = stage1_blocks(aligned ? len / 4 + 1 : len / kUnroll + 1);
    uint64_t* part = (uint64_t*)ch::scratch(2, sizeof(uint64_t) * blocks);
    if (!part) return CLEAVE_HIP_ERR_OOM;
    sum_u32_stage1<true><<<blocks, kThreads, 0, ch::stream()>>>(reinterpret_cast<const uint32_t*>(x), len, part,
                                                                 aligned);
    CH_LAUNCHED("sum_i32_stage1");
    sum_u64_stage2<<<1, kThreads, 0, ch::stream()>>>(part, (int)blocks, reinterpret_cast<uint64_t*>(out_dev));
    CH_LAUNCHED("sum_u64_stage2");
    return CLEAVE_HIP_OK;
}

// Host-returning forms (synchronise): the reduction lands in a library-owned
// device word that is copied back.
float cleave_hip_sum_f32(const float* x, int64_t len) {
    return reduce_to_host<float>([&](float* d) { return cleave_hip_reduce_sum_f32(x, len, d); }, NAN);
}

float cleave_hip_mean_f32(const float* x, int64_t len) {
    float s = cleave_hip_sum_f32(x, len);
    return s / (float)len;  // sum(v) / sitofp(N), stdlib/nn/nn.cleave:135-138
}

float cleave_hip_max_of_f32(const float* x, int64_t len) {
    return reduce_to_host<float>([&](float* d) { return cleave_hip_reduce_max_f32(x, len, d, nullptr); }, NAN);
}

int64_t cleave_hip_argmax_f32(const float* x, int64_t len) {
    return reduce_to_host<int64_t>([&](int64_t* d) { return cleave_hip_reduce_max_f32(x, len, nullptr, d); }, -1);
}

double cleave_hip_sum_f64(const double* x, int64_t len) {
    return reduce_to_host<double>([&](double* d) { return cleave_hip_reduce_sum_f64(x, len, d); }, NAN);
}

double cleave_hip_mean_f64(const double* x, int64_t len) {
    double s = cleave_hip_sum_f64(x, len);
    return s / (double)len;  // sum(v) / N.to() on f64, stdlib/nn/nn.cleave:135-138
}

double cleave_hip_max_of_f64(const double* x, int64_t len) {
    return reduce_to_host<double>([&](double* d) { return cleave_hip_reduce_max_f64(x, len, d, nullptr); }, NAN);
}

int64_t cleave_hip_argmax_f64(const double* x, int64_t len) {
    return reduce_to_host<int64_t>([&](int64_t* d) { return cleave_hip_reduce_max_f64(x, len, nullptr, d); }, -1);
}

int64_t cleave_hip_sum_i32_i64(const int32_t* x, int64_t len) {
    return reduce_to_host<int64_t>([&](int64_t* d) { return cleave_hip_reduce_sum_i32_i64(x, len, d); }, 0);
}

uint64_t cleave_hip_sum_u32_u64(const uint32_t* x, int64_t len) {
    return reduce_to_host<uint64_t>([&](uint64_t* d) { return cleave_hip_reduce_sum_u32_u64(x, len, d); }, 0);
}

}  // extern "C"
