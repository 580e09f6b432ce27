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
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// Stage-1 grid: enough blocks for 16 per CU (a function of the length and the
// CU count only, so results are reproducible on a given device).
unsigned stage1_blocks(int64_t nvec) {
    int64_t want = (nvec + (int64_t)kThreads * kUnroll - 1) / ((int64_t)kThreads * kUnroll);
    int64_t cap = (int64_t)ch::num_cus() * 16;
    if (want > cap) want = cap;
    return (unsigned)(want < 1 ? 1 : want);
}

// ---- sum f32 --------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ float block_sum(float v) {
    __shared__ float part[kThreads / 64];
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = 0.0f;
    if (threadIdx.x == 0)
        for (int w = 0; w < kThreads / 64; ++w) r += part[w];
    return r;  // valid in thread 0
}

__global__ __launch_bounds__(kThreads) void sum_f32_stage1(const float* __restrict__ x,
                                                           int64_t n, float* __restrict__ partial,
                                                           int aligned) {
    float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
    if (aligned) {
        const int64_t nv = n / 4;
        const int64_t step = (int64_t)gridDim.x * kThreads * kUnroll;
        for (int64_t base = (int64_t)blockIdx.x * kThreads * kUnroll + threadIdx.x; base < nv; base += step) {
            f4 v[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                int64_t i = base + (int64_t)u * kThreads;
                v[u] = i < nv ? __builtin_nontemporal_load(reinterpret_cast<const f4*>(x) + i) : f4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                acc0 += v[u][0];
                acc1 += v[u][1];
                acc2 += v[u][2];
                acc3 += v[u][3];
            }
        }
        if (blockIdx.x == 0 && threadIdx.x < (n & 3)) acc0 += x[nv * 4 + threadIdx.x];
    } else {
        for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
            acc0 += x[i];
    }
    float r = block_sum((acc0 + acc1) + (acc2 + acc3));
    if (threadIdx.x == 0) partial[blockIdx.x] = r;
}

// Stage 2 folds thread t's partials t, t + 256, ... in that order.  The
// loads of a run of kStage2Loads go out together before the adds: one memory
// latency per run instead of one per partial (5.2 us -> ~1.5 us for 4096
// partials; the order, and so the result, is unchanged).
constexpr int kStage2Loads = 16;

__global__ __launch_bounds__(kThreads) void sum_f32_stage2(const float* __restrict__ partial,
                                                           int nparts, float* __restrict__ out) {
    float acc = 0.f;
    for (int i0 = threadIdx.x; i0 < nparts; i0 += kThreads * kStage2Loads) {
        float v[kStage2Loads];
#pragma unroll
        for (int u = 0; u < kStage2Loads; ++u) {
            const int i = i0 + u * kThreads;
            v[u] = i < nparts ? partial[i] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < kStage2Loads; ++u)
            if (i0 + u * kThreads < nparts) acc += v[u];
    }
    float r = block_sum(acc);
    if (threadIdx.x == 0) *out = r;
}

// ---- max / argmax f32 -------------------------------------------------------
struct Best {
    float v;
    int64_t i;
};
__device__ __forceinline__ void take_better(Best& a, float v, int64_t i) {
    // Comparisons involving NaN are false, so a NaN candidate never wins.
    if (v > a.v || (v == a.v && i < a.i)) {
        a.v = v;
        a.i = i;
    }
}
__device__ __forceinline__ Best wave_best(Best b) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float v = __shfl_xor(b.v, o);
        int64_t i = __shfl_xor(b.i, o);
        take_better(b, v, i);
    }
    return b;
}
__device__ Best block_best(Best b) {
    __shared__ float pv[kThreads / 64];
    __shared__ int64_t pi[kThreads / 64];
    b = wave_best(b);
    if ((threadIdx.x & 63) == 0) {
        pv[threadIdx.x >> 6] = b.v;
        pi[threadIdx.x >> 6] = b.i;
    }
    __syncthreads();
    Best r{-INFINITY, INT64_MAX};
    if (threadIdx.x == 0)
        for (int w = 0; w < kThreads / 64; ++w) take_better(r, pv[w], pi[w]);
    return r;
}

__global__ __launch_bounds__(kThreads) void max_f32_stage1(const float* __restrict__ x, int64_t n,
                                                           float* __restrict__ pv,
                                                           int64_t* __restrict__ pi, int aligned) {
    Best b{-INFINITY, INT64_MAX};
    if (aligned) {
        const int64_t nv = n / 4;
        const int64_t step = (int64_t)gridDim.x * kThreads * kUnroll;
        for (int64_t base = (int64_t)blockIdx.x * kThreads * kUnroll + threadIdx.x; base < nv; base += step) {
            f4 v[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                int64_t i = base + (int64_t)u * kThreads;
                if (i < nv) v[u] = __builtin_nontemporal_load(reinterpret_cast<const f4*>(x) + i);
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                int64_t i = base + (int64_t)u * kThreads;
                if (i < nv) {
                    take_better(b, v[u][0], 4 * i + 0);
                    take_better(b, v[u][1], 4 * i + 1);
                    take_better(b, v[u][2], 4 * i + 2);
                    take_better(b, v[u][3], 4 * i + 3);
                }
            }
        }
        if (blockIdx.x == 0 && threadIdx.x < (n & 3)) take_better(b, x[nv * 4 + threadIdx.x], nv * 4 + threadIdx.x);
    } else {
        for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
            take_better(b, x[i], i);
    }
    Best r = block_best(b);
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = r.v;
        pi[blockIdx.x] = r.i;
    }
}

__global__ __launch_bounds__(kThreads) void max_f32_stage2(const float* __restrict__ x,
                                                           const float* __restrict__ pv,
                                                           const int64_t* __restrict__ pi,
                                                           int nparts, float* __restrict__ out_v,
                                                           int64_t* __restrict__ out_i) {
    Best b{-INFINITY, INT64_MAX};
    for (int i0 = threadIdx.x; i0 < nparts; i0 += kThreads * kStage2Loads) {
        float v[kStage2Loads];
        int64_t ix[kStage2Loads];
#pragma unroll
        for (int u = 0; u < kStage2Loads; ++u) {
            const int i = i0 + u * kThreads;
            v[u] = i < nparts ? pv[i] : -INFINITY;
            ix[u] = i < nparts ? pi[i] : INT64_MAX;
        }
#pragma unroll
        for (int u = 0; u < kStage2Loads; ++u)
            if (i0 + u * kThreads < nparts) take_better(b, v[u], ix[u]);
    }
    Best r = block_best(b);
    if (threadIdx.x == 0) {
        float x0 = x[0];
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

}  // namespace

extern "C" {

int32_t cleave_hip_reduce_sum_f32(const float* x, int64_t len, float* out_dev) {
    CH_REQUIRE(len >= 1, "cleave_hip_reduce_sum_f32: length must be >= 1 (sum reads v[0])");
    CH_REQUIRE(x && out_dev, "cleave_hip_reduce_sum_f32: null buffer");
    CH_INIT_OR_RETURN();
    CH_DEVICE("cleave_hip_reduce_sum_f32", x, len * 4);
    CH_DEVICE("cleave_hip_reduce_sum_f32", out_dev, 4);
    const int aligned = aligned16(x);
    unsigned blocks = stage1_blocks(aligned ? len / 4 + 1 : len / kUnroll + 1);
    float* part = (float*)ch::scratch(0, sizeof(float) * blocks);
    if (!part) return CLEAVE_HIP_ERR_OOM;
    sum_f32_stage1<<<blocks, kThreads, 0, ch::stream()>>>(x, len, part, aligned);
    CH_LAUNCHED("sum_f32_stage1");
    sum_f32_stage2<<<1, kThreads, 0, ch::stream()>>>(part, (int)blocks, out_dev);
    CH_LAUNCHED("sum_f32_stage2");
    return CLEAVE_HIP_OK;
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
    sum_f32_stage1<<<blocks, kThreads, 0, ch::stream()>>>(x, len, part, aligned);
    CH_LAUNCHED("sum_f32_stage1");
    sum_f32_stage2<<<1, kThreads, 0, ch::stream()>>>(part, (int)blocks, out_dev);
    CH_LAUNCHED("sum_f32_stage2");
    return CLEAVE_HIP_OK;
}

int32_t cleave_hip_reduce_max_f32(const float* x, int64_t len, float* max_dev, int64_t* argmax_dev) {
    CH_REQUIRE(len >= 1, "cleave_hip_reduce_max_f32: length must be >= 1 (max_of reads v[0])");
    CH_REQUIRE(x && (max_dev || argmax_dev), "cleave_hip_reduce_max_f32: null buffer");
    CH_INIT_OR_RETURN();
    CH_DEVICE("cleave_hip_reduce_max_f32", x, len * 4);
    if (max_dev) CH_DEVICE("cleave_hip_reduce_max_f32", max_dev, 4);
    if (argmax_dev) CH_DEVICE("cleave_hip_reduce_max_f32", argmax_dev, 8);
    const int aligned = aligned16(x);
    unsigned blocks = stage1_blocks(aligned ? len / 4 + 1 : len / kUnroll + 1);
    char* base = (char*)ch::scratch(1, (sizeof(float) + sizeof(int64_t)) * blocks + 64);
    if (!base) return CLEAVE_HIP_ERR_OOM;
    int64_t* pi = (int64_t*)base;
    float* pv = (float*)(base + sizeof(int64_t) * blocks);
    max_f32_stage1<<<blocks, kThreads, 0, ch::stream()>>>(x, len, pv, pi, aligned);
    CH_LAUNCHED("max_f32_stage1");
    max_f32_stage2<<<1, kThreads, 0, ch::stream()>>>(x, pv, pi, (int)blocks, max_dev, argmax_dev);
    CH_LAUNCHED("max_f32_stage2");
    return CLEAVE_HIP_OK;
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

// Host-returning forms: queue the reduction into a library-owned device word,
// then copy it back (synchronising the stream).
float cleave_hip_sum_f32(const float* x, int64_t len) {
    ch::clear_error();
    if (ch::ensure_init() != CLEAVE_HIP_OK) return NAN;
    float* d = (float*)ch::scratch(3, 64);
    if (!d) return NAN;
    if (cleave_hip_reduce_sum_f32(x, len, d) != CLEAVE_HIP_OK) return NAN;
    float r = NAN;
    if (cleave_hip_download(&r, d, sizeof(float)) != (int64_t)sizeof(float)) return NAN;
    return r;
}

float cleave_hip_mean_f32(const float* x, int64_t len) {
    float s = cleave_hip_sum_f32(x, len);
    return s / (float)len;  // sum(v) / sitofp(N), stdlib/nn/nn.cleave:135-138
}

float cleave_hip_max_of_f32(const float* x, int64_t len) {
    ch::clear_error();
    if (ch::ensure_init() != CLEAVE_HIP_OK) return NAN;
    float* d = (float*)ch::scratch(3, 64);
    if (!d) return NAN;
    if (cleave_hip_reduce_max_f32(x, len, d, nullptr) != CLEAVE_HIP_OK) return NAN;
    float r = NAN;
    if (cleave_hip_download(&r, d, sizeof(float)) != (int64_t)sizeof(float)) return NAN;
    return r;
}

int64_t cleave_hip_argmax_f32(const float* x, int64_t len) {
    ch::clear_error();
    if (ch::ensure_init() != CLEAVE_HIP_OK) return -1;
    int64_t* d = (int64_t*)ch::scratch(3, 64);
    if (!d) return -1;
    if (cleave_hip_reduce_max_f32(x, len, nullptr, d) != CLEAVE_HIP_OK) return -1;
    int64_t r = -1;
    if (cleave_hip_download(&r, d, sizeof(int64_t)) != (int64_t)sizeof(int64_t)) return -1;
    return r;
}

int64_t cleave_hip_sum_i32_i64(const int32_t* x, int64_t len) {
    ch::clear_error();
    if (ch::ensure_init() != CLEAVE_HIP_OK) return 0;
    int64_t* d = (int64_t*)ch::scratch(3, 64);
    if (!d) return 0;
    if (cleave_hip_reduce_sum_i32_i64(x, len, d) != CLEAVE_HIP_OK) return 0;
    int64_t r = 0;
    if (cleave_hip_download(&r, d, sizeof(int64_t)) != (int64_t)sizeof(int64_t)) return 0;
    return r;
}

uint64_t cleave_hip_sum_u32_u64(const uint32_t* x, int64_t len) {
    ch::clear_error();
    if (ch::ensure_init() != CLEAVE_HIP_OK) return 0;
    uint64_t* d = (uint64_t*)ch::scratch(3, 64);
    if (!d) return 0;
    if (cleave_hip_reduce_sum_u32_u64(x, len, d) != CLEAVE_HIP_OK) return 0;
    uint64_t r = 0;
    if (cleave_hip_download(&r, d, sizeof(uint64_t)) != (int64_t)sizeof(uint64_t)) return 0;
    return r;
}

}  // extern "C"
