// runtime.hip -- device/stream ownership, buffers, errors, events, synthetic
// input generators and the symbol table of libcleave_hip.so.
//
// Replaces cleave-rt's native surface (/root/reference/cleave-rt/src/lib.rs):
// cleave_alloc -> cleave_hip_buf_alloc (lib.rs:56-71), the JIT registration
// list (cleave/src/pipeline.rs:159-198) -> cleave_hip_symbols().
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <vector>

#include "common.hpp"

// The allocation-free entry point's workspace: in the code object's global
// segment, so each device the library loads on holds its own copy until the
// process ends, and no call allocates it.  In host code `scratch` names a host
// stand-in, never the device array: kernels are handed the address that
// hipGetSymbolAddress returns (State::noalloc below).
static __device__ __align__(256) float scratch[ch::kNoAllocFloats];

namespace ch {

namespace {
struct State {
    std::once_flag once;
    int32_t init_status = CLEAVE_HIP_ERR_RUNTIME;
    hipStream_t stream = nullptr;
    int cus = 0;
    void* scratch[kScratchSlots] = {};
    size_t scratch_bytes[kScratchSlots] = {};
    float* noalloc = nullptr;  // device address of ::scratch on device 0
};
State g;
int g_abort_on_error = 1;
thread_local int32_t t_last_error = CLEAVE_HIP_OK;
thread_local char t_last_msg[512] = "";
}  // namespace

hipStream_t stream() { return g.stream; }
int num_cus() { return g.cus; }
float* noalloc_workspace() { return g.noalloc; }

int32_t fail(int32_t code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_last_msg, sizeof(t_last_msg), fmt, ap);
    va_end(ap);
    t_last_error = code;
    if (g_abort_on_error) {
        fprintf(stderr, "cleave_hip: error %d: %s\n", code, t_last_msg);
        fflush(stderr);
        abort();
    }
    return code;
}

void clear_error() {
    t_last_error = CLEAVE_HIP_OK;
    t_last_msg[0] = 0;
}

int32_t check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return CLEAVE_HIP_OK;
    int32_t code = (e == hipErrorOutOfMemory) ? CLEAVE_HIP_ERR_OOM : CLEAVE_HIP_ERR_RUNTIME;
    return fail(code, "%s: %s", what, hipGetErrorString(e));
}

int32_t ensure_init() {
    std::call_once(g.once, [] {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
            (void)hipGetLastError();
            return;
        }
        if (hipSetDevice(0) != hipSuccess) return;
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, 0) != hipSuccess) return;
        g.cus = prop.multiProcessorCount;
        // Default priority stream, non-blocking w.r.t. the legacy null stream.
        if (hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking) != hipSuccess) return;
        // The library runs on device 0 only, which is current here: resolve
        // that device's copy of the static workspace once.
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(::scratch)) == hipSuccess && p != nullptr)
            g.noalloc = static_cast<float*>(p);
        else
            (void)hipGetLastError();  // only the allocation-free entry point needs it
        g.init_status = CLEAVE_HIP_OK;
    });
    if (g.init_status != CLEAVE_HIP_OK)
        return fail(CLEAVE_HIP_ERR_RUNTIME, "no usable HIP device (hipGetDeviceCount/hipSetDevice failed)");
    return CLEAVE_HIP_OK;
}

void* scratch(int slot, size_t bytes) {
    void* p = scratch_try(slot, bytes);
    if (!p) fail(CLEAVE_HIP_ERR_OOM, "scratch allocation of %zu bytes failed", bytes);
    return p;
}

namespace {
size_t release_cached();
}  // namespace

void* scratch_try(int slot, size_t bytes) {
    if (slot < 0 || slot >= kScratchSlots) return nullptr;
    if (g.scratch_bytes[slot] >= bytes && g.scratch[slot]) return g.scratch[slot];
    if (g.scratch[slot]) {
        // The old buffer may still be read by queued work.
        (void)hipStreamSynchronize(g.stream);
        (void)hipFree(g.scratch[slot]);
        g.scratch[slot] = nullptr;
        g.scratch_bytes[slot] = 0;
    }
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        (void)hipGetLastError();
        // The cache of freed buffers may hold the memory: return it to the
        // device and try once more, as buf_alloc does.
        if (release_cached() == 0 || hipMalloc(&p, bytes) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
    }
    g.scratch[slot] = p;
    g.scratch_bytes[slot] = bytes;
    return p;
}

namespace {
// Buffers of cleave_hip_buf_alloc.  A freed buffer goes to a cache of free
// blocks by size, for the next request of that size.  Everything runs on the
// library stream, so work queued by the next owner runs after every use by
// the previous one, and a free needs no synchronisation.  (hipFree took
// ~250 us for 1 GiB, after the stream synchronisation it needs, with the GPU
// idle meanwhile; a reverse-mode training step frees several such buffers.)
// Blocks are rounded up to 512 bytes, or to 2 MiB above 1 MiB.  The cache
// holds at most kPoolCap bytes, and is emptied (stream synchronised, blocks
// freed) when hipMalloc fails, before the allocation is tried again.
struct BufPool {
    std::mutex mu;
    std::map<uintptr_t, std::pair<uint64_t, size_t>> live;  // base -> (bytes asked for, block size)
    std::multimap<size_t, void*> cached;                     // block size -> free block
    std::map<uintptr_t, size_t> cached_at;                   // base -> block size, the same free blocks
    size_t cached_bytes = 0;
};
BufPool g_pool;
constexpr size_t kPoolCap = size_t(32) << 30;

size_t block_size(uint64_t bytes) {
    const uint64_t q = bytes <= (uint64_t(1) << 20) ? 512 : (uint64_t(2) << 20);
    return (size_t)((bytes + q - 1) / q * q);
}

// Returns every cached block to the device; the bytes released.
size_t release_cached() {
    std::vector<void*> blocks;
    size_t bytes = 0;
    {
        std::lock_guard<std::mutex> lk(g_pool.mu);
        for (auto& kv : g_pool.cached) blocks.push_back(kv.second);
        bytes = g_pool.cached_bytes;
        g_pool.cached.clear();
        g_pool.cached_at.clear();
        g_pool.cached_bytes = 0;
    }
    if (blocks.empty()) return 0;
    (void)hipStreamSynchronize(g.stream);
    for (void* b : blocks) (void)hipFree(b);
    (void)hipGetLastError();
    return bytes;
}

// True when p lies in a freed block that waits in the cache: a pointer into
// a buffer its owner already released.
bool in_cached_block(const void* p) {
    const uintptr_t q = (uintptr_t)p;
    std::lock_guard<std::mutex> lk(g_pool.mu);
    auto it = g_pool.cached_at.upper_bound(q);
    if (it == g_pool.cached_at.begin()) return false;
    --it;
    return q < it->first + it->second;
}

// The bytes from p to the end of the library buffer holding it (what its
// owner asked for; 0 past that); false when p is in no such buffer.
bool pool_extent(const void* p, uint64_t* avail) {
    const uintptr_t q = (uintptr_t)p;
    std::lock_guard<std::mutex> lk(g_pool.mu);
    auto it = g_pool.live.upper_bound(q);
    if (it == g_pool.live.begin()) return false;
    --it;
    const uintptr_t base = it->first;
    if (q >= base + it->second.second) return false;
    *avail = q < base + it->second.first ? base + it->second.first - q : 0;
    return true;
}
}  // namespace

void* buf_alloc(uint64_t bytes) {
    const size_t sz = block_size(bytes);
    void* p = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_pool.mu);
        auto it = g_pool.cached.find(sz);
        if (it != g_pool.cached.end()) {
            p = it->second;
            g_pool.cached.erase(it);
            g_pool.cached_at.erase((uintptr_t)p);
            g_pool.cached_bytes -= sz;
        }
    }
    if (!p) {
        hipError_t e = hipMalloc(&p, sz);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            release_cached();
            e = hipMalloc(&p, sz);
        }
        if (e != hipSuccess) {
            check_hip(e, "hipMalloc");
            return nullptr;
        }
    }
    std::lock_guard<std::mutex> lk(g_pool.mu);
    g_pool.live[(uintptr_t)p] = {bytes, sz};
    return p;
}

void buf_free(void* buf) {
    {
        std::lock_guard<std::mutex> lk(g_pool.mu);
        auto it = g_pool.live.find((uintptr_t)buf);
        if (it != g_pool.live.end()) {
            const size_t sz = it->second.second;
            g_pool.live.erase(it);
            if (g_pool.cached_bytes + sz <= kPoolCap) {
                g_pool.cached.emplace(sz, buf);
                g_pool.cached_at[(uintptr_t)buf] = sz;
                g_pool.cached_bytes += sz;
                return;
            }
        }
    }
    // Not cached (the cache is full, or the buffer is not the library's):
    // queued work may still use it.
    if (check_hip(hipStreamSynchronize(g.stream), "hipStreamSynchronize") != CLEAVE_HIP_OK) return;
    check_hip(hipFree(buf), "hipFree");
}

size_t buf_trim() { return release_cached(); }

size_t buf_cached_bytes() {
    std::lock_guard<std::mutex> lk(g_pool.mu);
    return g_pool.cached_bytes;
}

int32_t require_device(const char* fn, const char* what, const void* p, uint64_t bytes) {
    hipPointerAttribute_t at{};
    if (hipPointerGetAttributes(&at, p) != hipSuccess) {
        // A pointer the runtime does not know at all.
        (void)hipGetLastError();
        return fail(CLEAVE_HIP_ERR_ARG,
                    "%s: %s (%p) is not device memory; pass a buffer from cleave_hip_buf_alloc "
                    "(the _host entry points take host arrays)", fn, what, p);
    }
    // Unregistered (type 0, what ROCm 7 reports for pageable memory) or pinned
    // host memory: a kernel must not be handed either.
    if (at.type != hipMemoryTypeDevice && at.type != hipMemoryTypeManaged)
        return fail(CLEAVE_HIP_ERR_ARG,
                    "%s: %s (%p) is not device memory (memory type %d); pass a buffer from "
                    "cleave_hip_buf_alloc (the _host entry points take host arrays)", fn, what, p, (int)at.type);
    if (in_cached_block(p))
        return fail(CLEAVE_HIP_ERR_ARG,
                    "%s: %s (%p) points into a buffer that was freed (cleave_hip_buf_free); allocate a new one",
                    fn, what, p);
    uint64_t avail = 0;
    if (pool_extent(p, &avail)) {
        if (bytes > avail)
            return fail(CLEAVE_HIP_ERR_ARG,
                        "%s: %s needs %llu bytes from %p, but its allocation holds %llu bytes from there", fn, what,
                        (unsigned long long)bytes, p, (unsigned long long)avail);
        return CLEAVE_HIP_OK;
    }
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p) == hipSuccess) {
        const uintptr_t lo = (uintptr_t)base, q = (uintptr_t)p;
        if (q < lo || bytes > (uint64_t)(lo + size - q))
            return fail(CLEAVE_HIP_ERR_ARG,
                        "%s: %s needs %llu bytes from %p, but its allocation holds %llu bytes from there",
                        fn, what, (unsigned long long)bytes, p,
                        (unsigned long long)(q >= lo && q - lo <= size ? lo + size - q : 0));
    } else {
        (void)hipGetLastError();
    }
    return CLEAVE_HIP_OK;
}

}  // namespace ch

// ---------------------------------------------------------------------------
// generators (device side): counter-based splitmix64, identical integer
// stream to the CPU restatement, so uniform draws match bit for bit.
// ---------------------------------------------------------------------------
namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t splitmix_at(uint64_t seed, uint64_t i) {
    return mix64(seed + (i + 1) * 0x9E3779B97F4A7C15ULL);
}
__device__ __forceinline__ float unit24(uint64_t x) {
    return (float)(x >> 40) * 5.9604644775390625e-08f;
}

__global__ void fill_uniform_kernel(float* out, int64_t n, uint64_t seed, float lo, float w) {
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = lo + w * unit24(splitmix_at(seed, (uint64_t)i));
}

__global__ void fill_normal_kernel(float* out, int64_t n, uint64_t seed, float mean, float sd) {
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        uint64_t a = splitmix_at(seed, 2 * (uint64_t)i);
        uint64_t b = splitmix_at(seed, 2 * (uint64_t)i + 1);
        double u1 = ((double)(a >> 11) + 1.0) * 0x1.0p-53;
        double u2 = (double)(b >> 11) * 0x1.0p-53;
        double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        out[i] = (float)((double)mean + (double)sd * z);
    }
}

__global__ void fill_bernoulli_kernel(float* out, int64_t n, uint64_t seed, float p) {
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = unit24(splitmix_at(seed, (uint64_t)i)) < p ? 1.0f : 0.0f;
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__global__ void cast_f32_bf16_kernel(const float* in, uint16_t* out, int64_t n) {
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = f32_to_bf16_rne(in[i]);
}

unsigned grid_for(int64_t n, int threads) {
    int64_t blocks = (n + threads - 1) / threads;
    int64_t cap = (int64_t)ch::num_cus() * 16;
    if (cap < 1) cap = 1024;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    return (unsigned)blocks;
}

}  // namespace

// ---------------------------------------------------------------------------
// extern "C" runtime surface
// ---------------------------------------------------------------------------
extern "C" {

int32_t cleave_hip_init(void) { return ch::ensure_init(); }

int32_t cleave_hip_device_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n > 0 ? 1 : 0;
}

void* cleave_hip_buf_alloc(int64_t bytes) {
    if (ch::ensure_init() != CLEAVE_HIP_OK) return nullptr;
    if (bytes <= 0) {
        ch::fail(CLEAVE_HIP_ERR_ARG, "cleave_hip_buf_alloc: bytes must be > 0 (got %lld)", (long long)bytes);
        return nullptr;
    }
    return ch::buf_alloc((uint64_t)bytes);
}

void cleave_hip_buf_free(void* buf) {
    if (!buf) return;
    if (ch::ensure_init() != CLEAVE_HIP_OK) return;
    ch::buf_free(buf);
}

int64_t cleave_hip_buf_trim(void) {
    CH_INIT_OR_RETURN();
    return (int64_t)ch::buf_trim();
}

int64_t cleave_hip_buf_cached_bytes(void) {
    CH_INIT_OR_RETURN();
    return (int64_t)ch::buf_cached_bytes();
}

int64_t cleave_hip_upload(void* dst_dev, const void* src_host, int64_t bytes) {
    CH_REQUIRE(bytes >= 0 && (bytes == 0 || (dst_dev && src_host)),
               "cleave_hip_upload: null pointer or negative size");
    CH_INIT_OR_RETURN();
    if (bytes == 0) return 0;
    CH_DEVICE("cleave_hip_upload", dst_dev, bytes);
    CH_HIP(hipMemcpyAsync(dst_dev, src_host, (size_t)bytes, hipMemcpyHostToDevice, ch::stream()));
    CH_HIP(hipStreamSynchronize(ch::stream()));
    return bytes;
}

int64_t cleave_hip_download(void* dst_host, const void* src_dev, int64_t bytes) {
    CH_REQUIRE(bytes >= 0 && (bytes == 0 || (dst_host && src_dev)),
               "cleave_hip_download: null pointer or negative size");
    CH_INIT_OR_RETURN();
    if (bytes == 0) return 0;
    CH_DEVICE("cleave_hip_download", src_dev, bytes);
    CH_HIP(hipMemcpyAsync(dst_host, src_dev, (size_t)bytes, hipMemcpyDeviceToHost, ch::stream()));
    CH_HIP(hipStreamSynchronize(ch::stream()));
    return bytes;
}

int32_t cleave_hip_sync(void) {
    CH_INIT_OR_RETURN();
    CH_HIP(hipStreamSynchronize(ch::stream()));
    return CLEAVE_HIP_OK;
}

void cleave_hip_set_abort_on_error(int32_t on) { ch::g_abort_on_error = on ? 1 : 0; }
int32_t cleave_hip_last_error(void) { return ch::t_last_error; }
const char* cleave_hip_last_error_message(void) { return ch::t_last_msg; }

void* cleave_hip_event_create(void) {
    if (ch::ensure_init() != CLEAVE_HIP_OK) return nullptr;
    hipEvent_t ev = nullptr;
    if (ch::check_hip(hipEventCreate(&ev), "hipEventCreate") != CLEAVE_HIP_OK) return nullptr;
    return (void*)ev;
}

int32_t cleave_hip_event_record(void* ev) {
    CH_REQUIRE(ev != nullptr, "cleave_hip_event_record: null event");
    CH_INIT_OR_RETURN();
    CH_HIP(hipEventRecord((hipEvent_t)ev, ch::stream()));
    return CLEAVE_HIP_OK;
}

float cleave_hip_event_elapsed_ms(void* start, void* stop) {
    if (ch::ensure_init() != CLEAVE_HIP_OK) return -1.0f;
    if (!start || !stop) {
        ch::fail(CLEAVE_HIP_ERR_ARG, "cleave_hip_event_elapsed_ms: null event");
        return -1.0f;
    }
    if (ch::check_hip(hipEventSynchronize((hipEvent_t)stop), "hipEventSynchronize") != CLEAVE_HIP_OK)
        return -1.0f;
    float ms = 0.0f;
    if (ch::check_hip(hipEventElapsedTime(&ms, (hipEvent_t)start, (hipEvent_t)stop),
                      "hipEventElapsedTime") != CLEAVE_HIP_OK)
        return -1.0f;
    return ms;
}

void cleave_hip_event_destroy(void* ev) {
    if (ev) (void)hipEventDestroy((hipEvent_t)ev);
}

int32_t cleave_hip_fill_uniform_f32(float* out, int64_t len, uint64_t seed, float lo, float hi) {
    CH_REQUIRE(out && len > 0, "cleave_hip_fill_uniform_f32: null buffer or empty length");
    CH_INIT_OR_RETURN();
    CH_DEVICE("cleave_hip_fill_uniform_f32", out, len * 4);
    fill_uniform_kernel<<<grid_for(len, 256), 256, 0, ch::stream()>>>(out, len, seed, lo, hi - lo);
    CH_LAUNCHED("fill_uniform_kernel");
    return CLEAVE_HIP_OK;
}

int32_t cleave_hip_fill_normal_f32(float* out, int64_t len, uint64_t seed, float mean, float std) {
    CH_REQUIRE(out && len > 0, "cleave_hip_fill_normal_f32: null buffer or empty length");
    CH_INIT_OR_RETURN();
    CH_DEVICE("cleave_hip_fill_normal_f32", out, len * 4);
    fill_normal_kernel<<<grid_for(len, 256), 256, 0, ch::stream()>>>(out, len, seed, mean, std);
    CH_LAUNCHED("fill_normal_kernel");
    return CLEAVE_HIP_OK;
}

int32_t cleave_hip_fill_bernoulli_f32(float* out, int64_t len, uint64_t seed, float p) {
    CH_REQUIRE(out && len > 0, "cleave_hip_fill_bernoulli_f32: null buffer or empty length");
    CH_INIT_OR_RETURN();
    CH_DEVICE("cleave_hip_fill_bernoulli_f32", out, len * 4);
    fill_bernoulli_kernel<<<grid_for(len, 256), 256, 0, ch::stream()>>>(out, len, seed, p);
    CH_LAUNCHED("fill_bernoulli_kernel");
    return CLEAVE_HIP_OK;
}

int32_t cleave_hip_cast_f32_bf16(const float* in, int64_t inlen, uint16_t* out, int64_t outlen) {
    CH_REQUIRE(in && out && inlen > 0, "cleave_hip_cast_f32_bf16: null buffer or empty length");
    CH_REQUIRE(inlen == outlen, "cleave_hip_cast_f32_bf16: inlen %lld != outlen %lld",
               (long long)inlen, (long long)outlen);
    CH_INIT_OR_RETURN();
    CH_DEVICE("cleave_hip_cast_f32_bf16", in, inlen * 4);
    CH_DEVICE("cleave_hip_cast_f32_bf16", out, outlen * 2);
    cast_f32_bf16_kernel<<<grid_for(inlen, 256), 256, 0, ch::stream()>>>(in, out, inlen);
    CH_LAUNCHED("cast_f32_bf16_kernel");
    return CLEAVE_HIP_OK;
}

}  // extern "C"
