// host.cpp -- host-array forms (`<entry>_host`) of the compute entry points.
//
// cleave's extern lowering passes an array argument as the aligned pointer of
// a host memref plus its element count (cleave/src/mlir_lower.rs:1720-1751),
// and cleave-rt reads that memory on the host (sum_bytes,
// cleave-rt/src/lib.rs:86-90).  These entry points accept exactly that: every
// tensor operand is a borrowed, possibly pageable host array, valid only for
// the call.  Each one
//   1. copies its input arrays into a staging arena in HBM (on the library
//      stream; the arena is library scratch, grown on demand and kept),
//   2. runs the device entry point on the staged copies (same kernels, same
//      argument checks, same error contract),
//   3. copies its output arrays back and waits for the stream,
// so on return every output array holds its result and every array may be
// reused.  A call whose device entry point fails (bad lengths, shapes or
// flags, a launch error) leaves the output arrays unwritten.
//
// Copies of more than 4 MiB go through two pinned bounce buffers of 16 MiB:
// host threads copy one chunk between the pageable array and a bounce buffer
// while the DMA engine moves the other one, so the pageable side is copied
// (and its pages touched) by several cores at once instead of by the
// runtime's one staging thread.  Smaller copies are one hipMemcpyAsync.
#include <algorithm>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

#include <unistd.h>

#include "common.hpp"
#include "copy_split.hpp"

namespace {

constexpr size_t kBounceBytes = size_t(16) << 20;
constexpr size_t kDirectMax = size_t(4) << 20;
constexpr size_t kCopySlice = size_t(2) << 20;  // least bytes per copying thread

// Two pinned bounce buffers and the events that say when the DMA engine is
// done with each; allocated on the first large copy and kept until the
// process ends.
struct Bounce {
    char* buf[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool ready = false;
};
Bounce g_bounce;

int32_t bounce_init() {
    if (g_bounce.ready) return CLEAVE_HIP_OK;
    for (int b = 0; b < 2; ++b) {
        int32_t st = ch::check_hip(hipHostMalloc((void**)&g_bounce.buf[b], kBounceBytes, hipHostMallocDefault),
                                   "hipHostMalloc (bounce buffer)");
        if (st != CLEAVE_HIP_OK) return st;
        st = ch::check_hip(hipEventCreateWithFlags(&g_bounce.done[b], hipEventDisableTiming),
                           "hipEventCreateWithFlags (bounce buffer)");
        if (st != CLEAVE_HIP_OK) return st;
    }
    g_bounce.ready = true;
    return CLEAVE_HIP_OK;
}

// Worker threads for the bounce copies: up to 7 beside the caller, started
// on the first large copy and stopped when the process ends.
class CopyPool {
  public:
    ~CopyPool() {
        if (!started_ || getpid() != pid_) {  // a forked child has no workers to join
            for (auto& t : th_) t.detach();
            return;
        }
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        work_.notify_all();
        for (auto& t : th_) t.join();
    }
    size_t workers() {
        if (started_ && getpid() != pid_) return 0;  // forked child: copy on this thread
        if (!started_) {
            pid_ = getpid();
            const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
            const unsigned n = std::min(7u, hw > 1 ? hw - 1 : 0u);
            for (unsigned i = 0; i < n; ++i) th_.emplace_back([this] { run(); });
            started_ = true;
        }
        return th_.size();
    }
    // memcpy of n bytes, split over the workers and the calling thread
    // (ranges from copy_split.hpp: together they cover all n bytes).
    void copy(void* dst, const void* src, size_t n) {
        const ch::CopySplit s = ch::copy_split(n, workers() + 1, kCopySlice);
        if (s.parts <= 1) {
            memcpy(dst, src, n);
            return;
        }
        {
            std::lock_guard<std::mutex> lk(mu_);
            for (size_t p = 1; p < s.parts; ++p) {
                size_t off, len;
                ch::copy_range(s, n, p, &off, &len);
                if (len) {
                    tasks_.push_back(Task{(char*)dst + off, (const char*)src + off, len});
                    ++pending_;
                }
            }
        }
        work_.notify_all();
        size_t off0, len0;
        ch::copy_range(s, n, 0, &off0, &len0);
        memcpy(dst, src, len0);
        std::unique_lock<std::mutex> lk(mu_);
        done_.wait(lk, [this] { return pending_ == 0; });
    }

  private:
    struct Task {
        char* dst;
        const char* src;
        size_t n;
    };
    void run() {
        std::unique_lock<std::mutex> lk(mu_);
        for (;;) {
            work_.wait(lk, [this] { return stop_ || !tasks_.empty(); });
            if (tasks_.empty()) return;  // stop_ and nothing left
            const Task t = tasks_.back();
            tasks_.pop_back();
            lk.unlock();
            memcpy(t.dst, t.src, t.n);
            lk.lock();
            if (--pending_ == 0) done_.notify_all();
        }
    }
    std::vector<std::thread> th_;
    std::vector<Task> tasks_;
    std::mutex mu_;
    std::condition_variable work_, done_;
    size_t pending_ = 0;
    bool stop_ = false, started_ = false;
    pid_t pid_ = 0;
};
CopyPool g_pool;

void parallel_copy(void* dst, const void* src, size_t n) { g_pool.copy(dst, src, n); }

// host -> device on the library stream.  Returns when the host array may be
// reused (every chunk is in a bounce buffer or already copied).
int32_t to_device(void* dev, const void* host, size_t n) {
    if (n <= kDirectMax)
        return ch::check_hip(hipMemcpyAsync(dev, host, n, hipMemcpyHostToDevice, ch::stream()),
                             "hipMemcpyAsync (host array to staging)");
    int32_t st = bounce_init();
    if (st != CLEAVE_HIP_OK) return st;
    for (size_t off = 0, i = 0; off < n; off += kBounceBytes, ++i) {
        const int b = (int)(i & 1);
        const size_t len = std::min(kBounceBytes, n - off);
        // the DMA of the chunk two back, out of this buffer, is done
        st = ch::check_hip(hipEventSynchronize(g_bounce.done[b]), "hipEventSynchronize (bounce buffer)");
        if (st != CLEAVE_HIP_OK) return st;
        parallel_copy(g_bounce.buf[b], (const char*)host + off, len);
        st = ch::check_hip(hipMemcpyAsync((char*)dev + off, g_bounce.buf[b], len, hipMemcpyHostToDevice, ch::stream()),
                           "hipMemcpyAsync (bounce buffer to staging)");
        if (st != CLEAVE_HIP_OK) return st;
        st = ch::check_hip(hipEventRecord(g_bounce.done[b], ch::stream()), "hipEventRecord (bounce buffer)");
        if (st != CLEAVE_HIP_OK) return st;
    }
    return CLEAVE_HIP_OK;
}

// device -> host, after everything already queued on the library stream.
// Large copies have landed in the host array on return; small ones when the
// stream is next synchronised.
int32_t to_host(void* host, const void* dev, size_t n) {
    if (n <= kDirectMax)
        return ch::check_hip(hipMemcpyAsync(host, dev, n, hipMemcpyDeviceToHost, ch::stream()),
                             "hipMemcpyAsync (staging to host array)");
    int32_t st = bounce_init();
    if (st != CLEAVE_HIP_OK) return st;
    const size_t chunks = (n + kBounceBytes - 1) / kBounceBytes;
    auto dma = [&](size_t i) {
        const int b = (int)(i & 1);
        const size_t off = i * kBounceBytes, len = std::min(kBounceBytes, n - off);
        int32_t s2 = ch::check_hip(hipMemcpyAsync(g_bounce.buf[b], (const char*)dev + off, len, hipMemcpyDeviceToHost,
                                                  ch::stream()),
                                   "hipMemcpyAsync (staging to bounce buffer)");
        if (s2 == CLEAVE_HIP_OK)
            s2 = ch::check_hip(hipEventRecord(g_bounce.done[b], ch::stream()), "hipEventRecord (bounce buffer)");
        return s2;
    };
    for (size_t i = 0; i < std::min<size_t>(2, chunks); ++i) {
        // the buffer is free: no earlier copy of this call used it, and an
        // earlier call finished with it before returning
        st = dma(i);
        if (st != CLEAVE_HIP_OK) return st;
    }
    for (size_t i = 0; i < chunks; ++i) {
        const int b = (int)(i & 1);
        const size_t off = i * kBounceBytes, len = std::min(kBounceBytes, n - off);
        st = ch::check_hip(hipEventSynchronize(g_bounce.done[b]), "hipEventSynchronize (bounce buffer)");
        if (st != CLEAVE_HIP_OK) return st;
        parallel_copy((char*)host + off, g_bounce.buf[b], len);
        if (i + 2 < chunks) {
            st = dma(i + 2);
            if (st != CLEAVE_HIP_OK) return st;
        }
    }
    return CLEAVE_HIP_OK;
}

// Scratch slot of the staging arena (slots 0-5 belong to the reductions, the
// MLP step and the column sums).
constexpr int kArenaSlot = 6;
constexpr int kMaxArgs = 8;

// The host arrays of one call, staged through the arena.
class Staged {
  public:
    explicit Staged(const char* fn) : fn_(fn) {}

    // Declares host array i: `len` elements of `esz` bytes, copied to the
    // device before the call when `in`, and back after it when `out`.
    int add(const void* host, int64_t len, int esz, bool in, bool out) {
        const int i = n_++;
        if (i < kMaxArgs) args_[i] = Arg{host, len, esz, in, out, 0};
        return i;
    }
    int in(const void* host, int64_t len, int esz) { return add(host, len, esz, true, false); }
    int out(void* host, int64_t len, int esz) { return add(host, len, esz, false, true); }
    int inout(void* host, int64_t len, int esz) { return add(host, len, esz, true, true); }

    // Sizes the arena and queues the copies in.  Returns a status.
    int32_t stage() {
        if (n_ > kMaxArgs) return ch::fail(CLEAVE_HIP_ERR_ARG, "%s: too many operands", fn_);
        size_t total = 0;
        for (int i = 0; i < n_; ++i) {
            const Arg& a = args_[i];
            CH_REQUIRE(a.len >= 0, "%s: operand %d has negative length %lld", fn_, i, (long long)a.len);
            CH_REQUIRE(a.len == 0 || a.host != nullptr, "%s: operand %d is a null array of %lld elements",
                       fn_, i, (long long)a.len);
            CH_REQUIRE((uint64_t)a.len <= (UINT64_MAX >> 4) / (uint64_t)a.esz,
                       "%s: operand %d length %lld is too large", fn_, i, (long long)a.len);
            args_[i].off = total;
            total += ((size_t)a.len * a.esz + 255) & ~(size_t)255;  // 256-byte aligned sub-buffers
        }
        CH_INIT_OR_RETURN();
        base_ = (char*)ch::scratch(kArenaSlot, total ? total : 256);
        if (!base_) return CLEAVE_HIP_ERR_OOM;
        for (int i = 0; i < n_; ++i) {
            const Arg& a = args_[i];
            if (a.in && a.len > 0) {
                const int32_t st = to_device(base_ + a.off, a.host, (size_t)a.len * a.esz);
                if (st != CLEAVE_HIP_OK) return drain(st);
            }
        }
        staged_ = true;
        return CLEAVE_HIP_OK;
    }

    // Device address of staged array i (valid after stage()).
    template <class T>
    T* dev(int i) const {
        return reinterpret_cast<T*>(base_ + args_[i].off);
    }

    // After the device entry point returned `st`: when it succeeded, queues
    // the copies out; always waits for the stream.  Returns the first error.
    int32_t finish(int32_t st) {
        if (st == CLEAVE_HIP_OK && staged_) {
            for (int i = 0; i < n_; ++i) {
                const Arg& a = args_[i];
                if (a.out && a.len > 0) {
                    st = to_host(const_cast<void*>(a.host), base_ + a.off, (size_t)a.len * a.esz);
                    if (st != CLEAVE_HIP_OK) break;
                }
            }
        }
        return drain(st);
    }

  private:
    struct Arg {
        const void* host;
        int64_t len;
        int esz;
        bool in, out;
        size_t off;
    };

    // Waits for every queued copy, so no host array is touched after return.
    int32_t drain(int32_t st) {
        if (ch::stream() == nullptr) return st;
        const hipError_t e = hipStreamSynchronize(ch::stream());
        if (st != CLEAVE_HIP_OK) return st;
        return ch::check_hip(e, "hipStreamSynchronize");
    }

    const char* fn_;
    Arg args_[kMaxArgs] = {};
    int n_ = 0;
    char* base_ = nullptr;
    bool staged_ = false;
};

template <class T>
int32_t map1_host(const char* fn, int32_t (*f)(const T*, int64_t, T*, int64_t), const T* a, int64_t alen, T* out,
                  int64_t outlen) {
    Staged s(fn);
    const int ia = s.in(a, alen, sizeof(T)), io = s.out(out, outlen, sizeof(T));
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(f(s.dev<T>(ia), alen, s.dev<T>(io), outlen));
}

template <class T>
int32_t map2_host(const char* fn, int32_t (*f)(const T*, int64_t, const T*, int64_t, T*, int64_t), const T* a,
                  int64_t alen, const T* b, int64_t blen, T* out, int64_t outlen) {
    Staged s(fn);
    const int ia = s.in(a, alen, sizeof(T)), ib = s.in(b, blen, sizeof(T)), io = s.out(out, outlen, sizeof(T));
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(f(s.dev<T>(ia), alen, s.dev<T>(ib), blen, s.dev<T>(io), outlen));
}

// The matmul host forms: A and B staged in, C staged out.
template <class TA, class TC>
int32_t matmul_host(const char* fn,
                    int32_t (*f)(const TA*, int64_t, const TA*, int64_t, TC*, int64_t, int32_t, int32_t, int32_t,
                                 int32_t, int32_t, int32_t),
                    const TA* a, int64_t alen, const TA* b, int64_t blen, TC* c, int64_t clen, int32_t batch,
                    int32_t M, int32_t N, int32_t K, int32_t trans_a, int32_t trans_b) {
    Staged s(fn);
    const int ia = s.in(a, alen, sizeof(TA)), ib = s.in(b, blen, sizeof(TA)), ic = s.out(c, clen, sizeof(TC));
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(f(s.dev<TA>(ia), alen, s.dev<TA>(ib), blen, s.dev<TC>(ic), clen, batch, M, N, K, trans_a, trans_b));
}

// Scalar-returning reductions: stage x, then call the device form (which
// clears the error state, synchronises and returns the value).
template <class R, class T>
R reduce_host(const char* fn, R (*f)(const T*, int64_t), const T* x, int64_t len, R on_error) {
    ch::clear_error();
    Staged s(fn);
    const int ix = s.in(x, len, (int)sizeof(T));
    if (s.stage() != CLEAVE_HIP_OK) return on_error;
    const R r = f(s.dev<T>(ix), len);
    const int32_t err = cleave_hip_last_error();
    if (s.finish(CLEAVE_HIP_OK) != CLEAVE_HIP_OK || err != CLEAVE_HIP_OK) return on_error;
    return r;
}

}  // namespace

extern "C" {

// ---- MatMul -----------------------------------------------------------------

int32_t cleave_hip_matmul_f32_host(const float* a, int64_t alen, const float* b, int64_t blen, float* c,
                                   int64_t clen, int32_t M, int32_t N, int32_t K, int32_t trans_a,
                                   int32_t trans_b) {
    Staged s("cleave_hip_matmul_f32_host");
    const int ia = s.in(a, alen, 4), ib = s.in(b, blen, 4), ic = s.out(c, clen, 4);
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(cleave_hip_matmul_f32(s.dev<float>(ia), alen, s.dev<float>(ib), blen, s.dev<float>(ic), clen,
                                          M, N, K, trans_a, trans_b));
}

int32_t cleave_hip_matmul_batched_f32_host(const float* a, int64_t alen, const float* b, int64_t blen, float* c,
                                           int64_t clen, int32_t batch, int32_t M, int32_t N, int32_t K,
                                           int32_t trans_a, int32_t trans_b) {
    return matmul_host<float, float>("cleave_hip_matmul_batched_f32_host", &cleave_hip_matmul_batched_f32, a, alen, b,
                                     blen, c, clen, batch, M, N, K, trans_a, trans_b);
}

int32_t cleave_hip_matmul_bf16_host(const uint16_t* a, int64_t alen, const uint16_t* b, int64_t blen, float* c,
                                    int64_t clen, int32_t M, int32_t N, int32_t K, int32_t trans_a,
                                    int32_t trans_b) {
    Staged s("cleave_hip_matmul_bf16_host");
    const int ia = s.in(a, alen, 2), ib = s.in(b, blen, 2), ic = s.out(c, clen, 4);
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(cleave_hip_matmul_bf16(s.dev<uint16_t>(ia), alen, s.dev<uint16_t>(ib), blen,
                                           s.dev<float>(ic), clen, M, N, K, trans_a, trans_b));
}

int32_t cleave_hip_matmul_batched_bf16_host(const uint16_t* a, int64_t alen, const uint16_t* b, int64_t blen,
                                            float* c, int64_t clen, int32_t batch, int32_t M, int32_t N,
                                            int32_t K, int32_t trans_a, int32_t trans_b) {
    return matmul_host<uint16_t, float>("cleave_hip_matmul_batched_bf16_host", &cleave_hip_matmul_batched_bf16, a,
                                        alen, b, blen, c, clen, batch, M, N, K, trans_a, trans_b);
}

int32_t cleave_hip_matmul_f64_host(const double* a, int64_t alen, const double* b, int64_t blen, double* c,
                                   int64_t clen, int32_t M, int32_t N, int32_t K, int32_t trans_a, int32_t trans_b) {
    return matmul_host<double, double>("cleave_hip_matmul_f64_host", &cleave_hip_matmul_batched_f64, a, alen, b, blen,
                                       c, clen, 1, M, N, K, trans_a, trans_b);
}

int32_t cleave_hip_matmul_batched_f64_host(const double* a, int64_t alen, const double* b, int64_t blen, double* c,
                                           int64_t clen, int32_t batch, int32_t M, int32_t N, int32_t K,
                                           int32_t trans_a, int32_t trans_b) {
    return matmul_host<double, double>("cleave_hip_matmul_batched_f64_host", &cleave_hip_matmul_batched_f64, a, alen,
                                       b, blen, c, clen, batch, M, N, K, trans_a, trans_b);
}

// ---- Ring<Tensor>, Activation<Tensor>, backward maps ------------------------------

#define CH_MAP2_HOST(name, T)                                                                                \
    int32_t name##_host(const T* a, int64_t alen, const T* b, int64_t blen, T* out, int64_t outlen) {     \
        return map2_host<T>(#name "_host", &name, a, alen, b, blen, out, outlen);                          \
    }
#define CH_MAP1_HOST(name, T)                                                                                \
    int32_t name##_host(const T* a, int64_t alen, T* out, int64_t outlen) {                                \
        return map1_host<T>(#name "_host", &name, a, alen, out, outlen);                                   \
    }

CH_MAP2_HOST(cleave_hip_add_f32, float)
CH_MAP2_HOST(cleave_hip_sub_f32, float)
CH_MAP2_HOST(cleave_hip_mul_f32, float)
CH_MAP2_HOST(cleave_hip_div_f32, float)
CH_MAP1_HOST(cleave_hip_neg_f32, float)
CH_MAP1_HOST(cleave_hip_relu_f32, float)
CH_MAP1_HOST(cleave_hip_sigmoid_f32, float)
CH_MAP1_HOST(cleave_hip_tanh_f32, float)
CH_MAP2_HOST(cleave_hip_sigmoid_bwd_f32, float)
CH_MAP2_HOST(cleave_hip_tanh_bwd_f32, float)
CH_MAP2_HOST(cleave_hip_relu_bwd_f32, float)
CH_MAP2_HOST(cleave_hip_add_f64, double)
CH_MAP2_HOST(cleave_hip_sub_f64, double)
CH_MAP2_HOST(cleave_hip_mul_f64, double)
CH_MAP2_HOST(cleave_hip_div_f64, double)
CH_MAP1_HOST(cleave_hip_neg_f64, double)
CH_MAP1_HOST(cleave_hip_relu_f64, double)
CH_MAP1_HOST(cleave_hip_sigmoid_f64, double)
CH_MAP1_HOST(cleave_hip_tanh_f64, double)
CH_MAP2_HOST(cleave_hip_sigmoid_bwd_f64, double)
CH_MAP2_HOST(cleave_hip_tanh_bwd_f64, double)
CH_MAP2_HOST(cleave_hip_relu_bwd_f64, double)

int32_t cleave_hip_zero_f32_host(float* out, int64_t outlen) {
    Staged s("cleave_hip_zero_f32_host");
    const int io = s.out(out, outlen, 4);
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(cleave_hip_zero_f32(s.dev<float>(io), outlen));
}

int32_t cleave_hip_div_bwd_f32_host(const float* a, int64_t alen, const float* b, int64_t blen, const float* g,
                                    int64_t glen, float* da, int64_t dalen, float* db, int64_t dblen) {
    Staged s("cleave_hip_div_bwd_f32_host");
    const int ia = s.in(a, alen, 4), ib = s.in(b, blen, 4), ig = s.in(g, glen, 4);
    const int ida = s.out(da, dalen, 4), idb = s.out(db, dblen, 4);
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(cleave_hip_div_bwd_f32(s.dev<float>(ia), alen, s.dev<float>(ib), blen, s.dev<float>(ig), glen,
                                           s.dev<float>(ida), dalen, s.dev<float>(idb), dblen));
}

int32_t cleave_hip_sgd_update_f32_host(float* w, int64_t wlen, const float* g, int64_t glen, float lr) {
    Staged s("cleave_hip_sgd_update_f32_host");
    const int iw = s.inout(w, wlen, 4), ig = s.in(g, glen, 4);
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(cleave_hip_sgd_update_f32(s.dev<float>(iw), wlen, s.dev<float>(ig), glen, lr));
}

int32_t cleave_hip_add_row_bias_f32_host(const float* a, int64_t alen, const float* bias, int64_t blen,
                                         float* out, int64_t outlen, int32_t rows, int32_t cols) {
    Staged s("cleave_hip_add_row_bias_f32_host");
    const int ia = s.in(a, alen, 4), ib = s.in(bias, blen, 4), io = s.out(out, outlen, 4);
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(cleave_hip_add_row_bias_f32(s.dev<float>(ia), alen, s.dev<float>(ib), blen, s.dev<float>(io),
                                                outlen, rows, cols));
}

int32_t cleave_hip_sum_rows_f32_host(const float* g, int64_t glen, float* out, int64_t outlen, int32_t rows,
                                     int32_t cols) {
    Staged s("cleave_hip_sum_rows_f32_host");
    const int ig = s.in(g, glen, 4), io = s.out(out, outlen, 4);
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(cleave_hip_sum_rows_f32(s.dev<float>(ig), glen, s.dev<float>(io), outlen, rows, cols));
}

// Broadcasting maps and their reverse rule: the shapes are host arrays read
// by the device form; the operands are staged like the other maps'.
#define CH_BCAST_HOST(op, T, sfx)                                                                               \
    int32_t cleave_hip_##op##_bcast_##sfx##_host(const T* a, int64_t alen, const int32_t* ashape, int32_t arank, \
                                                const T* b, int64_t blen, const int32_t* bshape, int32_t brank,  \
                                                T* out, int64_t outlen) {                                        \
        Staged s("cleave_hip_" #op "_bcast_" #sfx "_host");                                                     \
        const int ia = s.in(a, alen, sizeof(T)), ib = s.in(b, blen, sizeof(T)), io = s.out(out, outlen, sizeof(T)); \
        int32_t st = s.stage();                                                                                  \
        if (st != CLEAVE_HIP_OK) return st;                                                                      \
        return s.finish(cleave_hip_##op##_bcast_##sfx(s.dev<T>(ia), alen, ashape, arank, s.dev<T>(ib), blen,      \
                                                      bshape, brank, s.dev<T>(io), outlen));                     \
    }
CH_BCAST_HOST(add, float, f32)
CH_BCAST_HOST(sub, float, f32)
CH_BCAST_HOST(mul, float, f32)
CH_BCAST_HOST(div, float, f32)
CH_BCAST_HOST(add, double, f64)
CH_BCAST_HOST(sub, double, f64)
CH_BCAST_HOST(mul, double, f64)
CH_BCAST_HOST(div, double, f64)
#undef CH_BCAST_HOST

int32_t cleave_hip_sum_to_shape_f32_host(const float* g, int64_t glen, const int32_t* gshape, int32_t grank,
                                         float* out, int64_t outlen, const int32_t* oshape, int32_t orank) {
    Staged s("cleave_hip_sum_to_shape_f32_host");
    const int ig = s.in(g, glen, 4), io = s.out(out, outlen, 4);
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(cleave_hip_sum_to_shape_f32(s.dev<float>(ig), glen, gshape, grank, s.dev<float>(io), outlen,
                                                oshape, orank));
}

int32_t cleave_hip_sum_to_shape_f64_host(const double* g, int64_t glen, const int32_t* gshape, int32_t grank,
                                         double* out, int64_t outlen, const int32_t* oshape, int32_t orank) {
    Staged s("cleave_hip_sum_to_shape_f64_host");
    const int ig = s.in(g, glen, 8), io = s.out(out, outlen, 8);
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(cleave_hip_sum_to_shape_f64(s.dev<double>(ig), glen, gshape, grank, s.dev<double>(io), outlen,
                                                oshape, orank));
}

int32_t cleave_hip_zero_f64_host(double* out, int64_t outlen) {
    Staged s("cleave_hip_zero_f64_host");
    const int io = s.out(out, outlen, 8);
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(cleave_hip_zero_f64(s.dev<double>(io), outlen));
}

int32_t cleave_hip_div_bwd_f64_host(const double* a, int64_t alen, const double* b, int64_t blen, const double* g,
                                    int64_t glen, double* da, int64_t dalen, double* db, int64_t dblen) {
    Staged s("cleave_hip_div_bwd_f64_host");
    const int ia = s.in(a, alen, 8), ib = s.in(b, blen, 8), ig = s.in(g, glen, 8);
    const int ida = s.out(da, dalen, 8), idb = s.out(db, dblen, 8);
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(cleave_hip_div_bwd_f64(s.dev<double>(ia), alen, s.dev<double>(ib), blen, s.dev<double>(ig), glen,
                                           s.dev<double>(ida), dalen, s.dev<double>(idb), dblen));
}

int32_t cleave_hip_sgd_update_f64_host(double* w, int64_t wlen, const double* g, int64_t glen, double lr) {
    Staged s("cleave_hip_sgd_update_f64_host");
    const int iw = s.inout(w, wlen, 8), ig = s.in(g, glen, 8);
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(cleave_hip_sgd_update_f64(s.dev<double>(iw), wlen, s.dev<double>(ig), glen, lr));
}

int32_t cleave_hip_add_row_bias_f64_host(const double* a, int64_t alen, const double* bias, int64_t blen,
                                         double* out, int64_t outlen, int32_t rows, int32_t cols) {
    Staged s("cleave_hip_add_row_bias_f64_host");
    const int ia = s.in(a, alen, 8), ib = s.in(bias, blen, 8), io = s.out(out, outlen, 8);
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(cleave_hip_add_row_bias_f64(s.dev<double>(ia), alen, s.dev<double>(ib), blen,
                                                s.dev<double>(io), outlen, rows, cols));
}

int32_t cleave_hip_sum_rows_f64_host(const double* g, int64_t glen, double* out, int64_t outlen, int32_t rows,
                                     int32_t cols) {
    Staged s("cleave_hip_sum_rows_f64_host");
    const int ig = s.in(g, glen, 8), io = s.out(out, outlen, 8);
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(cleave_hip_sum_rows_f64(s.dev<double>(ig), glen, s.dev<double>(io), outlen, rows, cols));
}

// ---- Sum / Mean / Max ----------------------------------------------------------

float cleave_hip_sum_f32_host(const float* x, int64_t len) {
    return reduce_host<float, float>("cleave_hip_sum_f32_host", &cleave_hip_sum_f32, x, len, NAN);
}

float cleave_hip_mean_f32_host(const float* x, int64_t len) {
    return reduce_host<float, float>("cleave_hip_mean_f32_host", &cleave_hip_mean_f32, x, len, NAN);
}

float cleave_hip_max_of_f32_host(const float* x, int64_t len) {
    return reduce_host<float, float>("cleave_hip_max_of_f32_host", &cleave_hip_max_of_f32, x, len, NAN);
}

int64_t cleave_hip_argmax_f32_host(const float* x, int64_t len) {
    return reduce_host<int64_t, float>("cleave_hip_argmax_f32_host", &cleave_hip_argmax_f32, x, len, -1);
}

uint64_t cleave_hip_sum_u32_u64_host(const uint32_t* x, int64_t len) {
    return reduce_host<uint64_t, uint32_t>("cleave_hip_sum_u32_u64_host", &cleave_hip_sum_u32_u64, x, len, 0);
}

int64_t cleave_hip_sum_i32_i64_host(const int32_t* x, int64_t len) {
    return reduce_host<int64_t, int32_t>("cleave_hip_sum_i32_i64_host", &cleave_hip_sum_i32_i64, x, len, 0);
}

double cleave_hip_sum_f64_host(const double* x, int64_t len) {
    return reduce_host<double, double>("cleave_hip_sum_f64_host", &cleave_hip_sum_f64, x, len, NAN);
}

double cleave_hip_mean_f64_host(const double* x, int64_t len) {
    return reduce_host<double, double>("cleave_hip_mean_f64_host", &cleave_hip_mean_f64, x, len, NAN);
}

double cleave_hip_max_of_f64_host(const double* x, int64_t len) {
    return reduce_host<double, double>("cleave_hip_max_of_f64_host", &cleave_hip_max_of_f64, x, len, NAN);
}

int64_t cleave_hip_argmax_f64_host(const double* x, int64_t len) {
    return reduce_host<int64_t, double>("cleave_hip_argmax_f64_host", &cleave_hip_argmax_f64, x, len, -1);
}

// ---- Index<Tensor> ---------------------------------------------------------------

float cleave_hip_index_f32_host(const float* t, int64_t len, const int32_t* dims, int64_t ndims,
                                const int32_t* idx, int64_t nidx) {
    ch::clear_error();
    Staged s("cleave_hip_index_f32_host");
    const int it = s.in(t, len, 4);
    if (s.stage() != CLEAVE_HIP_OK) return NAN;
    const float v = cleave_hip_index_f32(s.dev<float>(it), len, dims, ndims, idx, nidx);
    const int32_t err = cleave_hip_last_error();
    if (s.finish(CLEAVE_HIP_OK) != CLEAVE_HIP_OK || err != CLEAVE_HIP_OK) return NAN;
    return v;
}

int32_t cleave_hip_index_bwd_f32_host(float g, float* dt, int64_t len, const int32_t* dims, int64_t ndims,
                                      const int32_t* idx, int64_t nidx) {
    Staged s("cleave_hip_index_bwd_f32_host");
    const int it = s.inout(dt, len, 4);
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(cleave_hip_index_bwd_f32(g, s.dev<float>(it), len, dims, ndims, idx, nidx));
}

double cleave_hip_index_f64_host(const double* t, int64_t len, const int32_t* dims, int64_t ndims,
                                 const int32_t* idx, int64_t nidx) {
    ch::clear_error();
    Staged s("cleave_hip_index_f64_host");
    const int it = s.in(t, len, 8);
    if (s.stage() != CLEAVE_HIP_OK) return NAN;
    const double v = cleave_hip_index_f64(s.dev<double>(it), len, dims, ndims, idx, nidx);
    const int32_t err = cleave_hip_last_error();
    if (s.finish(CLEAVE_HIP_OK) != CLEAVE_HIP_OK || err != CLEAVE_HIP_OK) return NAN;
    return v;
}

int32_t cleave_hip_index_bwd_f64_host(double g, double* dt, int64_t len, const int32_t* dims, int64_t ndims,
                                      const int32_t* idx, int64_t nidx) {
    Staged s("cleave_hip_index_bwd_f64_host");
    const int it = s.inout(dt, len, 8);
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(cleave_hip_index_bwd_f64(g, s.dev<double>(it), len, dims, ndims, idx, nidx));
}

// ---- escape_count map ---------------------------------------------------------------

int32_t cleave_hip_mandelbrot_u32_host(uint32_t* out, int64_t outlen, int32_t width, int32_t height, float x0,
                                       float y0, float dx, float dy, int32_t max_iter) {
    Staged s("cleave_hip_mandelbrot_u32_host");
    const int io = s.out(out, outlen, 4);
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(cleave_hip_mandelbrot_u32(s.dev<uint32_t>(io), outlen, width, height, x0, y0, dx, dy, max_iter));
}

// ---- MLP step -----------------------------------------------------------------------

int32_t cleave_hip_mlp_step_f32_host(const float* x, int64_t xlen, const float* y, int64_t ylen, float* w1,
                                     int64_t w1len, float* w2, int64_t w2len, float* dw1, int64_t dw1len,
                                     float* dw2, int64_t dw2len, float* loss, int32_t B, int32_t D, int32_t Hd,
                                     float lr) {
    Staged s("cleave_hip_mlp_step_f32_host");
    const int ix = s.in(x, xlen, 4), iy = s.in(y, ylen, 4);
    const int iw1 = s.inout(w1, w1len, 4), iw2 = s.inout(w2, w2len, 4);
    const int idw1 = dw1 ? s.out(dw1, dw1len, 4) : -1;
    const int idw2 = dw2 ? s.out(dw2, dw2len, 4) : -1;
    const int il = loss ? s.out(loss, 1, 4) : -1;
    int32_t st = s.stage();
    if (st != CLEAVE_HIP_OK) return st;
    return s.finish(cleave_hip_mlp_step_f32(
        s.dev<float>(ix), xlen, s.dev<float>(iy), ylen, s.dev<float>(iw1), w1len, s.dev<float>(iw2), w2len,
        idw1 >= 0 ? s.dev<float>(idw1) : nullptr, dw1len, idw2 >= 0 ? s.dev<float>(idw2) : nullptr, dw2len,
        il >= 0 ? s.dev<float>(il) : nullptr, B, D, Hd, lr));
}

// ---- output-first forms for cleave's array-return identity ----------------------
// An extern whose cleave result is an array returns i64 at the C level and
// hands back its first array argument (cleave/src/mlir_lower.rs:1062-1075,
// :1123-1124).  These forms put the output array first and return its
// element count on success (like print_bytes returning its length,
// cleave-rt/src/lib.rs:114-122), or the negative status of the `_host` call
// they forward to.

#define CH_INTO_RESULT(call, outlen)                      \
    do {                                                  \
        const int32_t _st = (call);                       \
        return _st == CLEAVE_HIP_OK ? (outlen) : (int64_t)_st; \
    } while (0)

int64_t cleave_hip_matmul_f32_into(float* c, int64_t clen, const float* a, int64_t alen, const float* b,
                                   int64_t blen, int32_t M, int32_t N, int32_t K, int32_t trans_a,
                                   int32_t trans_b) {
    CH_INTO_RESULT(cleave_hip_matmul_f32_host(a, alen, b, blen, c, clen, M, N, K, trans_a, trans_b), clen);
}

int64_t cleave_hip_matmul_f64_into(double* c, int64_t clen, const double* a, int64_t alen, const double* b,
                                   int64_t blen, int32_t M, int32_t N, int32_t K, int32_t trans_a,
                                   int32_t trans_b) {
    CH_INTO_RESULT(cleave_hip_matmul_f64_host(a, alen, b, blen, c, clen, M, N, K, trans_a, trans_b), clen);
}

#define CH_MAP2_INTO(op, T, sfx)                                                                          \
    int64_t cleave_hip_##op##_##sfx##_into(T* out, int64_t outlen, const T* a, int64_t alen, const T* b, \
                                           int64_t blen) {                                              \
        CH_INTO_RESULT(cleave_hip_##op##_##sfx##_host(a, alen, b, blen, out, outlen), outlen);         \
    }
#define CH_MAP1_INTO(op, T, sfx)                                                                          \
    int64_t cleave_hip_##op##_##sfx##_into(T* out, int64_t outlen, const T* x, int64_t xlen) {          \
        CH_INTO_RESULT(cleave_hip_##op##_##sfx##_host(x, xlen, out, outlen), outlen);                  \
    }
#define CH_INTO_ENTRIES(T, sfx) \
    CH_MAP2_INTO(add, T, sfx)   \
    CH_MAP2_INTO(sub, T, sfx)   \
    CH_MAP2_INTO(mul, T, sfx)   \
    CH_MAP2_INTO(div, T, sfx)   \
    CH_MAP1_INTO(neg, T, sfx)   \
    CH_MAP1_INTO(relu, T, sfx)  \
    CH_MAP1_INTO(sigmoid, T, sfx) \
    CH_MAP1_INTO(tanh, T, sfx)  \
    CH_MAP2_INTO(sigmoid_bwd, T, sfx) \
    CH_MAP2_INTO(tanh_bwd, T, sfx) \
    CH_MAP2_INTO(relu_bwd, T, sfx)

CH_INTO_ENTRIES(float, f32)
CH_INTO_ENTRIES(double, f64)

// Escape counts as cleave's i32 (escape_count returns i32,
// examples/mandelbrot.cleave:14): counts are at most max_iter < 2^31, so the
// u32 counts of the same grid have the same bits.
int64_t cleave_hip_escape_grid_i32(int32_t* out, int64_t outlen, int32_t width, int32_t height, float x0,
                                   float y0, float dx, float dy, int32_t max_iter) {
    CH_INTO_RESULT(cleave_hip_mandelbrot_u32_host(reinterpret_cast<uint32_t*>(out), outlen, width, height, x0, y0,
                                                  dx, dy, max_iter),
                   outlen);
}

}  // extern "C"
