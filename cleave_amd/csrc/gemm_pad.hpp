// gemm_pad.hpp -- ragged GEMM shapes through the aligned kernels.
//
// The fast kernels want M and N multiples of their block tile, K a multiple
// of their k-tile and 16-byte aligned rows.  A large product that misses
// those runs on zero-padded copies instead: each operand that does not
// already fit is copied, in the caller's layout, into a buffer whose extents
// are rounded up (K to 64 or 2048, M and N to 128 or 256) with zeros past the valid
// region; the product is computed on the padded shape; and, when M or N was
// rounded up, the valid M x N corner of the padded C is copied out.
//
// The zeros change no valid entry: a padded k adds 0 * 0 = +0 to a sum that
// starts at +0 (x + (+0) == x for every x but -0, and a sum started at +0
// never is -0), and padded rows or columns only feed entries of C that are
// not copied out.
#pragma once

#include "common.hpp"

namespace ch {

struct PadPlan {
    bool ok;         // the padded extents fit int and at most triple the work
    int M, N, K;     // valid shape
    int Mp, Np, Kp;  // padded shape
    bool copy_a, copy_b, crop_c;
    size_t bytes_a, bytes_b, bytes_c;  // scratch bytes of each padded operand (0: used in place)
};

inline int64_t pad_up(int x, int q) { return ((int64_t)x + q - 1) / q * q; }

// Measured throughput of the aligned kernels, as a fraction of peak; they
// price the two paddings.
struct PadModel {
    double eff256;    // 256 x 256 tiles, one workgroup per CU
    double eff128;    // 128 x 128 tiles
    bool rounds128;   // price 128 x 128 tiles by rounds too
    double min256;    // fewest 256 x 256 tiles the kernels take, per CU
};

// Padded shape: K to a multiple of 64 (of 2048 from 16384); M and N to multiples of 128, or of 256
// when that gives the 256 x 256 kernels enough tiles (model.min256 per CU)
// and is estimated faster.
// Time ~ padded area / efficiency, and, where a CU holds one workgroup, / the
// fill of the rounds of tiles (the last round may leave CUs idle; where a CU
// holds several, a lone workgroup runs faster and this is not counted).  An
// operand whose stored extents and alignment already match is used in place.
inline PadPlan pad_plan(int M, int N, int K, int batch, bool ta, bool tb, const void* a, const void* b,
                        int esz, int cus, const PadModel& model) {
    PadPlan p{};
    p.M = M, p.N = N, p.K = K;
    // a long K goes to a multiple of 2048 (at most 1/8 more), so that the
    // padded product can still be cut into K slices of equal depth
    const int64_t kp = pad_up(K, K >= 16384 ? 2048 : 64);
    const int64_t m2 = pad_up(M, 256), n2 = pad_up(N, 256), m1 = pad_up(M, 128), n1 = pad_up(N, 128);
    auto cost = [](double area, int64_t tiles, int64_t per_round, double eff) {
        const int64_t rounds = (tiles + per_round - 1) / per_round;
        return area / (eff * ((double)tiles / (double)(rounds * per_round)));
    };
    const int64_t t2 = (m2 / 256) * (n2 / 256) * batch, t1 = (m1 / 128) * (n1 / 128) * batch;
    const int c = cus > 0 ? cus : 1;
    const double c128 = model.rounds128 ? cost((double)m1 * n1, t1, c, model.eff128)
                                        : (double)m1 * n1 / model.eff128;
    const bool use256 = (double)t2 >= model.min256 * c && cost((double)m2 * n2, t2, c, model.eff256) < c128;
    const int64_t mp = use256 ? m2 : m1, np = use256 ? n2 : n1;
    // Padding at most triples the work: smaller products (16^3 padded to
    // 128 x 128 x 64 is 256x) stay on the general kernel, which computes
    // whole tiles too but moves no padded copies.
    p.ok = mp <= INT32_MAX && np <= INT32_MAX && kp <= INT32_MAX &&
           (double)mp * np * kp <= 3.0 * M * N * K;
    if (!p.ok) return p;
    p.Mp = (int)mp, p.Np = (int)np, p.Kp = (int)kp;
    const bool a_al = ((uintptr_t)a & 15) == 0 && ((int64_t)(ta ? M : K) * esz) % 16 == 0;
    const bool b_al = ((uintptr_t)b & 15) == 0 && ((int64_t)(tb ? K : N) * esz) % 16 == 0;
    p.copy_a = !(p.Mp == M && p.Kp == K && a_al);
    p.copy_b = !(p.Np == N && p.Kp == K && b_al);
    p.crop_c = !(p.Mp == M && p.Np == N);
    // round each buffer to 256 bytes so the next one stays aligned
    auto r256 = [](size_t x) { return (x + 255) / 256 * 256; };
    p.bytes_a = p.copy_a ? r256((size_t)batch * p.Mp * p.Kp * esz) : 0;
    p.bytes_b = p.copy_b ? r256((size_t)batch * p.Kp * p.Np * esz) : 0;
    p.bytes_c = p.crop_c ? r256((size_t)batch * p.Mp * p.Np * sizeof(float)) : 0;
    return p;
}

// One padded copy: dst (batch matrices of rows_p x cols_p, row pitch cols_p)
// = src (batch matrices of rows x cols, row pitch cols), zeros past row
// `rows` and column `cols`; total_rows = batch * rows_p (0: nothing to copy).
// cols_p % 8 == 0 and dst 16-byte aligned.  vec_src: src rows are 16-byte
// aligned, so whole chunks load as vectors.
template <typename T>
struct PadCopy {
    const T* src;
    T* dst;
    int rows, cols, rows_p, cols_p;
    int64_t total_rows;
    bool vec_src;
    __host__ __device__ int64_t chunks() const { return total_rows * (cols_p / 8); }
};

// Destination row rr of one padded copy, each thread 8 consecutive elements.
template <typename T>
__device__ __forceinline__ void pad_copy_row(const PadCopy<T>& j, int64_t rr) {
    typedef T v8 __attribute__((ext_vector_type(8), aligned(16)));  // 16-byte alignment is all that is checked
    const int64_t bt = rr / j.rows_p;
    const int r = (int)(rr - bt * j.rows_p);
    const T* s = j.src + (bt * j.rows + r) * (int64_t)j.cols;
    T* d = j.dst + rr * (int64_t)j.cols_p;
    for (int c0 = threadIdx.x * 8; c0 < j.cols_p; c0 += 256 * 8) {
        v8 v;
        if (r < j.rows && c0 + 8 <= j.cols) {
            if (j.vec_src) {
                v = *reinterpret_cast<const v8*>(s + c0);
            } else {
#pragma unroll
                for (int t = 0; t < 8; ++t) v[t] = s[c0 + t];
            }
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) v[t] = (r < j.rows && c0 + t < j.cols) ? s[c0 + t] : (T)0;
        }
        *reinterpret_cast<v8*>(d + c0) = v;
    }
}

// Both operands' padded copies in one launch: destination rows 0 ..
// a.total_rows - 1 are a's, the next b.total_rows are b's.  One workgroup
// per destination row, grid-strided.
template <typename T>
__global__ __launch_bounds__(256) void pad_copy_kernel(PadCopy<T> a, PadCopy<T> b) {
    const int64_t total = a.total_rows + b.total_rows;
    for (int64_t rr = blockIdx.x; rr < total; rr += gridDim.x) {
        if (rr < a.total_rows) pad_copy_row(a, rr);
        else pad_copy_row(b, rr - a.total_rows);
    }
}

// 8 consecutive elements from s, in the widest loads its alignment allows
// (a source row that is not whole 16-byte chunks starts 8, 4 or 2 bytes
// off in every other row).
template <typename T>
__device__ __forceinline__ void load8(const T* s, T (&v)[8]) {
    constexpr int ES = (int)sizeof(T);
    const uintptr_t al = (uintptr_t)s & 15;
    if (al == 0) {
        typedef uint32_t w4 __attribute__((ext_vector_type(4)));
        w4 w[ES / 2];
#pragma unroll
        for (int i = 0; i < ES / 2; ++i) w[i] = reinterpret_cast<const w4*>(s)[i];
        __builtin_memcpy(v, w, sizeof(v));
    } else if ((al & 7) == 0) {
        uint64_t w[ES];
#pragma unroll
        for (int i = 0; i < ES; ++i) w[i] = reinterpret_cast<const uint64_t*>(s)[i];
        __builtin_memcpy(v, w, sizeof(v));
    } else if ((al & 3) == 0) {
        uint32_t w[2 * ES];
#pragma unroll
        for (int i = 0; i < 2 * ES; ++i) w[i] = reinterpret_cast<const uint32_t*>(s)[i];
        __builtin_memcpy(v, w, sizeof(v));
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) v[t] = s[t];
    }
}

// Destination chunk q (8 elements; row q / (cols_p / 8)) of one padded copy.
template <typename T>
__device__ __forceinline__ void pad_copy_chunk(const PadCopy<T>& j, int64_t q) {
    const int cpr = j.cols_p / 8;
    int64_t rr, bt;
    if (q < (1ll << 32)) {  // 32-bit divisions (a 64-bit one costs ~10x the instructions)
        const uint32_t r32 = (uint32_t)q / (uint32_t)cpr;
        rr = r32;
        bt = r32 / (uint32_t)j.rows_p;
    } else {
        rr = q / cpr;
        bt = rr / j.rows_p;
    }
    const int c0 = (int)(q - rr * cpr) * 8;
    const int r = (int)(rr - bt * j.rows_p);
    const T* s = j.src + (bt * j.rows + r) * (int64_t)j.cols + c0;
    T v[8];
    if (r < j.rows && c0 + 8 <= j.cols) {
        load8(s, v);
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) v[t] = (r < j.rows && c0 + t < j.cols) ? s[t] : (T)0;
    }
    typedef uint32_t w4 __attribute__((ext_vector_type(4)));
    w4 w[sizeof(T) / 2];
    __builtin_memcpy(w, v, sizeof(v));
    w4* d = reinterpret_cast<w4*>(j.dst + rr * (int64_t)j.cols_p + c0);
#pragma unroll
    for (int i = 0; i < (int)sizeof(T) / 2; ++i) d[i] = w[i];
}

// The same copies, one thread per 8-element destination chunk (grid-
// strided): chunks 0 .. a.chunks() - 1 are a's, the next b.chunks() are b's.
template <typename T>
__global__ __launch_bounds__(256) void pad_copy_chunks_kernel(PadCopy<T> a, PadCopy<T> b) {
    const int64_t na = a.chunks(), total = na + b.chunks();
    for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < total; q += (int64_t)gridDim.x * 256) {
        if (q < na) pad_copy_chunk(a, q);
        else pad_copy_chunk(b, q - na);
    }
}

// dst (batch x M x N, pitch N) = the top-left M x N of each src matrix
// (batch x Mp x Np, pitch Np); Np % 4 == 0 and src 16-byte aligned (for
// T = float).
template <typename T>
__global__ __launch_bounds__(256) void crop_kernel(const T* __restrict__ src, T* __restrict__ dst, int M, int N,
                                                   int Mp, int Np, int64_t total_rows, bool vec_dst) {
    typedef T v4 __attribute__((ext_vector_type(4)));
    for (int64_t rr = blockIdx.x; rr < total_rows; rr += gridDim.x) {
        const int64_t bt = rr / M;
        const int r = (int)(rr - bt * M);
        const T* s = src + (bt * Mp + r) * (int64_t)Np;
        T* d = dst + rr * (int64_t)N;
        for (int c0 = threadIdx.x * 4; c0 < N; c0 += 256 * 4) {
            const v4 v = *reinterpret_cast<const v4*>(s + c0);
            if (vec_dst && c0 + 4 <= N) {
                *reinterpret_cast<v4*>(d + c0) = v;
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    if (c0 + t < N) d[c0 + t] = v[t];
            }
        }
    }
}

// Grid of the row-strided copy kernels: one workgroup per row, at most 64
// per CU.
inline unsigned pad_grid(int64_t total_rows, int cus) {
    const int64_t cap = (int64_t)(cus > 0 ? cus : 1) * 64;
    return (unsigned)(total_rows < cap ? total_rows : cap);
}

// Launches the padded copies a and b (either may be empty).  A workgroup per
// destination row (pad_copy_kernel) unless a copied operand has rows under
// 512 elements or fewer rows than CUs: then a thread per chunk
// (pad_copy_chunks_kernel, at most 8 workgroups per CU, full occupancy),
// which keeps every thread busy (a row of 300 bf16 leaves 218 of 256
// threads idle) and every CU fed.  Same box, copy kernel alone: 64 x 700 x
// 900 x 300 (rows of 300 and 900 bf16) 37.5 -> 30.3 us (the product 94.7 ->
// 87.8), 200 rows of 12300 10.2 -> 8.4.  As chunks, more rows of 1000 or
// more elements copied slower than a row per workgroup: f32 6000^3 118
// against 104 us, bf16 1001 x 32768 (K rounded to 2048) 24.2 against 21.8,
// 1500^3 10.4 against 9.7.  (One kernel taking either mapping per operand
// made the row path slower still, 27.9 against 21.8 at 1001 x 32768.)
template <typename T>
int32_t launch_pad_copies(const PadCopy<T>& a, const PadCopy<T>& b, int cus) {
    const int64_t rows = a.total_rows + b.total_rows;
    if (rows == 0) return CLEAVE_HIP_OK;
    auto short_rows = [cus](const PadCopy<T>& j) {
        return j.total_rows > 0 && (j.cols_p < 512 || j.total_rows < cus);
    };
    if (short_rows(a) || short_rows(b)) {
        const int64_t cap = (int64_t)(cus > 0 ? cus : 1) * 8, need = (a.chunks() + b.chunks() + 255) / 256;
        pad_copy_chunks_kernel<T><<<(unsigned)(need < cap ? need : cap), 256, 0, stream()>>>(a, b);
        return check_hip(hipGetLastError(), "pad_copy_chunks_kernel");
    }
    pad_copy_kernel<T><<<pad_grid(rows, cus), 256, 0, stream()>>>(a, b);
    return check_hip(hipGetLastError(), "pad_copy_kernel");
}

// Runs `gemm(a, b, c, Mp, Np, Kp)` (which must take the padded shape with
// 16-byte aligned rows) on padded copies as `p` plans them, then crops C.
// Returns false, launching nothing, when the scratch buffer cannot be had.
template <typename T, typename Gemm>
bool run_padded(const PadPlan& p, const T* a, const T* b, float* c, int batch, bool ta, bool tb, Gemm gemm,
                int32_t* status) {
    constexpr int kSlot = 7;
    if (!p.ok) return false;
    const size_t total = p.bytes_a + p.bytes_b + p.bytes_c;
    char* base = (char*)scratch_try(kSlot, total ? total : 256);
    if (!base) return false;
    const int cus = num_cus();
    const T* pa = a;
    const T* pb = b;
    float* pc = c;
    PadCopy<T> ja{}, jb{};
    if (p.copy_a) {
        T* d = (T*)base;
        const int rows = ta ? p.K : p.M, cols = ta ? p.M : p.K;
        const int rows_p = ta ? p.Kp : p.Mp, cols_p = ta ? p.Mp : p.Kp;
        const bool vec = ((uintptr_t)a & 15) == 0 && ((int64_t)cols * sizeof(T)) % 16 == 0;
        ja = PadCopy<T>{a, d, rows, cols, rows_p, cols_p, (int64_t)batch * rows_p, vec};
        pa = d;
    }
    if (p.copy_b) {
        T* d = (T*)(base + p.bytes_a);
        const int rows = tb ? p.N : p.K, cols = tb ? p.K : p.N;
        const int rows_p = tb ? p.Np : p.Kp, cols_p = tb ? p.Kp : p.Np;
        const bool vec = ((uintptr_t)b & 15) == 0 && ((int64_t)cols * sizeof(T)) % 16 == 0;
        jb = PadCopy<T>{b, d, rows, cols, rows_p, cols_p, (int64_t)batch * rows_p, vec};
        pb = d;
    }
    int32_t st = launch_pad_copies(ja, jb, cus);
    if (p.crop_c) pc = (float*)(base + p.bytes_a + p.bytes_b);
    if (st == CLEAVE_HIP_OK) st = gemm(pa, pb, pc, p.Mp, p.Np, p.Kp);
    if (st == CLEAVE_HIP_OK && p.crop_c) {
        const int64_t tr = (int64_t)batch * p.M;
        const bool vec = ((uintptr_t)c & 15) == 0 && p.N % 4 == 0;
        crop_kernel<float><<<pad_grid(tr, cus), 256, 0, stream()>>>(pc, c, p.M, p.N, p.Mp, p.Np, tr, vec);
        st = check_hip(hipGetLastError(), "crop_kernel");
    }
    *status = st;
    return true;
}

// Ragged products whose only obstacle to the guarded-edge kernels is
// alignment: an operand row that is not a whole number of 16-byte chunks (a
// contiguous extent not a multiple of Q = 16 / element size) or a base that
// is not 16-byte aligned.  Each such operand is copied, in the caller's
// layout, with its contiguous extent rounded up to a multiple of 8 (zeros
// past it); when K is not a multiple of Q, K is rounded up to Kq in both
// operands (zero k-columns or k-rows), so that no 16-byte chunk of a
// k-contiguous operand straddles the kernels' K (or further, kround below).  The guarded-edge kernels
// then run on the copies with C written in place: C is neither padded nor
// cropped, and only the operands move once more.  The zeros change no entry,
// as for the padded copies above.
struct AlignPlan {
    bool ok;            // an operand needs its copy, and the copies fit the edge kernels
    int Kq;             // K rounded up to Q
    bool copy_a, copy_b;
    int64_t lda, ldb;   // pitches of the operands the kernels read, in elements
    int64_t sA, sB;     // their per-product strides
    int64_t rows_a, rows_b;  // rows of each copy (its stored layout)
    size_t bytes_a, bytes_b;  // scratch bytes of each copy (0: used in place)
};

// kround: K is rounded up to a multiple of it (at least Q), e.g. so that K
// slices divide it.
inline AlignPlan align_plan(int M, int N, int K, int batch, bool ta, bool tb, const void* a, const void* b,
                            int esz, int kround = 1) {
    AlignPlan p{};
    const int q = 16 / esz;
    const int64_t kq = pad_up(K, kround > q ? kround : q);
    const int64_t pa = ta ? M : K, pb = tb ? K : N;  // stored pitches
    const bool a_al = ((uintptr_t)a & 15) == 0 && pa % q == 0;
    const bool b_al = ((uintptr_t)b & 15) == 0 && pb % q == 0;
    p.copy_a = !a_al || kq != K;
    p.copy_b = !b_al || kq != K;
    if ((!p.copy_a && !p.copy_b) || kq > INT32_MAX) return p;
    p.Kq = (int)kq;
    p.rows_a = ta ? kq : M;
    p.rows_b = tb ? N : kq;
    p.lda = p.copy_a ? pad_up((int)(ta ? M : kq), 8) : pa;
    p.ldb = p.copy_b ? pad_up((int)(tb ? kq : N), 8) : pb;
    p.sA = p.rows_a * p.lda;
    p.sB = p.rows_b * p.ldb;
    // the edge kernels address each product's operand with 32-bit byte offsets
    p.ok = p.sA * esz < (1ll << 31) && p.sB * esz < (1ll << 31);
    auto r256 = [](size_t x) { return (x + 255) / 256 * 256; };
    p.bytes_a = p.copy_a ? r256((size_t)batch * p.sA * esz) : 0;
    p.bytes_b = p.copy_b ? r256((size_t)batch * p.sB * esz) : 0;
    return p;
}

// Copies the operands `p` names and runs `gemm(pa, pb, lda, ldb, sA, sB, Kq,
// status)`, which launches a guarded-edge kernel on M x N x Kq with C in
// place and returns whether it did.  Returns false when nothing was launched
// for the product (plan not ok, no scratch, or `gemm` declined after the
// copies: the caller then takes another route on the original operands).
template <typename T, typename Gemm>
bool run_aligned(const AlignPlan& p, const T* a, const T* b, int M, int N, int K, int batch, bool ta, bool tb,
                 Gemm gemm, int32_t* status) {
    constexpr int kSlot = 7;
    if (!p.ok) return false;
    char* base = (char*)scratch_try(kSlot, p.bytes_a + p.bytes_b);
    if (!base) return false;
    const T* pa = a;
    const T* pb = b;
    PadCopy<T> ja{}, jb{};
    if (p.copy_a) {
        T* d = (T*)base;
        const int rows = ta ? K : M, cols = ta ? M : K;
        const bool vec = ((uintptr_t)a & 15) == 0 && ((int64_t)cols * sizeof(T)) % 16 == 0;
        ja = PadCopy<T>{a, d, rows, cols, (int)p.rows_a, (int)p.lda, (int64_t)batch * p.rows_a, vec};
        pa = d;
    }
    if (p.copy_b) {
        T* d = (T*)(base + p.bytes_a);
        const int rows = tb ? N : K, cols = tb ? K : N;
        const bool vec = ((uintptr_t)b & 15) == 0 && ((int64_t)cols * sizeof(T)) % 16 == 0;
        jb = PadCopy<T>{b, d, rows, cols, (int)p.rows_b, (int)p.ldb, (int64_t)batch * p.rows_b, vec};
        pb = d;
    }
    int32_t st = launch_pad_copies(ja, jb, num_cus());
    if (st != CLEAVE_HIP_OK) {
        *status = st;
        return true;
    }
    return gemm(pa, pb, p.lda, p.ldb, p.sA, p.sB, p.Kq, status);
}

}  // namespace ch
