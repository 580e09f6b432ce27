// mandelbrot.hip -- escape-time map of examples/mandelbrot.cleave:14-26 in f32.
//
// escape_count(c): z = 0; for n in 0..max_iter { z = z*z + c;
// if |z|^2 > 4 { return n } }; return max_iter.  Complex mul/add and
// magnitude_sq follow stdlib/complex/complex.cleave:25-32 and :54:
//   re = zr*zr - zi*zi;  im = zr*zi + zi*zr;  z = (re + cr, im + ci);
//   |z|^2 = zr*zr + zi*zi.
// The reference latches the first escape and keeps iterating; this kernel
// does the same inside unrolled blocks of iterations and stops a wave once all
// of its lanes have escaped, which returns the same n.
//
// Bit-exactness: the library is compiled with -ffp-contract=off, so no mul+add
// is fused behind the code's back.  Three rewrites are exact and save work:
//   * the zr*zr and zi*zi of the |z|^2 test are the same rounded products the
//     next step's re needs;
//   * zr*zi + zi*zr == p + p with p = fl(zr*zi) (the same rounded product
//     added to itself), and p + p == 2p exactly;
//   * so im + ci = fl(fl(2p) + ci) = fl(2p + ci) = fma(2, p, ci): 2p is exact
//     in binary floating point (subnormals included), so the fma's single
//     rounding is the two-step sum's second one.  Where 2p overflows, |ci|
//     is far below half an ulp of FLT_MAX and both forms give the same inf.
//
// Mapping: one wave per 8 x 8 pixel block (neighbouring pixels have similar
// iteration counts, so waves diverge less than with 64 x 1 strips); a
// 256-thread workgroup covers 16 x 16 pixels.
#include "common.hpp"

namespace {

// Iterations per block of the unrolled loop.  Inside a block every lane
// iterates, and the lanes still inside the radius after each iteration are
// kept as a wave mask (the escape compare writes a mask, a scalar AND narrows
// it).  A lane whose first escape is iteration n gets count n, and one that
// never escapes gets max_iter (the reference's `escaped`/`count` latch,
// examples/mandelbrot.cleave:14-26).  Per iteration: 7 arithmetic ops and a
// compare on the VALU, one scalar AND -- no branch, no count update.  Only in
// a block where some lane escapes are the escaping lanes' counts formed, from
// the block's masks: n = the block's first iteration + the number of the
// block's masks that still hold the lane.  The wave leaves once no lane is
// alive.  With 9 VALU per iteration (before 2p + ci became one fma), at
// 16384^2 x 1000 blocks of 8 measured 6.10 ms, blocks of 16 6.28 ms, and a
// count added every iteration 6.69 ms; on another box blocks of 4, 6, 8 and
// 12 measured 6.40, 6.19, 6.12 and 6.21 ms.  The fma form: 5.61 ms.
constexpr int kBlockIters = 8;

// count + 1 in the lanes set in `lanes` (a wave lane mask), as one
// v_addc_co_u32 whose carry-in is that mask.  The carry-out goes to a scratch
// SGPR pair of its own, so consecutive adds do not serialise on VCC.
__device__ __forceinline__ uint32_t count_lanes(uint32_t count, uint64_t lanes) {
    uint32_t r;
    uint64_t carry_out;
    asm("v_addc_co_u32_e64 %0, %1, 0, %2, %3" : "=v"(r), "=s"(carry_out) : "v"(count), "s"(lanes));
    (void)carry_out;
    return r;
}

// if_set in the lanes set in `lanes`, if_clear in the others.
__device__ __forceinline__ uint32_t select_lanes(uint64_t lanes, uint32_t if_set, uint32_t if_clear) {
    uint32_t r;
    asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(if_clear), "v"(if_set), "s"(lanes));
    return r;
}

__global__ __launch_bounds__(256) void mandelbrot_kernel(uint32_t* __restrict__ out, int width,
                                                         int height, float x0, float y0, float dx,
                                                         float dy, int max_iter) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = blockIdx.x * 16 + (wave & 1) * 8 + (lane & 7);
    const int row = blockIdx.y * 16 + (wave >> 1) * 8 + (lane >> 3);
    const bool inside = col < width && row < height;
    const float cr = x0 + (float)col * dx;
    const float ci = y0 + (float)row * dy;
    float zr = 0.0f, zi = 0.0f, zr2 = 0.0f, zi2 = 0.0f;
    uint32_t count = 0;  // final in the lanes that have escaped
    uint64_t alive = __builtin_amdgcn_ballot_w64(inside);
    int n = 0;
    // Whole blocks: lanes past their escape keep iterating (z may overflow to
    // inf/NaN, which no longer matters: the count is latched).
    for (; n + kBlockIters <= max_iter; n += kBlockIters) {
        const uint64_t before = alive;
        uint64_t after[kBlockIters];  // alive after each iteration of the block
#pragma unroll
        for (int u = 0; u < kBlockIters; ++u) {
            const float p = zr * zi;
            const float re = zr2 - zi2;
            zr = re + cr;
            zi = __builtin_fmaf(2.0f, p, ci);  // (p + p) + ci, exactly
            zr2 = zr * zr;
            zi2 = zi * zi;
            alive &= __builtin_amdgcn_ballot_w64(!(zr2 + zi2 > 4.0f));
            after[u] = alive;
        }
        const uint64_t escaped = before & ~alive;
        if (escaped != 0) {  // wave-uniform
            uint32_t c = (uint32_t)n;
#pragma unroll
            for (int u = 0; u < kBlockIters; ++u) c = count_lanes(c, after[u]);
            count = select_lanes(escaped, c, count);
        }
        if (alive == 0) break;
    }
    // Remaining max_iter % kBlockIters iterations (only when some lane survived).
    for (int m = n; m < max_iter && alive != 0; ++m) {
        const uint64_t before = alive;
        const float p = zr * zi;
        const float re = zr2 - zi2;
        zr = re + cr;
        zi = __builtin_fmaf(2.0f, p, ci);
        zr2 = zr * zr;
        zi2 = zi * zi;
        alive &= __builtin_amdgcn_ballot_w64(!(zr2 + zi2 > 4.0f));
        count = select_lanes(before & ~alive, (uint32_t)m, count);
    }
    count = select_lanes(alive, (uint32_t)max_iter, count);  // never escaped
    if (inside) out[(int64_t)row * width + col] = count;
}

}  // namespace

extern "C" int32_t cleave_hip_mandelbrot_u32(uint32_t* out, int64_t outlen, int32_t width,
                                             int32_t height, float x0, float y0, float dx,
                                             float dy, int32_t max_iter) {
    CH_REQUIRE(width > 0 && height > 0, "cleave_hip_mandelbrot_u32: width/height must be positive");
    CH_REQUIRE(max_iter >= 0, "cleave_hip_mandelbrot_u32: max_iter must be >= 0");
    CH_REQUIRE(outlen == (int64_t)width * height, "cleave_hip_mandelbrot_u32: outlen %lld != width*height %lld",
               (long long)outlen, (long long)width * height);
    CH_REQUIRE(out != nullptr, "cleave_hip_mandelbrot_u32: null buffer");
    CH_INIT_OR_RETURN();
    CH_DEVICE("cleave_hip_mandelbrot_u32", out, outlen * 4);
    dim3 grid((unsigned)((width + 15) / 16), (unsigned)((height + 15) / 16));
    CH_REQUIRE(grid.y <= 65535u, "cleave_hip_mandelbrot_u32: height %d too large", height);
    mandelbrot_kernel<<<grid, 256, 0, ch::stream()>>>(out, width, height, x0, y0, dx, dy, max_iter);
    CH_LAUNCHED("mandelbrot_kernel");
    return CLEAVE_HIP_OK;
}
