// mlp.hip -- one SGD step of a 2-layer sigmoid MLP with MSE loss, in the style
// of examples/xor_tensor.cleave:38-92 (config: batch mean, no biases).
//
// Forward ops are the stdlib bodies (matmul stdlib/linalg/matrix.cleave:27-61,
// sigmoid stdlib/nn/nn.cleave:87-93, mean stdlib/nn/nn.cleave:135-138); the
// backward applies the reference's derivative rules in reverse mode:
//   MatMul product rule (stdlib/linalg/matrix.cleave:24) -> dA = dC B^T, dB = A^T dC
//   d(e*e) = de*e + e*de (stdlib/num/num.cleave:125)      -> dL/dyhat = (e+e)/B
//   sigmoid via quotient + exp rules (num.cleave:132-134, :222) -> s(1-s)
//
// Kernel sequence on the library stream (device-resident, no host sync):
//   1. H = X W1                         gemm_f32 NN   (M=B, N=Hd, K=D)
//   2. H = sigmoid(H)                   map, in place
//   3. row pass: z2 = H W2, yhat, e, sq = e*e, d2 = (e+e)/B * yhat(1-yhat)
//   4. loss = sum(sq) / B               2-stage reduction
//   5. column pass over H: dW2 partials += h*d2[m]; H <- d1 = (d2[m] W2[n]) h(1-h)
//   6. dW2 = sum of partials; W2 -= lr dW2
//   7. dW1 partials = X^T d1            gemm_f32 TN, split-K slices
//   8. dW1 = sum of slices; W1 -= lr dW1
#include "common.hpp"
#include "gemm_f32_pingpong.hpp"

namespace ch {
int32_t gemm_f32_device(const float* a, const float* b, float* c, int M, int N, int K, int ta,
                        int tb, int splits);
}

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float sigmoidf_ref(float x) { return 1.0f / (1.0f + expf(-x)); }

__global__ __launch_bounds__(kThreads) void sigmoid_inplace_kernel(float* __restrict__ h, int64_t n) {
    const int64_t nv = n / 4;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < nv; i += (int64_t)gridDim.x * kThreads) {
        float4 v = reinterpret_cast<float4*>(h)[i];
        v.x = sigmoidf_ref(v.x);
        v.y = sigmoidf_ref(v.y);
        v.z = sigmoidf_ref(v.z);
        v.w = sigmoidf_ref(v.w);
        reinterpret_cast<float4*>(h)[i] = v;
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) h[nv * 4 + threadIdx.x] = sigmoidf_ref(h[nv * 4 + threadIdx.x]);
}

// H[row,:] . W2 by one wave (every lane returns the sum).
__device__ __forceinline__ float row_dot(const float* __restrict__ h, const float* __restrict__ W2, int Hd) {
    const int lane = threadIdx.x & 63;
    float acc = 0.0f;
    if ((Hd & 3) == 0) {
        for (int c = lane * 4; c < Hd; c += 256) {
            float4 a = *reinterpret_cast<const float4*>(h + c);
            float4 w = *reinterpret_cast<const float4*>(W2 + c);
            acc += a.x * w.x + a.y * w.y + a.z * w.z + a.w * w.w;
        }
    } else {
        for (int c = lane; c < Hd; c += 64) acc += h[c] * W2[c];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    return acc;
}

// One wave per row: z2 = H[m,:] . W2, then the per-row loss pieces.
__global__ __launch_bounds__(kThreads) void row_pass_kernel(const float* __restrict__ H,
                                                            const float* __restrict__ W2,
                                                            const float* __restrict__ y, int B,
                                                            int Hd, float* __restrict__ sq,
                                                            float* __restrict__ d2) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (row >= B) return;
    const float acc = row_dot(H + (int64_t)row * Hd, W2, Hd);
    if (lane == 0) {
        float yh = sigmoidf_ref(acc);
        float e = yh - y[row];
        sq[row] = e * e;
        float gy = (e + e) / (float)B;
        d2[row] = gy * yh * (1.0f - yh);
    }
}

// Fused path, after the MODE-1 GEMM: z2[row] = sum of the P partials of
// H[row] . W2 (in order; loads eight at a time), then the same per-row loss
// pieces as row_pass_kernel.  Each block also reduces its rows' squared
// errors into sqpart[block] (wave shuffles, then the 4 wave sums in order),
// which loss_kernel adds up.
constexpr int kPartUnroll = 8;

// The P partials of row `row` of H W2, added in order (eight loads in flight).
__device__ __forceinline__ float sum_row_partials(const float* __restrict__ zpart, int P, int B, int row) {
    float z = zpart[row];
    int p = 1;
    for (; p + kPartUnroll <= P; p += kPartUnroll) {
        float v[kPartUnroll];
#pragma unroll
        for (int u = 0; u < kPartUnroll; ++u) v[u] = zpart[(int64_t)(p + u) * B + row];
#pragma unroll
        for (int u = 0; u < kPartUnroll; ++u) z += v[u];
    }
    for (; p < P; ++p) z += zpart[(int64_t)p * B + row];
    return z;
}

__global__ __launch_bounds__(kThreads) void row_finish_kernel(const float* __restrict__ zpart, int P,
                                                              const float* __restrict__ y, int B,
                                                              float* __restrict__ sqpart,
                                                              float* __restrict__ d2) {
    __shared__ float wsum[kThreads / 64];
    const int row = blockIdx.x * kThreads + threadIdx.x;
    float sq = 0.0f;
    if (row < B) {
        const float z = sum_row_partials(zpart, P, B, row);
        const float yh = sigmoidf_ref(z);
        const float e = yh - y[row];
        sq = e * e;
        const float gy = (e + e) / (float)B;
        d2[row] = gy * yh * (1.0f - yh);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sq += __shfl_xor(sq, o);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = sq;
    __syncthreads();
    if (threadIdx.x == 0) {
        float r = wsum[0];
        for (int w = 1; w < kThreads / 64; ++w) r += wsum[w];
        sqpart[blockIdx.x] = r;
    }
}

// The hidden layer's z = H W2 alone: from the fused GEMM's partials (the z of
// row_finish_kernel), or one wave per row (the z of row_pass_kernel).
__global__ __launch_bounds__(kThreads) void z_finish_kernel(const float* __restrict__ zpart, int P, int B,
                                                            float* __restrict__ z) {
    const int row = blockIdx.x * kThreads + threadIdx.x;
    if (row < B) z[row] = sum_row_partials(zpart, P, B, row);
}

__global__ __launch_bounds__(kThreads) void row_dot_kernel(const float* __restrict__ H, const float* __restrict__ W2,
                                                           int B, int Hd, float* __restrict__ z) {
    const int row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (row >= B) return;
    const float acc = row_dot(H + (int64_t)row * Hd, W2, Hd);
    if ((threadIdx.x & 63) == 0) z[row] = acc;
}

// Column pass: each thread owns 4 consecutive columns of a band of rows.
// Writes d1 (over H when D1 is H) and one dW2 partial per (row band, column).
constexpr int kRowsPerBand = 256;
__global__ __launch_bounds__(kThreads) void col_pass_kernel(const float* H, float* D1,
                                                            const float* __restrict__ W2,
                                                            const float* __restrict__ d2, int B,
                                                            int Hd, float* __restrict__ part) {
    const int c = (blockIdx.x * kThreads + threadIdx.x) * 4;
    if (c >= Hd) return;
    const int r0 = blockIdx.y * kRowsPerBand;
    const int r1 = min(B, r0 + kRowsPerBand);
    const int nc = min(4, Hd - c);
    float w[4], s[4] = {0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < 4; ++j) w[j] = j < nc ? W2[c + j] : 0.0f;
    for (int r = r0; r < r1; ++r) {
        const float* h = H + (int64_t)r * Hd + c;
        float* d1 = D1 + (int64_t)r * Hd + c;
        const float dm = d2[r];
        for (int j = 0; j < nc; ++j) {
            float hv = h[j];
            s[j] += hv * dm;
            float g = dm * w[j];
            d1[j] = g * hv * (1.0f - hv);
        }
    }
    for (int j = 0; j < nc; ++j) part[(int64_t)blockIdx.y * Hd + c + j] = s[j];
}

// out[i] = sum_s part[s*n + i] (fixed order); optional copy to dW; W -= lr * out.
__global__ __launch_bounds__(kThreads) void sum_slices_sgd_kernel(const float* __restrict__ part,
                                                                  int slices, int64_t n,
                                                                  float* __restrict__ dw,
                                                                  float* __restrict__ w, float lr) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
        float g = part[i];
        int s = 1;
        for (; s + kPartUnroll <= slices; s += kPartUnroll) {  // kPartUnroll loads in flight, same order
            float v[kPartUnroll];
#pragma unroll
            for (int u = 0; u < kPartUnroll; ++u) v[u] = part[(int64_t)(s + u) * n + i];
#pragma unroll
            for (int u = 0; u < kPartUnroll; ++u) g += v[u];
        }
        for (; s < slices; ++s) g += part[(int64_t)s * n + i];
        if (dw) dw[i] = g;
        if (lr != 0.0f) w[i] = w[i] - lr * g;
    }
}

// Fused path: dW1[m][n] = w2[n] * sum_s part[s][m][n] (fixed order) -- the
// column factor of d1 = (d2 w2) h(1-h), left out of the GEMM's operand
// transform -- with an optional copy to dW, then W -= lr * dW1.  Blocks cover
// 256 columns and stride over rows.
__global__ __launch_bounds__(kThreads) void dw1_finish_kernel(const float* __restrict__ part, int slices,
                                                              int rows, int cols, const float* __restrict__ w2,
                                                              float* __restrict__ dw, float* __restrict__ w,
                                                              float lr) {
    const int c = blockIdx.x * kThreads + threadIdx.x;
    if (c >= cols) return;
    const float f = w2[c];
    const int64_t n = (int64_t)rows * cols;
    for (int r = blockIdx.y; r < rows; r += gridDim.y) {
        const int64_t i = (int64_t)r * cols + c;
        float g = part[i];
        for (int s = 1; s < slices; ++s) g += part[(int64_t)s * n + i];
        g = f * g;
        if (dw) dw[i] = g;
        if (lr != 0.0f) w[i] = w[i] - lr * g;
    }
}

// loss = (sum of the n values v) / count: per-row squared errors (unfused
// path, n = B) or per-block sums of them (fused path).
__global__ __launch_bounds__(kThreads) void loss_kernel(const float* __restrict__ v, int n, float count,
                                                        float* __restrict__ loss) {
    __shared__ float part[kThreads / 64];
    float acc = 0.0f;
    // v[t], v[t + 256], ... in that order, kPartUnroll loads in flight
    int i = threadIdx.x;
    for (; i + (kPartUnroll - 1) * kThreads < n; i += kPartUnroll * kThreads) {
        float w[kPartUnroll];
#pragma unroll
        for (int u = 0; u < kPartUnroll; ++u) w[u] = v[i + u * kThreads];
#pragma unroll
        for (int u = 0; u < kPartUnroll; ++u) acc += w[u];
    }
    for (; i < n; i += kThreads) acc += v[i];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        float r = 0.0f;
        for (int w = 0; w < kThreads / 64; ++w) r += part[w];
        *loss = r / count;
    }
}

unsigned capped_grid(int64_t n) {
    int64_t want = (n + kThreads - 1) / kThreads;
    int64_t cap = (int64_t)ch::num_cus() * 8;
    if (want > cap) want = cap;
    return (unsigned)(want < 1 ? 1 : want);
}

// Split count for X^T d1: enough workgroups to fill the chip, K divisible.
int choose_splits(int D, int Hd, int B) {
    const int tiles = ((D + 127) / 128) * ((Hd + 127) / 128);
    int splits = 1;
    while (splits < 16 && tiles * splits < 4 * ch::num_cus() && B % (splits * 2 * 16) == 0) splits *= 2;
    return splits;
}

// ---- fused path (shapes that divide the 256 x 256 x 16 f32 tile) -----------
//   1. H = sigmoid(X W1) and partials of H W2      f32 ping-pong GEMM, MODE 1
//   2. z2, yhat, e, sq, d2 per row; loss           row_finish, loss kernels
//   3. slices of X^T (d1 / W2) with d1 / W2 = d2 H(1-H) formed as the MFMA
//      reads H, and dW2 partials                   f32 ping-pong GEMM, MODE 2
//   4. dW1 = W2 (column factor) * sum of slices, W1 -= lr dW1; dW2 likewise
//      (W2 is updated last: steps 3 and 4 read it)
using FusedTile1 = ch::F32PingPong<true, false, 1>;
using FusedTile2 = ch::F32PingPong<false, false, 2>;

int fused_splits(int B, int D, int Hd) {
    const int tiles = (D / 256) * (Hd / 256);
    int splits = 1;
    while (tiles * splits < ch::num_cus() && splits < 64 && B % (splits * 2 * 16) == 0) splits *= 2;
    return splits;
}

bool fused_fits(const float* x, const float* w1, int B, int D, int Hd) {
    if (B % 256 || D % 256 || Hd % 256) return false;
    if (((uintptr_t)x & 15) || ((uintptr_t)w1 & 15)) return false;  // 16-byte operand loads
    const int splits = fused_splits(B, D, Hd);
    return FusedTile1::fits(B, Hd, D, D, Hd) && FusedTile2::fits(D, Hd, B / splits, D, Hd);
}

int32_t fused_step(const float* x, const float* y, float* w1, float* w2, float* dw1, float* dw2,
                   float* loss_dev, int B, int D, int Hd, float lr, hipStream_t st) {
    const int splits = fused_splits(B, D, Hd);
    const int P = (Hd / 256) * 4;  // H W2 partials per row (tiles_n x waves along N)
    const int row_blocks = (B + kThreads - 1) / kThreads;
    // dW2 partials: one per (split, M-tile, row-half wave), see MlpFuse
    const int dw2_slices = splits * (D / 256) * 2;
    // Scratch slot 4: H | zpart | sq | d2 | dW2 partials | dW1 slices | loss.
    const size_t nH = (size_t)B * Hd, nZ = (size_t)P * B, nPart = (size_t)dw2_slices * Hd,
                 nSl = (size_t)splits * D * Hd;
    auto up = [](size_t n) { return (n + 63) & ~(size_t)63; };
    const size_t total = up(nH) + up(nZ) + up(B) + up(B) + up(nPart) + up(nSl) + 64;
    float* base = (float*)ch::scratch(4, total * sizeof(float));
    if (!base) return CLEAVE_HIP_ERR_OOM;
    float* H = base;
    float* zpart = H + up(nH);
    float* sq = zpart + up(nZ);
    float* d2 = sq + up(B);
    float* part = d2 + up(B);
    float* slices = part + up(nPart);
    float* loss_tmp = slices + up(nSl);

    ch::MlpFuse f1;
    f1.w2 = w2;
    f1.zpart = zpart;
    ch::gemm_f32_pingpong_kernel<true, false, 1>
        <<<dim3((unsigned)((B / 256) * (Hd / 256))), FusedTile1::THREADS, 0, st>>>(
            x, w1, H, B, Hd, D, D, Hd, 0, 0, 0, B / 256, Hd / 256, 1, 1, f1);
    CH_LAUNCHED("gemm_f32_pingpong_kernel(MODE 1)");
    row_finish_kernel<<<row_blocks, kThreads, 0, st>>>(zpart, P, y, B, sq, d2);
    CH_LAUNCHED("row_finish_kernel");
    // mean of the squared errors: the row blocks' sums, added in order, over B
    loss_kernel<<<1, kThreads, 0, st>>>(sq, row_blocks, (float)B, loss_dev ? loss_dev : loss_tmp);
    CH_LAUNCHED("loss_kernel");
    const int kk = B / splits;
    ch::MlpFuse f2;
    f2.d2 = d2;
    f2.dw2part = part;
    ch::gemm_f32_pingpong_kernel<false, false, 2>
        <<<dim3((unsigned)((D / 256) * (Hd / 256) * splits)), FusedTile2::THREADS, 0, st>>>(
            x, H, slices, D, Hd, kk, D, Hd, (int64_t)kk * D, (int64_t)kk * Hd, (int64_t)D * Hd, D / 256,
            Hd / 256, splits, 1, f2);
    CH_LAUNCHED("gemm_f32_pingpong_kernel(MODE 2)");
    dw1_finish_kernel<<<dim3((unsigned)((Hd + kThreads - 1) / kThreads), (unsigned)(D < 1024 ? D : 1024)),
                        kThreads, 0, st>>>(slices, splits, D, Hd, w2, dw1, w1, lr);
    CH_LAUNCHED("dw1_finish_kernel");
    sum_slices_sgd_kernel<<<capped_grid(Hd), kThreads, 0, st>>>(part, dw2_slices, Hd, dw2, w2, lr);
    CH_LAUNCHED("sum_slices_sgd_kernel(dW2)");
    return CLEAVE_HIP_OK;
}

// ---- the hidden layer alone: z = sigmoid(X W1) w2 and its reverse rule ----------
// The same kernels as the step, for a host (the reverse-mode tape) that meets
// this subgraph in a program: forward writes H and z; backward takes H and
// g = dL/dz and writes dW1 = X^T d1, dW2 = H^T g with d1 = (g w2^T) H(1-H).
bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

bool layer_fwd_fits(const float* x, const float* w1, const float* h, int B, int D, int Hd) {
    return B % 256 == 0 && D % 256 == 0 && Hd % 256 == 0 && aligned16(x) && aligned16(w1) && aligned16(h) &&
           FusedTile1::fits(B, Hd, D, D, Hd);
}

bool layer_bwd_fits(const float* x, const float* h, int B, int D, int Hd) {
    return B % 256 == 0 && D % 256 == 0 && Hd % 256 == 0 && aligned16(x) && aligned16(h) &&
           FusedTile2::fits(D, Hd, B / fused_splits(B, D, Hd), D, Hd);
}

int32_t hidden_fwd(const float* x, const float* w1, const float* w2, float* h, float* z, int B, int D, int Hd,
                   hipStream_t st) {
    if (layer_fwd_fits(x, w1, h, B, D, Hd)) {
        const int P = (Hd / 256) * 4;
        float* zpart = (float*)ch::scratch(4, sizeof(float) * (size_t)P * B);
        if (!zpart) return CLEAVE_HIP_ERR_OOM;
        ch::MlpFuse f1;
        f1.w2 = w2;
        f1.zpart = zpart;
        ch::gemm_f32_pingpong_kernel<true, false, 1>
            <<<dim3((unsigned)((B / 256) * (Hd / 256))), FusedTile1::THREADS, 0, st>>>(
                x, w1, h, B, Hd, D, D, Hd, 0, 0, 0, B / 256, Hd / 256, 1, 1, f1);
        CH_LAUNCHED("gemm_f32_pingpong_kernel(MODE 1)");
        z_finish_kernel<<<(B + kThreads - 1) / kThreads, kThreads, 0, st>>>(zpart, P, B, z);
        CH_LAUNCHED("z_finish_kernel");
        return CLEAVE_HIP_OK;
    }
    int32_t rc = ch::gemm_f32_device(x, w1, h, B, Hd, D, 0, 0, 1);
    if (rc != CLEAVE_HIP_OK) return rc;
    const int64_t nH = (int64_t)B * Hd;
    sigmoid_inplace_kernel<<<capped_grid(nH / 4 + 1), kThreads, 0, st>>>(h, nH);
    CH_LAUNCHED("sigmoid_inplace_kernel");
    row_dot_kernel<<<(B + 3) / 4, kThreads, 0, st>>>(h, w2, B, Hd, z);
    CH_LAUNCHED("row_dot_kernel");
    return CLEAVE_HIP_OK;
}

int32_t hidden_bwd(const float* x, const float* h, const float* w2, const float* g, float* dw1, float* dw2, int B,
                   int D, int Hd, hipStream_t st) {
    auto up = [](size_t n) { return (n + 63) & ~(size_t)63; };
    if (layer_bwd_fits(x, h, B, D, Hd)) {
        const int splits = fused_splits(B, D, Hd);
        const int dw2_slices = splits * (D / 256) * 2;
        const size_t nPart = (size_t)dw2_slices * Hd, nSl = (size_t)splits * D * Hd;
        float* part = (float*)ch::scratch(4, sizeof(float) * (up(nPart) + up(nSl)));
        if (!part) return CLEAVE_HIP_ERR_OOM;
        float* slices = part + up(nPart);
        const int kk = B / splits;
        ch::MlpFuse f2;
        f2.d2 = g;
        f2.dw2part = part;
        ch::gemm_f32_pingpong_kernel<false, false, 2>
            <<<dim3((unsigned)((D / 256) * (Hd / 256) * splits)), FusedTile2::THREADS, 0, st>>>(
                x, h, slices, D, Hd, kk, D, Hd, (int64_t)kk * D, (int64_t)kk * Hd, (int64_t)D * Hd, D / 256,
                Hd / 256, splits, 1, f2);
        CH_LAUNCHED("gemm_f32_pingpong_kernel(MODE 2)");
        if (dw1) {
            dw1_finish_kernel<<<dim3((unsigned)((Hd + kThreads - 1) / kThreads), (unsigned)(D < 1024 ? D : 1024)),
                                kThreads, 0, st>>>(slices, splits, D, Hd, w2, dw1, nullptr, 0.0f);
            CH_LAUNCHED("dw1_finish_kernel");
        }
        if (dw2) {
            sum_slices_sgd_kernel<<<capped_grid(Hd), kThreads, 0, st>>>(part, dw2_slices, Hd, dw2, nullptr, 0.0f);
            CH_LAUNCHED("sum_slices_sgd_kernel(dW2)");
        }
        return CLEAVE_HIP_OK;
    }
    const int splits = choose_splits(D, Hd, B);
    const int bands = (B + kRowsPerBand - 1) / kRowsPerBand;
    const size_t nH = (size_t)B * Hd, nPart = (size_t)bands * Hd, nSl = (size_t)splits * D * Hd;
    float* d1 = (float*)ch::scratch(4, sizeof(float) * (up(nH) + up(nPart) + up(nSl)));
    if (!d1) return CLEAVE_HIP_ERR_OOM;
    float* part = d1 + up(nH);
    float* slices = part + up(nPart);
    dim3 cgrid((unsigned)((Hd + 4 * kThreads - 1) / (4 * kThreads)), (unsigned)bands);
    col_pass_kernel<<<cgrid, kThreads, 0, st>>>(h, d1, w2, g, B, Hd, part);
    CH_LAUNCHED("col_pass_kernel");
    if (dw2) {
        sum_slices_sgd_kernel<<<capped_grid(Hd), kThreads, 0, st>>>(part, bands, Hd, dw2, nullptr, 0.0f);
        CH_LAUNCHED("sum_slices_sgd_kernel(dW2)");
    }
    if (dw1) {
        int32_t rc = ch::gemm_f32_device(x, d1, slices, D, Hd, B, 1, 0, splits);
        if (rc != CLEAVE_HIP_OK) return rc;
        sum_slices_sgd_kernel<<<capped_grid((int64_t)D * Hd), kThreads, 0, st>>>(slices, splits, (int64_t)D * Hd,
                                                                                  dw1, nullptr, 0.0f);
        CH_LAUNCHED("sum_slices_sgd_kernel(dW1)");
    }
    return CLEAVE_HIP_OK;
}

}  // namespace

extern "C" int32_t cleave_hip_mlp_step_f32(const float* x, int64_t xlen, const float* y,
                                           int64_t ylen, float* w1, int64_t w1len, float* w2,
                                           int64_t w2len, float* dw1, int64_t dw1len, float* dw2,
                                           int64_t dw2len, float* loss_dev, int32_t B, int32_t D,
                                           int32_t Hd, float lr) {
    CH_REQUIRE(B > 0 && D > 0 && Hd > 0, "cleave_hip_mlp_step_f32: dims must be positive (B=%d D=%d Hd=%d)", B, D, Hd);
    CH_REQUIRE(xlen == (int64_t)B * D, "cleave_hip_mlp_step_f32: xlen %lld != B*D", (long long)xlen);
    CH_REQUIRE(ylen == B, "cleave_hip_mlp_step_f32: ylen %lld != B", (long long)ylen);
    CH_REQUIRE(w1len == (int64_t)D * Hd, "cleave_hip_mlp_step_f32: w1len %lld != D*Hd", (long long)w1len);
    CH_REQUIRE(w2len == Hd, "cleave_hip_mlp_step_f32: w2len %lld != Hd", (long long)w2len);
    CH_REQUIRE(!dw1 || dw1len == (int64_t)D * Hd, "cleave_hip_mlp_step_f32: dw1len %lld != D*Hd", (long long)dw1len);
    CH_REQUIRE(!dw2 || dw2len == Hd, "cleave_hip_mlp_step_f32: dw2len %lld != Hd", (long long)dw2len);
    CH_REQUIRE(x && y && w1 && w2, "cleave_hip_mlp_step_f32: null buffer");
    CH_REQUIRE(((uintptr_t)w2 & 15) == 0, "cleave_hip_mlp_step_f32: w2 must be 16-byte aligned");
    CH_INIT_OR_RETURN();
    const char* fn = "cleave_hip_mlp_step_f32";
    CH_DEVICE(fn, x, xlen * 4);
    CH_DEVICE(fn, y, ylen * 4);
    CH_DEVICE(fn, w1, w1len * 4);
    CH_DEVICE(fn, w2, w2len * 4);
    if (dw1) CH_DEVICE(fn, dw1, dw1len * 4);
    if (dw2) CH_DEVICE(fn, dw2, dw2len * 4);
    if (loss_dev) CH_DEVICE(fn, loss_dev, 4);

    hipStream_t st = ch::stream();
    if (fused_fits(x, w1, B, D, Hd)) return fused_step(x, y, w1, w2, dw1, dw2, loss_dev, B, D, Hd, lr, st);

    const int splits = choose_splits(D, Hd, B);
    const int bands = (B + kRowsPerBand - 1) / kRowsPerBand;
    // Scratch slot 4: H/d1 | sq | d2 | dW2 partials | dW1 slices | loss.
    const size_t nH = (size_t)B * Hd, nPart = (size_t)bands * Hd, nSl = (size_t)splits * D * Hd;
    auto up = [](size_t n) { return (n + 63) & ~(size_t)63; };
    const size_t total = up(nH) + up(B) + up(B) + up(nPart) + up(nSl) + 64;
    float* base = (float*)ch::scratch(4, total * sizeof(float));
    if (!base) return CLEAVE_HIP_ERR_OOM;
    float* H = base;
    float* sq = H + up(nH);
    float* d2 = sq + up(B);
    float* part = d2 + up(B);
    float* slices = part + up(nPart);
    float* loss_tmp = slices + up(nSl);

    int32_t rc = ch::gemm_f32_device(x, w1, H, B, Hd, D, 0, 0, 1);
    if (rc != CLEAVE_HIP_OK) return rc;
    sigmoid_inplace_kernel<<<capped_grid(nH / 4 + 1), kThreads, 0, st>>>(H, (int64_t)nH);
    CH_LAUNCHED("sigmoid_inplace_kernel");
    row_pass_kernel<<<(B + 3) / 4, kThreads, 0, st>>>(H, w2, y, B, Hd, sq, d2);
    CH_LAUNCHED("row_pass_kernel");
    loss_kernel<<<1, kThreads, 0, st>>>(sq, B, (float)B, loss_dev ? loss_dev : loss_tmp);
    CH_LAUNCHED("loss_kernel");
    dim3 cgrid((unsigned)((Hd + 4 * kThreads - 1) / (4 * kThreads)), (unsigned)bands);
    col_pass_kernel<<<cgrid, kThreads, 0, st>>>(H, H, w2, d2, B, Hd, part);
    CH_LAUNCHED("col_pass_kernel");
    sum_slices_sgd_kernel<<<capped_grid(Hd), kThreads, 0, st>>>(part, bands, Hd, dw2, w2, lr);
    CH_LAUNCHED("sum_slices_sgd_kernel(dW2)");
    rc = ch::gemm_f32_device(x, H, slices, D, Hd, B, 1, 0, splits);
    if (rc != CLEAVE_HIP_OK) return rc;
    sum_slices_sgd_kernel<<<capped_grid((int64_t)D * Hd), kThreads, 0, st>>>(slices, splits, (int64_t)D * Hd, dw1, w1, lr);
    CH_LAUNCHED("sum_slices_sgd_kernel(dW1)");
    return CLEAVE_HIP_OK;
}

extern "C" int32_t cleave_hip_sigmoid_hidden_fwd_f32(const float* x, int64_t xlen, const float* w1, int64_t w1len,
                                                     const float* w2, int64_t w2len, float* h, int64_t hlen,
                                                     float* z, int64_t zlen, int32_t B, int32_t D, int32_t Hd) {
    const char* fn = "cleave_hip_sigmoid_hidden_fwd_f32";
    CH_REQUIRE(B > 0 && D > 0 && Hd > 0, "%s: dims must be positive (B=%d D=%d Hd=%d)", fn, B, D, Hd);
    CH_REQUIRE(xlen == (int64_t)B * D && w1len == (int64_t)D * Hd && w2len == Hd && hlen == (int64_t)B * Hd &&
                   zlen == B,
               "%s: lengths (%lld, %lld, %lld, %lld, %lld) do not match B=%d D=%d Hd=%d", fn, (long long)xlen,
               (long long)w1len, (long long)w2len, (long long)hlen, (long long)zlen, B, D, Hd);
    CH_REQUIRE(x && w1 && w2 && h && z, "%s: null buffer", fn);
    CH_REQUIRE(aligned16(w2) && aligned16(h), "%s: w2 and h must be 16-byte aligned", fn);
    CH_INIT_OR_RETURN();
    CH_DEVICE(fn, x, xlen * 4);
    CH_DEVICE(fn, w1, w1len * 4);
    CH_DEVICE(fn, w2, w2len * 4);
    CH_DEVICE(fn, h, hlen * 4);
    CH_DEVICE(fn, z, zlen * 4);
    return hidden_fwd(x, w1, w2, h, z, B, D, Hd, ch::stream());
}

extern "C" int32_t cleave_hip_sigmoid_hidden_bwd_f32(const float* x, int64_t xlen, const float* h, int64_t hlen,
                                                     const float* w2, int64_t w2len, const float* g, int64_t glen,
                                                     float* dw1, int64_t dw1len, float* dw2, int64_t dw2len,
                                                     int32_t B, int32_t D, int32_t Hd) {
    const char* fn = "cleave_hip_sigmoid_hidden_bwd_f32";
    CH_REQUIRE(B > 0 && D > 0 && Hd > 0, "%s: dims must be positive (B=%d D=%d Hd=%d)", fn, B, D, Hd);
    CH_REQUIRE(xlen == (int64_t)B * D && hlen == (int64_t)B * Hd && w2len == Hd && glen == B,
               "%s: lengths (%lld, %lld, %lld, %lld) do not match B=%d D=%d Hd=%d", fn, (long long)xlen,
               (long long)hlen, (long long)w2len, (long long)glen, B, D, Hd);
    CH_REQUIRE(!dw1 || dw1len == (int64_t)D * Hd, "%s: dw1len %lld != D*Hd", fn, (long long)dw1len);
    CH_REQUIRE(!dw2 || dw2len == Hd, "%s: dw2len %lld != Hd", fn, (long long)dw2len);
    CH_REQUIRE(x && h && w2 && g, "%s: null buffer", fn);
    CH_INIT_OR_RETURN();
    CH_DEVICE(fn, x, xlen * 4);
    CH_DEVICE(fn, h, hlen * 4);
    CH_DEVICE(fn, w2, w2len * 4);
    CH_DEVICE(fn, g, glen * 4);
    if (dw1) CH_DEVICE(fn, dw1, dw1len * 4);
    if (dw2) CH_DEVICE(fn, dw2, dw2len * 4);
    if (!dw1 && !dw2) return CLEAVE_HIP_OK;
    return hidden_bwd(x, h, w2, g, dw1, dw2, B, D, Hd, ch::stream());
}
