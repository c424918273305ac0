// Elementwise and row kernels around the GEMM: bias, ReLU forward/backward,
// column sums, row softmax, softmax cross-entropy (loss and gradient), SGD
// and the Philox random fills.  All are HBM- or latency-bound; none uses
// atomics, so every result is deterministic run to run.
#include "fdl_device.hpp"
#include "fdl_internal.hpp"

#include <algorithm>

namespace fdl {

namespace {

constexpr int kBlock = 256;

inline unsigned grid_for(int64_t n, int per_thread = 1) {
    const int64_t threads = (n + per_thread - 1) / per_thread;
    const int64_t blocks = (threads + kBlock - 1) / kBlock;
    return (unsigned)std::min<int64_t>(blocks, 1 << 20);
}

// out[r, c] += bias[c]   (src/kernels/cuda/bias.cu:5-12 semantics)
__global__ void add_row_bias_kernel(float* __restrict__ out,
                                    const float* __restrict__ bias,
                                    int64_t rows, int64_t cols) {
    const int64_t n = rows * cols;
    for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        out[idx] += bias[idx % cols];
    }
}

__global__ void relu_kernel(const float* __restrict__ in, float* __restrict__ out,
                            int64_t n) {
    for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        out[idx] = fmaxf(0.0f, in[idx]);
    }
}

__global__ void relu_backward_kernel(const float* __restrict__ g,
                                     const float* __restrict__ act,
                                     float* __restrict__ out, int64_t n) {
    for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        out[idx] = act[idx] > 0.0f ? g[idx] : 0.0f;
    }
}

__global__ void __launch_bounds__(kColsumThreads)
colsum_kernel(const float* __restrict__ x, float* __restrict__ out,
              float* __restrict__ param, float lr, int64_t rows, int64_t cols) {
    colsum_body(x, out, param, lr, rows, cols, blockIdx.x);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Row softmax: one wave per row, 4 rows per block.
__global__ void softmax_kernel(const float* __restrict__ in, float* __restrict__ out,
                               int64_t rows, int64_t cols) {
    const int lane = threadIdx.x & 63;
    const int64_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* x = in + row * cols;
    float* y = out + row * cols;
    float mx = -INFINITY;
    for (int64_t c = lane; c < cols; c += 64) mx = fmaxf(mx, x[c]);
    mx = wave_max(mx);
    float s = 0.0f;
    for (int64_t c = lane; c < cols; c += 64) s += expf(x[c] - mx);
    s = wave_sum(s);
    for (int64_t c = lane; c < cols; c += 64) y[c] = expf(x[c] - mx) / s;
}

// Softmax cross-entropy over the whole batch in one block: thread t owns rows
// t, t+256, ...; per-thread loss partials are combined by a fixed tree, so
// the loss is deterministic (the reference used a float atomicAdd per row).
__global__ void __launch_bounds__(kBlock)
softmax_xent_kernel(const float* __restrict__ logits,
                    const int64_t* __restrict__ labels, float* __restrict__ loss,
                    float* __restrict__ grad, int64_t batch, int64_t classes) {
    __shared__ float part[kBlock];
    const float inv_b = 1.0f / (float)batch;
    float lsum = 0.0f;
    for (int64_t row = threadIdx.x; row < batch; row += kBlock) {
        const float* z = logits + row * classes;
        float mx = z[0];
        for (int64_t c = 1; c < classes; ++c) mx = fmaxf(mx, z[c]);
        float s = 0.0f;
        for (int64_t c = 0; c < classes; ++c) s += expf(z[c] - mx);
        const int64_t label = labels[row];
        const bool valid = label >= 0 && label < classes;
        if (valid) lsum += (logf(s) + mx - z[label]) * inv_b;
        if (grad) {
            float* g = grad + row * classes;
            const float inv_s = 1.0f / s;
            for (int64_t c = 0; c < classes; ++c) {
                float pc = expf(z[c] - mx) * inv_s;
                if (valid && c == label) pc -= 1.0f;
                g[c] = pc * inv_b;
            }
        }
    }
    part[threadIdx.x] = lsum;
    __syncthreads();
    for (int w = kBlock / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0 && loss) loss[0] = part[0];
}

// Softmax cross-entropy for classes <= kXentFusedMaxClasses with the bias
// gradient and the bias SGD step fused: one block walks the batch in chunks of
// 256 rows staged through LDS with coalesced loads (thread t owns row t of
// the chunk), writes the gradient through LDS with coalesced stores, and adds
// each chunk's gradient column sums in row order.  db and bparam are written
// once at the end.
__global__ void __launch_bounds__(kBlock)
softmax_xent_db_sgd_kernel(const float* __restrict__ logits,
                           const int64_t* __restrict__ labels, float* __restrict__ loss,
                           float* __restrict__ grad, float* __restrict__ db,
                           float* __restrict__ bparam, float lr, int64_t batch,
                           int64_t classes) {
#pragma clang fp contract(off)
    __shared__ float zs[kBlock * kXentFusedMaxClasses];
    __shared__ float part[kBlock];
    __shared__ float wpart[kBlock / 64];
    const int t = threadIdx.x;
    const float inv_b = 1.0f / (float)batch;
    // Loads whose values are needed late are issued first, so the step pays
    // one global-memory round trip, not one per phase.
    const float bold = t < classes ? bparam[t] : 0.0f;
    float lsum = 0.0f;
    // Column sums of the gradient: thread t adds class cls over the rows
    // r = grp, grp + ngrp, ... of each chunk (ngrp groups of cpad threads).
    const int cpad = classes <= 8 ? 8 : (classes <= 16 ? 16 : 32);
    const int ngrp = kBlock / cpad;
    const int cls = t % cpad;
    const int grp = t / cpad;
    float dbc = 0.0f;
    for (int64_t r0 = 0; r0 < batch; r0 += kBlock) {
        const int rows = (int)min<int64_t>(kBlock, batch - r0);
        const int n = rows * (int)classes;
        const int64_t label = t < rows ? labels[r0 + t] : -1;
        const float* zsrc = logits + r0 * classes;
        for (int e = t; e < n; e += kBlock) zs[e] = zsrc[e];
        __syncthreads();
        if (t < rows) {
            float* z = zs + t * classes;
            float mx = z[0];
            for (int c = 1; c < classes; ++c) mx = fmaxf(mx, z[c]);
            float s = 0.0f;
            for (int c = 0; c < classes; ++c) s += expf(z[c] - mx);
            const bool valid = label >= 0 && label < classes;
            if (valid) lsum += (logf(s) + mx - z[label]) * inv_b;
            const float inv_s = 1.0f / s;
            for (int c = 0; c < classes; ++c) {
                float pc = expf(z[c] - mx) * inv_s;
                if (valid && c == label) pc -= 1.0f;
                z[c] = pc * inv_b;
            }
        }
        __syncthreads();
        float* gdst = grad + r0 * classes;
        for (int e = t; e < n; e += kBlock) gdst[e] = zs[e];
        if (cls < classes) {
            for (int r = grp; r < rows; r += ngrp) dbc += zs[r * classes + cls];
        }
        __syncthreads();
    }
    // Group partials of each class, added in group order; the loss is summed
    // within each wave, then over the waves in wave order.
    part[t] = dbc;
    lsum = wave_sum(lsum);
    if ((t & 63) == 0) wpart[t >> 6] = lsum;
    __syncthreads();
    if (t < classes) {
        float d = part[t];
        for (int g = 1; g < ngrp; ++g) d += part[g * cpad + t];
        db[t] = d;
        const float step = lr * d;
        bparam[t] = bold - step;
    }
    if (t == 0 && loss) {
        float l = wpart[0];
        for (int w = 1; w < kBlock / 64; ++w) l += wpart[w];
        loss[0] = l;
    }
}

// p -= lr * g with the product rounded before the subtraction (no FMA
// contraction), as the reference's x86 host update computes it.
__global__ void sgd_kernel(float* __restrict__ p, const float* __restrict__ g,
                           float lr, int64_t n) {
    sgd_body(p, g, lr, n, blockIdx.x, gridDim.x);
}

struct SgdMulti {
    float* p[4];
    const float* g[4];
    int64_t n[4];
};

// blockIdx.y selects the tensor; the x grid strides over the largest one.
__global__ void sgd_multi_kernel(SgdMulti args, float lr) {
#pragma clang fp contract(off)
    const int t = blockIdx.y;
    float* __restrict__ p = args.p[t];
    const float* __restrict__ g = args.g[t];
    const int64_t n = args.n[t];
    for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        p[idx] -= lr * g[idx];
    }
}

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
// easy as 1, 2, 3", SC'11): counter (i_lo, i_hi, 0, 0), key = seed.
struct Philox4 {
    uint32_t v[4];
};

__device__ __forceinline__ Philox4 philox4x32_10(uint64_t ctr, uint64_t seed) {
    uint32_t c0 = (uint32_t)ctr, c1 = (uint32_t)(ctr >> 32), c2 = 0u, c3 = 0u;
    uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
    constexpr uint32_t kM0 = 0xD2511F53u, kM1 = 0xCD9E8D57u;
    constexpr uint32_t kW0 = 0x9E3779B9u, kW1 = 0xBB67AE85u;
#pragma unroll
    for (int round = 0; round < 10; ++round) {
        const uint32_t hi0 = __umulhi(kM0, c0), lo0 = kM0 * c0;
        const uint32_t hi1 = __umulhi(kM1, c2), lo1 = kM1 * c2;
        const uint32_t n0 = hi1 ^ c1 ^ k0;
        const uint32_t n2 = hi0 ^ c3 ^ k1;
        c0 = n0;
        c1 = lo1;
        c2 = n2;
        c3 = lo0;
        k0 += kW0;
        k1 += kW1;
    }
    Philox4 out;
    out.v[0] = c0;
    out.v[1] = c1;
    out.v[2] = c2;
    out.v[3] = c3;
    return out;
}

// 24 random bits -> (0, 1].
__device__ __forceinline__ float u01_open_closed(uint32_t x) {
    return (float)((x >> 8) + 1u) * (1.0f / 16777216.0f);
}

__global__ void fill_uniform_kernel(float* __restrict__ data, int64_t n, float low,
                                    float high, uint64_t seed) {
    for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const Philox4 r = philox4x32_10((uint64_t)idx, seed);
        data[idx] = low + u01_open_closed(r.v[0]) * (high - low);
    }
}

// Box-Muller on two uniforms of the same counter.
__global__ void fill_normal_kernel(float* __restrict__ data, int64_t n, float mean,
                                   float stddev, uint64_t seed) {
    for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const Philox4 r = philox4x32_10((uint64_t)idx, seed);
        const float u1 = u01_open_closed(r.v[0]);
        const float u2 = (float)(r.v[1] >> 8) * (1.0f / 16777216.0f);
        const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
        data[idx] = mean + stddev * z;
    }
}

}  // namespace

hipError_t launch_add_row_bias(float* out, const float* bias, int64_t rows,
                               int64_t cols, hipStream_t stream) {
    const int64_t n = rows * cols;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(add_row_bias_kernel, dim3(grid_for(n)), dim3(kBlock), 0,
                       stream, out, bias, rows, cols);
    return hipGetLastError();
}

hipError_t launch_relu(const float* in, float* out, int64_t n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(relu_kernel, dim3(grid_for(n)), dim3(kBlock), 0, stream,
                       in, out, n);
    return hipGetLastError();
}

hipError_t launch_relu_backward(const float* g, const float* act, float* out,
                                int64_t n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(relu_backward_kernel, dim3(grid_for(n)), dim3(kBlock), 0,
                       stream, g, act, out, n);
    return hipGetLastError();
}

hipError_t launch_colsum_sgd(const float* x, float* out, float* param, float lr,
                             int64_t rows, int64_t cols, hipStream_t stream) {
    if (cols == 0) return hipSuccess;
    const unsigned blocks = (unsigned)((cols + kColsumCols - 1) / kColsumCols);
    hipLaunchKernelGGL(colsum_kernel, dim3(blocks), dim3(kColsumThreads), 0,
                       stream, x, out, param, lr, rows, cols);
    return hipGetLastError();
}

hipError_t launch_colsum(const float* x, float* out, int64_t rows, int64_t cols,
                         hipStream_t stream) {
    return launch_colsum_sgd(x, out, nullptr, 0.0f, rows, cols, stream);
}

hipError_t launch_softmax(const float* in, float* out, int64_t rows, int64_t cols,
                          hipStream_t stream) {
    if (rows == 0 || cols == 0) return hipSuccess;
    const unsigned blocks = (unsigned)((rows + 3) / 4);
    hipLaunchKernelGGL(softmax_kernel, dim3(blocks), dim3(kBlock), 0, stream, in,
                       out, rows, cols);
    return hipGetLastError();
}

hipError_t launch_softmax_xent(const float* logits, const int64_t* labels,
                               float* loss, float* grad, int64_t batch,
                               int64_t classes, hipStream_t stream) {
    hipLaunchKernelGGL(softmax_xent_kernel, dim3(1), dim3(kBlock), 0, stream,
                       logits, labels, loss, grad, batch, classes);
    return hipGetLastError();
}

hipError_t launch_softmax_xent_db_sgd(const float* logits, const int64_t* labels,
                                      float* loss, float* grad, float* db, float* bparam,
                                      float lr, int64_t batch, int64_t classes,
                                      hipStream_t stream) {
    if (classes > kXentFusedMaxClasses || !grad || !db || !bparam) return hipErrorInvalidValue;
    hipLaunchKernelGGL(softmax_xent_db_sgd_kernel, dim3(1), dim3(kBlock), 0, stream, logits,
                       labels, loss, grad, db, bparam, lr, batch, classes);
    return hipGetLastError();
}

hipError_t launch_sgd(float* param, const float* grad, float lr, int64_t n,
                      hipStream_t stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(sgd_kernel, dim3(grid_for(n, 4)), dim3(kBlock), 0, stream,
                       param, grad, lr, n);
    return hipGetLastError();
}

hipError_t launch_sgd_multi(int count, float* const* params,
                            const float* const* grads, const int64_t* sizes,
                            float lr, hipStream_t stream) {
    if (count <= 0 || count > 4) return hipErrorInvalidValue;
    SgdMulti args{};
    int64_t nmax = 0;
    for (int t = 0; t < count; ++t) {
        args.p[t] = params[t];
        args.g[t] = grads[t];
        args.n[t] = sizes[t];
        nmax = std::max(nmax, sizes[t]);
    }
    if (nmax == 0) return hipSuccess;
    hipLaunchKernelGGL(sgd_multi_kernel, dim3(grid_for(nmax, 4), count),
                       dim3(kBlock), 0, stream, args, lr);
    return hipGetLastError();
}

hipError_t launch_fill_uniform(float* data, int64_t n, float low, float high,
                               uint64_t seed, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_uniform_kernel, dim3(grid_for(n, 4)), dim3(kBlock), 0,
                       stream, data, n, low, high, seed);
    return hipGetLastError();
}

hipError_t launch_fill_normal(float* data, int64_t n, float mean, float stddev,
                              uint64_t seed, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_normal_kernel, dim3(grid_for(n, 4)), dim3(kBlock), 0,
                       stream, data, n, mean, stddev, seed);
    return hipGetLastError();
}

}  // namespace fdl
