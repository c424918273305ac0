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

// dst[e] = src[e] for e < n by a block of kBlock threads, 16 loads in flight
// per thread before their LDS stores (a plain strided loop waits out one
// global-memory round trip per iteration).
__device__ __forceinline__ void stage_to_lds(float* __restrict__ dst, const float* __restrict__ src,
                                             int n) {
    constexpr int kBatch = 16;
    const int t = threadIdx.x;
    for (int e0 = 0; e0 < n; e0 += kBatch * kBlock) {
        float v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int e = e0 + u * kBlock + t;
            v[u] = e < n ? src[e] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int e = e0 + u * kBlock + t;
            if (e < n) dst[e] = v[u];
        }
    }
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
        stage_to_lds(zs, logits + r0 * classes, n);
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

// The MLP step's head: kHeadRows rows per block, one half-wave (32 lanes) per
// row; CM >= classes and 32 * NH >= hidden are compile-time bounds.  Lane l
// holds H[row][l + 32 k].  W2 is staged in LDS as 32 * NH rows of CM floats
// (row stride CM + 4), zero past `hidden` rows and `classes` columns, so every loop over classes
// runs to CM with no bounds test (the padding adds exact zeros) and its LDS
// reads are issued together.
//   logits[row][c] = sum_j H[row][j] W2[j][c] + b2[c]: the 32 lane partials
//     meet in an xor butterfly, so every lane of the row ends with the same
//     sums; the bias is added after the sum, as in linear_cpu
//     (tests/tensor/linear_tensor_test.cpp:17-25).
//   loss share and G2[row][c] as in softmax_xent_db_sgd_kernel (the legacy
//     SoftmaxCrossEntropyLoss forward and backward,
//     legacy/src/ops/SoftmaxCrossEntropyLoss.cpp:39-51).
//   G1[row][j] = H[row][j] > 0 ? sum_c G2[row][c] W2[j][c] : 0 (the NT product
//     dY1 = G2 W2^T of legacy/src/ops/Layers.cpp:36 through the ReLU mask).
// The block's record at part + block * (classes + 1): the column sums of its
// G2 rows (rows in order), then the sum of its rows' loss shares;
// xent_finalize_body adds the records in block order.
// Lane exchanges within a half-wave (32 lanes) for the head's reductions.
// Step 0 pairs lane i with i ^ 16 (ds_swizzle), step 1 with 15 - i within
// 16 lanes (DPP row_mirror), step 2 with 7 - i within 8 (row_half_mirror),
// steps 3 and 4 with i ^ 2 and i ^ 1 (quad permutations).  Step s always
// pairs lanes that differ in bit 4 - s and agree in the bits above it, so
// applying op(x, partner(x)) for s = 0..4 reduces over all 32 lanes and
// leaves the same value on every lane (each pair computes a op b and b op a).
template <int kCtrl>
__device__ __forceinline__ float dpp_mov(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                                 kCtrl, 0xF, 0xF, false));
}

template <int kStep>
__device__ __forceinline__ float half_wave_partner(float x) {
    if constexpr (kStep == 0) {
        constexpr int kXor16 = 0x401F;  // ds_swizzle bit mode: and 0x1f, xor 0x10
        return __builtin_bit_cast(float,
                                  __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), kXor16));
    } else if constexpr (kStep == 1) {
        return dpp_mov<0x140>(x);  // row_mirror
    } else if constexpr (kStep == 2) {
        return dpp_mov<0x141>(x);  // row_half_mirror
    } else if constexpr (kStep == 3) {
        return dpp_mov<0x4E>(x);   // quad_perm [2, 3, 0, 1]
    } else {
        return dpp_mov<0xB1>(x);   // quad_perm [1, 0, 3, 2]
    }
}

__device__ __forceinline__ float half_wave_max(float x) {
    x = fmaxf(x, half_wave_partner<0>(x));
    x = fmaxf(x, half_wave_partner<1>(x));
    x = fmaxf(x, half_wave_partner<2>(x));
    x = fmaxf(x, half_wave_partner<3>(x));
    return fmaxf(x, half_wave_partner<4>(x));
}

__device__ __forceinline__ float half_wave_sum(float x) {
    x += half_wave_partner<0>(x);
    x += half_wave_partner<1>(x);
    x += half_wave_partner<2>(x);
    x += half_wave_partner<3>(x);
    return x + half_wave_partner<4>(x);
}

// One step of the transposing reduction: each lane holds N partial sums
// (one per class of its current set); it keeps the lower or upper half of
// the set (by the lane bit this step's pairing splits on) and adds the
// partner's partial sums of the same half.  Each lane sends the half its
// partner keeps, so a step costs N/2 exchanges.
template <int kStep, int N>
__device__ __forceinline__ void transpose_step(float (&v)[N], int lane) {
    constexpr int kHalf = N / 2;
    const bool upper = (lane >> (4 - kStep)) & 1;
#pragma unroll
    for (int i = 0; i < kHalf; ++i) {
        const float send = upper ? v[i] : v[kHalf + i];
        const float keep = upper ? v[kHalf + i] : v[i];
        v[i] = keep + half_wave_partner<kStep>(send);
    }
}

// Sums CM per-lane partials over the 32 lanes of a half-wave, class by
// class, leaving each lane with one class's total: class lane & 31 for
// CM = 32, class (lane & 31) >> 1 for CM = 16 (lanes 2c and 2c + 1 hold the
// same total).  31 (or 16) exchanges instead of 5 per class.
template <int CM>
__device__ __forceinline__ float transpose_sum(float (&v)[CM], int lane) {
    static_assert(CM == 16 || CM == 32, "16 or 32 classes");
    if constexpr (CM == 32) {
        transpose_step<0, 32>(v, lane);
        transpose_step<1, 16>(*reinterpret_cast<float(*)[16]>(v), lane);
        transpose_step<2, 8>(*reinterpret_cast<float(*)[8]>(v), lane);
        transpose_step<3, 4>(*reinterpret_cast<float(*)[4]>(v), lane);
        transpose_step<4, 2>(*reinterpret_cast<float(*)[2]>(v), lane);
        return v[0];
    } else {
        transpose_step<0, 16>(v, lane);
        transpose_step<1, 8>(*reinterpret_cast<float(*)[8]>(v), lane);
        transpose_step<2, 4>(*reinterpret_cast<float(*)[4]>(v), lane);
        transpose_step<3, 2>(*reinterpret_cast<float(*)[2]>(v), lane);
        return v[0] + half_wave_partner<4>(v[0]);
    }
}

template <int CM, int NH>
__global__ void __launch_bounds__(kBlock)
mlp_head_kernel(const float* __restrict__ H, const float* __restrict__ W2,
                const float* __restrict__ b2, const int64_t* __restrict__ labels,
                float* __restrict__ logits, float* __restrict__ G2, float* __restrict__ G1,
                float* __restrict__ part, int batch, int hidden, int classes) {
    constexpr int JR = 32 * NH;                  // W2 rows staged
    constexpr int LR = CM + 4;                   // LDS row stride: 16 consecutive lanes
                                                 // read 16-byte pieces on distinct banks
    constexpr int kPerThread = JR * CM / kBlock;  // staged floats per thread
    static_assert(kPerThread % 16 == 0, "staging runs in batches of 16 loads");
    __shared__ __attribute__((aligned(16))) float w2s[JR * LR];
    __shared__ float b2s[CM];
    __shared__ float g2s[kHeadRows][CM];
    __shared__ float ls[kHeadRows];
    const int t = threadIdx.x;
    const int lane = t & 31;
    const int rl = t >> 5;
    const int row = blockIdx.x * kHeadRows + rl;
    const bool live = row < batch;
    const int rowc = live ? row : batch - 1;  // clamped: loads stay in bounds
    // Every global load below is issued unconditionally at an address
    // clamped into its array, and values outside the problem are zeroed by
    // a select after the load: a load under a lane-divergent branch makes
    // the compiler wait for it before issuing the ones after it, which
    // turned the staging into two dependent round trips.
    const int64_t label = labels[rowc];
    const float* hrow = H + (int64_t)rowc * hidden;
    float h[NH];
#pragma unroll
    for (int k = 0; k < NH; ++k) h[k] = hrow[min(lane + 32 * k, hidden - 1)];
    const float b2v = b2[min(t, classes - 1)];
    // W2 in batches of sixteen loads in flight per thread.
#pragma unroll
    for (int b0 = 0; b0 < kPerThread; b0 += 16) {
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int e = (b0 + u) * kBlock + t;
            const int j = e / CM, c = e % CM;
            v[u] = W2[min(j, hidden - 1) * classes + min(c, classes - 1)];
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int e = (b0 + u) * kBlock + t;
            const int j = e / CM, c = e % CM;
            w2s[j * LR + c] = (j < hidden && c < classes) ? v[u] : 0.0f;
        }
    }
#pragma unroll
    for (int k = 0; k < NH; ++k) h[k] = lane + 32 * k < hidden ? h[k] : 0.0f;
    if (t < CM) b2s[t] = t < classes ? b2v : 0.0f;
    __syncthreads();

    float z[CM];
#pragma unroll
    for (int c = 0; c < CM; ++c) z[c] = 0.0f;
#pragma unroll
    for (int k = 0; k < NH; ++k) {
        const float* w = w2s + (lane + 32 * k) * LR;
#pragma unroll
        for (int c = 0; c < CM; ++c) z[c] = fmaf(h[k], w[c], z[c]);
    }
    // Each lane ends with one class's logit: class c of lane (c for CM = 32,
    // lanes 2c and 2c + 1 for CM = 16).  The softmax runs on that class
    // alone; the row's maximum, exponent sum and label logit are half-wave
    // reductions.  Lanes of padded classes (c >= classes) hold 0 and take
    // no part.
    const int c = CM == 32 ? lane : lane >> 1;
    const bool owner = CM == 32 || (lane & 1) == 0;  // counts class c once
    const bool cls = c < classes;
    float zc = transpose_sum<CM>(z, lane);
    float gc;
    float loss_share = 0.0f;
    {
#pragma clang fp contract(off)
        const float inv_b = 1.0f / (float)batch;
        zc = zc + b2s[c];
        const float mx = half_wave_max(cls ? zc : -INFINITY);
        const float ez = cls ? expf(zc - mx) : 0.0f;
        const float s = half_wave_sum(owner ? ez : 0.0f);
        const bool valid = label >= 0 && label < classes;
        const float zl = half_wave_sum(owner && c == label ? zc : 0.0f);
        if (valid && live) loss_share = (logf(s) + mx - zl) * inv_b;
        const float inv_s = 1.0f / s;
        float pc = cls ? ez * inv_s : 0.0f;
        if (valid && c == label) pc -= 1.0f;
        gc = pc * inv_b;
    }
    if (owner && cls) {
        if (live) {
            logits[(int64_t)row * classes + c] = zc;
            G2[(int64_t)row * classes + c] = gc;
        }
        g2s[rl][c] = live ? gc : 0.0f;
    }
    if (lane == 0) ls[rl] = loss_share;
    if (owner && !cls && c < CM) g2s[rl][c] = 0.0f;  // padded classes of the row
    __syncthreads();

    // G1 = (G2 W2^T) * [H > 0]: the row's G2 comes back from LDS as
    // broadcast reads, summed in class order.
    float g[CM];
#pragma unroll
    for (int q = 0; q < CM; ++q) g[q] = g2s[rl][q];
    float* g1row = G1 + (int64_t)rowc * hidden;
#pragma unroll
    for (int k = 0; k < NH; ++k) {
        const int j = lane + 32 * k;
        const float* w = w2s + j * LR;
        float v = 0.0f;
#pragma unroll
        for (int q = 0; q < CM; ++q) v = fmaf(g[q], w[q], v);
        if (live && j < hidden) g1row[j] = h[k] > 0.0f ? v : 0.0f;
    }
    if (t <= classes) {
#pragma clang fp contract(off)
        float acc = 0.0f;
        if (t < classes) {
#pragma unroll
            for (int r = 0; r < kHeadRows; ++r) acc += g2s[r][t];
        } else {
#pragma unroll
            for (int r = 0; r < kHeadRows; ++r) acc += ls[r];
        }
        part[(int64_t)blockIdx.x * (classes + 1) + t] = acc;
    }
}

// Reductions over the 16 lanes of a DPP row (steps 1 to 4 of the half-wave
// exchanges), leaving the result on every lane of the row.
__device__ __forceinline__ float row16_max(float x) {
    x = fmaxf(x, half_wave_partner<1>(x));
    x = fmaxf(x, half_wave_partner<2>(x));
    x = fmaxf(x, half_wave_partner<3>(x));
    return fmaxf(x, half_wave_partner<4>(x));
}

__device__ __forceinline__ float row16_sum(float x) {
    x += half_wave_partner<1>(x);
    x += half_wave_partner<2>(x);
    x += half_wave_partner<3>(x);
    return x + half_wave_partner<4>(x);
}

// The head fused with dX = G1 W1^T (the NT product of the legacy backward,
// legacy/src/ops/Layers.cpp:36-40), so that the W1 step can share the next
// launch with dW1: dX's last read of W1 is in this launch.  A block takes
// kHdxRows = 16 rows of the batch and kHdxCols = 64 columns of dX; every
// block recomputes the head for its rows and the blocks of column chunk 0
// store logits, G2 and G1.  All three products run on
// v_mfma_f32_16x16x4_f32:
//   operand a: lane l supplies A[i = l % 16][k]
//   operand b: lane l supplies B[k][j = l % 16]
//   result   : lane l, register r holds D[4 * (l / 16) + r][l % 16]
// with the k permutation of the split-K kernels (at step s of a group of 16,
// lane quarter q supplies k0 + 4q + s, so a lane's four values are one
// 16-byte load).
//   z = H W2 (16 rows x CT tiles of 16 classes): wave w adds hidden
//     [32w, 32w + 32) straight from H's rows; the eight waves' tiles meet in
//     LDS and wave 0 adds them in wave order, adds b2 after the sum (as
//     linear_cpu, tests/tensor/linear_tensor_test.cpp:17-25), and takes the
//     softmax of each row over the 16 lanes of a DPP row: G2 as
//     softmax_xent_kernel (legacy SoftmaxCrossEntropyLoss,
//     legacy/src/ops/SoftmaxCrossEntropyLoss.cpp:39-51).  The loss is left to
//     head_finalize_body, which reads the stored logits.
//   G1 = (G2 W2^T) * [H > 0] (legacy/src/ops/Layers.cpp:36 through the ReLU
//     mask): wave w makes hidden tiles 2w and 2w + 1, K = the classes.
//   dX = G1 W1^T: wave w makes column tile w % NCT over part w / NCT of the
//     hidden range; the other parts' sums reach part 0's wave through LDS
//     and are added in part order.
// W2 is staged in LDS as rows of CM floats (laid out by head_w2_at), zero
// past `hidden` rows and `classes` columns.  The head's global loads are all
// issued before its first wait, and dX's W1 fragments right after the
// staging barrier (loads complete in order, so the head's waits never count
// them), all at addresses clamped into the arrays; values outside the
// problem are zeroed where they are used.
// Needs hidden <= 256, hidden % 4 == 0, classes <= 16 * CT, and H and W1
// 16-byte aligned (the host checks).
constexpr int kHdxThreads = kHdxRows * 32;
constexpr int kWave = 64;

// LDS layouts of the head, chosen against gfx950's bank rules as measured
// with the LDS bank-conflict counter on single-wave access patterns: a
// 32-bit access is served in two halves of 32 lanes, each free of conflicts
// when its lanes' dword addresses differ mod 32 (equal addresses are free
// for reads); a ds_read_b128 is served in four passes of 16 lanes -- lane l
// in the pass of (l / 32, parity of bits 2..4 of l) -- each free of conflicts
// when its lanes' 16-byte slots differ mod 16.
//
// W2 and G2 tiles of 16 columns (CM == 16): row j sits at 48 j, moved on by
// 16 floats and with its 4-column slots swapped in pairs (XOR 8) when bit 2
// of j is set.  The staging stores (rows j and j + 1 in a half-wave), the z
// reads (rows j and j + 4), the G2 stores (rows r and r + 4) and the G1 b128
// reads (16 rows x 4 slots) are then all free of conflicts.  The shift and
// the swap depend on bit 2 of j alone, so row 4m + s (s < 4) sits s rows
// from row 4m, and adding a multiple of 8 rows or of 16 columns moves an
// address by exactly that many rows and columns: each access below takes a
// per-lane base plus immediate offsets.  Wider tiles keep a padded row of
// CM + 4 floats, for which the same holds.
template <int CM>
__device__ __forceinline__ int head_w2_at(int j, int c) {
    if constexpr (CM == 16) {
        const int b = (j >> 2) & 1;
        return 48 * j + 16 * b + (c ^ (8 * b));
    } else {
        return j * (CM + 4) + c;
    }
}
template <int CM>
constexpr int head_w2_row() { return CM == 16 ? 48 : CM + 4; }

// G1 tile (kHdxRows = 16 rows x 256 hidden, row stride 260): rows whose
// bits 2 and 3 differ swap the 4-column slots of each pair (XOR 4), so the G1
// stores (rows 4q + r of a half-wave, 16 columns each) and the dX b128 reads
// (16 rows, slot q) are both free of conflicts.  The swap depends on r / 4
// alone and touches bit 2 of the column alone, so rows 4q + r (r < 4) and
// columns c + 16k sit r rows and 16k columns from row 4q, column c.
constexpr int kHdxG1Row = 260;
__device__ __forceinline__ int head_g1_at(int r, int c) {
    return r * kHdxG1Row + (c ^ (4 * (((r >> 2) ^ (r >> 3)) & 1)));
}

template <int CT>
__global__ void __launch_bounds__(kHdxThreads)
mlp_head_dx_kernel(int batch, int in_features, int hidden, int classes,
                   const float* __restrict__ H, const float* __restrict__ W2,
                   const float* __restrict__ b2, const int64_t* __restrict__ labels,
                   const float* __restrict__ W1, float* __restrict__ logits,
                   float* __restrict__ G2, float* __restrict__ G1, float* __restrict__ dX) {
    // (the shape and the loaded operands lead the arguments: the first 14
    // dwords arrive preloaded in SGPRs, so the first loads' addresses wait
    // for no scalar load of the rest)
    constexpr int CM = 16 * CT;                  // classes padded to whole tiles
    constexpr int JR = 256;                      // hidden <= JR
    constexpr int LR = head_w2_row<CM>();        // floats per row of w2s and g2s
    constexpr int NW = kHdxThreads / kWave;      // 8 waves
    constexpr int KZ = JR / NW;                  // hidden range of a wave for z
    constexpr int NCT = kHdxCols / 16;           // dX column tiles of a block
    constexpr int NKS = NW / NCT;                // hidden range split in NKS parts
    constexpr int KH = JR / NKS;                 // hidden range of a wave for dX
    constexpr int NG = KH / 16;
    constexpr int kPerThread = JR * CM / kHdxThreads;  // W2 floats staged per thread
    static_assert(KZ == 32 && NW == 8, "z takes two groups of 16 per wave");
    static_assert(JR <= kHdxG1Row, "g1s rows hold the hidden range");
    __shared__ __attribute__((aligned(16))) float w2s[JR * LR];
    __shared__ __attribute__((aligned(16))) float g1s[kHdxRows * kHdxG1Row];
    __shared__ __attribute__((aligned(16))) float g2s[kHdxRows * LR];
    __shared__ __attribute__((aligned(16))) floatx4 zred[NW][CT][kWave];
    __shared__ __attribute__((aligned(16))) floatx4 red[NKS - 1][NCT][kWave];
    __shared__ int64_t lbls[kHdxRows];
    __shared__ float b2s[CM];
    const int t = threadIdx.x;
    const int l64 = t & (kWave - 1);
    const int w = __builtin_amdgcn_readfirstlane(t / kWave);
    const int q = l64 >> 4;
    const int i16 = l64 & 15;
    const int chunk = blockIdx.x;
    const int r0 = blockIdx.y * kHdxRows;
    const bool store_head = chunk == 0;

    // ---- loads ----
    // softmax inputs, staged in LDS with W2 (a load used only inside the
    // softmax branch would be issued there, a round trip late)
    const int64_t lab_t = labels[min(r0 + (t & (kHdxRows - 1)), batch - 1)];
    const float b2_t = b2[min(t & (CM - 1), classes - 1)];
    float v[kPerThread];
#pragma unroll
    for (int u = 0; u < kPerThread; ++u) {
        const int e = u * kHdxThreads + t;
        const int j = e / CM, c = e % CM;
        v[u] = W2[min(j, hidden - 1) * classes + min(c, classes - 1)];
    }
    // z operand a: H[r0 + i16][32w + 16g + 4q .. + 3]
    const float* harow = H + (int64_t)min(r0 + i16, batch - 1) * hidden;
    floatx4 ha[2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        ha[g] = *reinterpret_cast<const floatx4*>(harow + min(w * KZ + 16 * g + 4 * q, hidden - 4));
    }
    // G1's mask: H[r0 + 4q + r][16 (2w + tt) + i16]
    float hm[2][4];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            hm[tt][r] = H[(int64_t)min(r0 + 4 * q + r, batch - 1) * hidden +
                          min(16 * (2 * w + tt) + i16, hidden - 1)];
    // dX's column of this lane (its W1 fragments are loaded after the staging
    // barrier, below)
    const int ct4 = w % NCT;
    const int kh = w / NCT;
    const int col = chunk * kHdxCols + ct4 * 16 + i16;
    // element u * kHdxThreads + t is row u * kStageRows + t / CM, column t % CM
    constexpr int kStageRows = kHdxThreads / CM;
    static_assert(kHdxThreads % CM == 0 && kStageRows % 8 == 0, "staging rows step by 8");
    const int stage_at = head_w2_at<CM>(t / CM, t % CM);
#pragma unroll
    for (int u = 0; u < kPerThread; ++u) {
        const int j = u * kStageRows + t / CM, c = t % CM;
        w2s[stage_at + u * kStageRows * LR] = (j < hidden && c < classes) ? v[u] : 0.0f;
    }
    // every thread stores (threads with equal indices store equal values): a
    // store under a branch would pull its load into the branch
    lbls[t & (kHdxRows - 1)] = lab_t;
    b2s[t & (CM - 1)] = (t & (CM - 1)) < classes ? b2_t : 0.0f;
    __syncthreads();
    // dX operand b: W1[col][k0 .. k0 + 3].  Issued after the barrier, where
    // the head's own loads are in: issued at the start with them, these 64 KB
    // per block competed with them (16.52 -> 16.37 us per step), and issued
    // after the z products' barrier they arrived late for dX (16.64 us).
    const float* w1row = W1 + (int64_t)min(col, in_features - 1) * hidden;
    floatx4 wb[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        wb[g] = *reinterpret_cast<const floatx4*>(w1row + min(kh * KH + 16 * g + 4 * q, hidden - 4));
    }

    // ---- z = H W2: this wave's 32 hidden values ----
    const floatx4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    const bool row_in = r0 + i16 < batch;
    const float* zb = w2s + head_w2_at<CM>(4 * q, i16);   // + (k0 + s2) rows, 16 ct columns
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
        floatx4 zacc = zero4;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const int k0 = w * KZ + 16 * g;
            const floatx4 a = (row_in && k0 + 4 * q < hidden) ? ha[g] : zero4;
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2) {
                const float b = zb[(k0 + s2) * LR + 16 * ct];
                zacc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s2], b, zacc, 0, 0, 0);
            }
        }
        zred[w][ct][l64] = zacc;
    }
    __syncthreads();

    // ---- softmax and G2: wave r (< 4) takes register r of the tiles, so a
    // lane holds row 4q + r, class 16 ct + i16, and a DPP row of 16 lanes one
    // row of the batch ----
    if (w < 4) {
#pragma clang fp contract(off)
        const int r = w;
        float zc[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            float zz = zred[0][ct][l64][r];
#pragma unroll
            for (int ww = 1; ww < NW; ++ww) zz += zred[ww][ct][l64][r];
            zc[ct] = zz + b2s[16 * ct + i16];
        }
        const int row = r0 + 4 * q + r;
        const bool live = row < batch;
        float* g2row = g2s + head_w2_at<CM>(4 * q, i16) + r * LR;  // + 16 ct columns
        const int64_t label = lbls[4 * q + r];
        const bool valid = label >= 0 && label < classes;
        const float inv_b = 1.0f / (float)batch;
        float mx = -INFINITY;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            if (16 * ct + i16 < classes) mx = fmaxf(mx, zc[ct]);
        }
        mx = row16_max(mx);
        float ez[CT];
        float es = 0.0f;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            ez[ct] = 16 * ct + i16 < classes ? expf(zc[ct] - mx) : 0.0f;
            es += ez[ct];
        }
        const float inv_s = 1.0f / row16_sum(es);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            const int c = 16 * ct + i16;
            float pc = ez[ct] * inv_s;
            if (valid && c == label) pc -= 1.0f;
            const float gc = pc * inv_b;
            if (live && store_head && c < classes) {
                logits[(int64_t)row * classes + c] = zc[ct];
                G2[(int64_t)row * classes + c] = gc;
            }
            g2row[16 * ct] = (live && c < classes) ? gc : 0.0f;
        }
    }
    __syncthreads();

    // ---- G1 = (G2 W2^T) * [H > 0]: hidden tiles 2w and 2w + 1 ----
    const int frag_at = head_w2_at<CM>(i16, 4 * q);   // + 16 rows per tile, 16 g columns
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int j = 16 * (2 * w + tt) + i16;
        floatx4 gacc = zero4;
#pragma unroll
        for (int g = 0; g < CT; ++g) {
            const floatx4 a = *reinterpret_cast<const floatx4*>(g2s + frag_at + 16 * g);
            const floatx4 b = *reinterpret_cast<const floatx4*>(w2s + frag_at + 16 * (2 * w + tt) * LR + 16 * g);
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2) {
                gacc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s2], b[s2], gacc, 0, 0, 0);
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = r0 + 4 * q + r;
            const bool keep = row < batch && j < hidden;
            const float g1 = (keep && hm[tt][r] > 0.0f) ? gacc[r] : 0.0f;
            g1s[head_g1_at(4 * q, j) + r * kHdxG1Row] = g1;
            if (keep && store_head) G1[(int64_t)row * hidden + j] = g1;
        }
    }
    __syncthreads();

    // ---- dX tile: 16 rows x 16 columns per wave over its part of the hidden range ----
    floatx4 acc = zero4;
    const float* arow = g1s + head_g1_at(i16, 4 * q) + kh * KH;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const floatx4 a = *reinterpret_cast<const floatx4*>(arow + 16 * g);
        const floatx4 b = kh * KH + 16 * g + 4 * q < hidden ? wb[g] : zero4;
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s2], b[s2], acc, 0, 0, 0);
        }
    }
    if (kh > 0) red[kh - 1][ct4][l64] = acc;
    __syncthreads();
    if (kh == 0) {
#pragma unroll
        for (int p = 0; p < NKS - 1; ++p) acc += red[p][ct4][l64];
        if (col < in_features) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int orow = r0 + 4 * q + r;
                if (orow < batch) dX[(int64_t)orow * in_features + col] = acc[r];
            }
        }
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

// data[0 .. bytes) = 0: 16-byte stores over the aligned body, byte stores at
// the ends.  A kernel rather than hipMemsetAsync, so that a caller may capture
// it into a graph (a captured memset node gave wrong results on replays).
__global__ void zero_fill_kernel(unsigned char* __restrict__ data, int64_t head, int64_t n16,
                                 int64_t tail) {
    const int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    uint4* body = reinterpret_cast<uint4*>(data + head);
    for (int64_t e = i; e < n16; e += stride) body[e] = make_uint4(0u, 0u, 0u, 0u);
    if (i < head) data[i] = 0;
    if (i < tail) data[head + 16 * n16 + i] = 0;
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

template <int CM, int NH>
hipError_t launch_mlp_head_cfg(const float* H, const float* W2, const float* b2,
                               const int64_t* labels, float* logits, float* G2, float* G1,
                               float* part, int64_t batch, int64_t hidden, int64_t classes,
                               hipStream_t stream) {
    hipLaunchKernelGGL((mlp_head_kernel<CM, NH>), dim3((unsigned)head_blocks(batch)),
                       dim3(kBlock), 0, stream, H, W2, b2, labels, logits, G2, G1, part,
                       (int)batch, (int)hidden, (int)classes);
    return hipGetLastError();
}

hipError_t launch_mlp_head(const float* H, const float* W2, const float* b2,
                           const int64_t* labels, float* logits, float* G2, float* G1,
                           float* part, int64_t batch, int64_t hidden, int64_t classes,
                           hipStream_t stream) {
    if (!head_supported(hidden, classes) || batch < 1 || batch > INT32_MAX) {
        return hipErrorInvalidValue;
    }
    if (classes <= 16) {
        return hidden <= 256 ? launch_mlp_head_cfg<16, 8>(H, W2, b2, labels, logits, G2, G1,
                                                          part, batch, hidden, classes, stream)
                             : launch_mlp_head_cfg<16, 32>(H, W2, b2, labels, logits, G2, G1,
                                                           part, batch, hidden, classes, stream);
    }
    return hidden <= 256 ? launch_mlp_head_cfg<32, 8>(H, W2, b2, labels, logits, G2, G1, part,
                                                      batch, hidden, classes, stream)
                         : launch_mlp_head_cfg<32, 16>(H, W2, b2, labels, logits, G2, G1, part,
                                                       batch, hidden, classes, stream);
}

hipError_t launch_mlp_head_dx(const float* H, const float* W2, const float* b2,
                              const int64_t* labels, const float* W1, float* logits, float* G2,
                              float* G1, float* dX, int64_t batch, int64_t in_features,
                              int64_t hidden, int64_t classes, hipStream_t stream) {
    if (!head_dx_supported(batch, in_features, hidden, classes, H, W1)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((in_features + kHdxCols - 1) / kHdxCols),
                    (unsigned)((batch + kHdxRows - 1) / kHdxRows));
    if (classes <= 16) {
        hipLaunchKernelGGL((mlp_head_dx_kernel<1>), grid, dim3(kHdxThreads), 0, stream,
                           (int)batch, (int)in_features, (int)hidden, (int)classes, H, W2, b2,
                           labels, W1, logits, G2, G1, dX);
    } else {
        hipLaunchKernelGGL((mlp_head_dx_kernel<2>), grid, dim3(kHdxThreads), 0, stream,
                           (int)batch, (int)in_features, (int)hidden, (int)classes, H, W2, b2,
                           labels, W1, logits, G2, G1, dX);
    }
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

hipError_t launch_zero_fill(void* data, int64_t bytes, hipStream_t stream) {
    auto* p = static_cast<unsigned char*>(data);
    const int64_t head = std::min<int64_t>((16 - (reinterpret_cast<uintptr_t>(p) & 15u)) & 15u,
                                           bytes);
    const int64_t n16 = (bytes - head) / 16;
    const int64_t tail = bytes - head - 16 * n16;
    hipLaunchKernelGGL(zero_fill_kernel, dim3(std::max(1u, grid_for(n16, 4))), dim3(kBlock), 0,
                       stream, p, head, n16, tail);
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
