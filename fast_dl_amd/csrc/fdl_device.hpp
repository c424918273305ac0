// Device bodies shared by standalone kernels and grouped launches.  Each body
// takes its block index (and block count) explicitly so that a grouped kernel
// can run it on a sub-range of its grid.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace fdl {

// Waits until no vector-memory operation of this wave is outstanding
// (s_waitcnt vmcnt(0), lgkmcnt and expcnt unconstrained).  Placed before a
// run of stores whose values use operands loaded early: where the compiler
// cannot prove those loads have landed (a path that skips the main loop
// merges in), it waits for them before each store, and since stores count in
// vmcnt with the loads, each of those waits also waits for the stores just
// issued.  On the main path nothing is outstanding here, so this costs nothing.
__device__ __forceinline__ void wait_vmem_idle() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Column sums of a row-major rows x cols matrix, 32 columns per block and 8
// row groups per column (256 threads).  Row groups are added in group order,
// so the result is deterministic.  With `param`, the block also applies
// param[c] -= lr * sum (the SGD step of a bias).
constexpr int kColsumCols = 32;
constexpr int kColsumGroups = 8;
constexpr int kColsumThreads = kColsumCols * kColsumGroups;

__device__ __forceinline__ void colsum_body(const float* __restrict__ x, float* __restrict__ out,
                                            float* __restrict__ param, float lr, int64_t rows,
                                            int64_t cols, int block) {
#pragma clang fp contract(off)
    __shared__ float part[kColsumGroups][kColsumCols];
    const int cl = threadIdx.x % kColsumCols;
    const int grp = threadIdx.x / kColsumCols;
    const int64_t c = block * (int64_t)kColsumCols + cl;
    const int64_t cc = c < cols ? c : cols - 1;  // clamped: loads stay in bounds
    // The parameter's value, fetched now (`param` is the same on every lane, so
    // this is a scalar branch): loaded after the sums it costs a second round
    // trip to memory at the end of the block.
    float pv = 0.0f;
    if (param) pv = param[cc];
    // Rows are added in order (grp, grp + 8, grp + 16, ...); the loads of
    // 32 of them are in flight at once, so a 256-row matrix costs one
    // round trip to memory instead of four.
    float s = 0.0f;
    int64_t r = grp;
    for (; r + 31 * kColsumGroups < rows; r += 32 * kColsumGroups) {
        float v[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) v[u] = x[(r + u * kColsumGroups) * cols + cc];
#pragma unroll
        for (int u = 0; u < 32; ++u) s += v[u];
    }
    for (; r + 7 * kColsumGroups < rows; r += 8 * kColsumGroups) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = x[(r + u * kColsumGroups) * cols + cc];
#pragma unroll
        for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; r < rows; r += kColsumGroups) s += x[r * cols + cc];
    part[grp][cl] = s;
    __syncthreads();
    if (grp == 0 && c < cols) {
        float t = part[0][cl];
#pragma unroll
        for (int g = 1; g < kColsumGroups; ++g) t += part[g][cl];
        const float step = lr * t;
        const float np = pv - step;
        wait_vmem_idle();
        out[c] = t;
        if (param) param[c] = np;
    }
}

// Final reduction of the MLP head's per-block partials (one block): part holds
// nparts records of classes + 1 floats, the block's bias-gradient column sums
// then its loss.  Records are added in block order (deterministic); then
// db[c] = sum, bparam[c] -= lr * sum, loss[0] = sum of the loss partials.
__device__ __forceinline__ void xent_finalize_body(const float* __restrict__ part, int nparts,
                                                   int classes, float* __restrict__ loss,
                                                   float* __restrict__ db,
                                                   float* __restrict__ bparam, float lr) {
#pragma clang fp contract(off)
    const int t = threadIdx.x;
    if (t > classes) return;
    const int stride = classes + 1;
    // Records in block order, 32 of them in flight at once.
    float s = 0.0f;
    int b = 0;
    for (; b + 32 <= nparts; b += 32) {
        float v[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) v[u] = part[(b + u) * stride + t];
#pragma unroll
        for (int u = 0; u < 32; ++u) s += v[u];
    }
    for (; b + 8 <= nparts; b += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = part[(b + u) * stride + t];
#pragma unroll
        for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; b < nparts; ++b) s += part[b * stride + t];
    if (t < classes) {
        db[t] = s;
        const float step = lr * s;
        bparam[t] = bparam[t] - step;
    } else if (loss) {
        loss[0] = s;
    }
}

// The MLP head's reductions from its stored outputs, split over two blocks
// of 256 threads (classes <= kColsumCols) so that their loads proceed side by
// side.  Block `which` = 0: the loss, each row's share
// (logf(sum_c expf(z_c - max)) + max - z_label) / rows computed from its
// stored logits z as the head computes it (classes in order; rows with a
// label outside [0, classes) add nothing); a thread takes rows t, t + 256,
// ..., summed in row order, then over each wave by a fixed exchange tree and
// over the waves in order.  Block 1: db = column sums of G with the bias step
// bparam -= lr * db, the sums and their order exactly as colsum_body's.  Each
// block issues all its loads of the first 256 rows (the rows' logits and
// labels; the bias and 32 rows of G per thread) at clamped addresses before
// it uses any.
template <int CM>
__device__ __forceinline__ void head_finalize_body(int which, const float* __restrict__ logits,
                                                   const float* __restrict__ g,
                                                   const int64_t* __restrict__ labels,
                                                   int64_t rows, int64_t classes,
                                                   float* __restrict__ loss,
                                                   float* __restrict__ db,
                                                   float* __restrict__ bparam, float lr) {
#pragma clang fp contract(off)
    static_assert(CM <= kColsumCols, "one block of column sums");
    __shared__ float part[kColsumGroups][kColsumCols];
    __shared__ float wpart[kColsumThreads / 64];
    constexpr int kFirst = 32;  // column-sum rows per thread issued up front
    const int t = threadIdx.x;
    if (which == 0) {
        if (!loss) return;
        const int64_t r0 = t < rows ? t : rows - 1;
        float z[CM];
#pragma unroll
        for (int c = 0; c < CM; ++c) z[c] = logits[r0 * classes + (c < classes ? c : classes - 1)];
        const int64_t label0 = labels[r0];
        const float inv_b = 1.0f / (float)rows;
        float s = 0.0f;
        for (int64_t r = t; r < rows; r += kColsumThreads) {
            int64_t label = label0;
            if (r != t) {  // rows past the first 256: load them here
                label = labels[r];
#pragma unroll
                for (int c = 0; c < CM; ++c) z[c] = logits[r * classes + (c < classes ? c : classes - 1)];
            }
            // `classes` is the same on every lane: the tests below are
            // scalar branches, so padded classes cost no expf
            float mx = z[0];
#pragma unroll
            for (int c = 1; c < CM; ++c) {
                if (c < classes) mx = fmaxf(mx, z[c]);
            }
            float e = 0.0f;
            float zl = 0.0f;
#pragma unroll
            for (int c = 0; c < CM; ++c) {
                if (c < classes) {
                    e += expf(z[c] - mx);
                    zl = c == label ? z[c] : zl;
                }
            }
            if (label >= 0 && label < classes) s += (logf(e) + mx - zl) * inv_b;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
        if ((t & 63) == 0) wpart[t >> 6] = s;
        __syncthreads();
        if (t == 0) {
            float l = wpart[0];
#pragma unroll
            for (int i = 1; i < kColsumThreads / 64; ++i) l += wpart[i];
            loss[0] = l;
        }
        return;
    }

    // Column sums, rows grp, grp + 8, ... in order (colsum_body's order).
    const int cl = t % kColsumCols;
    const int grp = t / kColsumCols;
    const int64_t cc = cl < classes ? cl : classes - 1;
    const float pv = bparam ? bparam[cc] : 0.0f;
    float gv[kFirst];
#pragma unroll
    for (int u = 0; u < kFirst; ++u) {
        const int64_t r = grp + (int64_t)u * kColsumGroups;
        gv[u] = g[(r < rows ? r : rows - 1) * classes + cc];
    }
    float cs = 0.0f;
#pragma unroll
    for (int u = 0; u < kFirst; ++u) {
        if (grp + (int64_t)u * kColsumGroups < rows) cs += gv[u];
    }
    int64_t r = grp + (int64_t)kFirst * kColsumGroups;
    for (; r + 31 * kColsumGroups < rows; r += 32 * kColsumGroups) {
        float v[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) v[u] = g[(r + u * kColsumGroups) * classes + cc];
#pragma unroll
        for (int u = 0; u < 32; ++u) cs += v[u];
    }
    for (; r + 7 * kColsumGroups < rows; r += 8 * kColsumGroups) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = g[(r + u * kColsumGroups) * classes + cc];
#pragma unroll
        for (int u = 0; u < 8; ++u) cs += v[u];
    }
    for (; r < rows; r += kColsumGroups) cs += g[r * classes + cc];
    part[grp][cl] = cs;
    __syncthreads();
    if (grp == 0 && cl < classes) {
        float tsum = part[0][cl];
#pragma unroll
        for (int q = 1; q < kColsumGroups; ++q) tsum += part[q][cl];
        const float step = lr * tsum;
        const float np = pv - step;
        wait_vmem_idle();
        db[cl] = tsum;
        if (bparam) bparam[cl] = np;
    }
}

// p[i] -= lr * g[i] over a grid-stride range; the product is rounded before
// the subtraction (no FMA contraction), as in the reference's host update.
__device__ __forceinline__ void sgd_body(float* __restrict__ p, const float* __restrict__ g,
                                         float lr, int64_t n, int block, int nblocks) {
#pragma clang fp contract(off)
    for (int64_t idx = block * (int64_t)blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)nblocks * blockDim.x) {
        p[idx] -= lr * g[idx];
    }
}

}  // namespace fdl
