// IDX batch gather: byte rows resident in HBM -> fp32 rows and int64 labels
// (fdl_idx_gather in include/fastdl_data.h).
//
// HBM-bound streaming work: 1 byte read and 4 bytes written per pixel, plus
// one 8-byte index per row.  The per-chunk work is a few instructions (a
// quotient-table read per pixel, one integer division per thread) so that the
// vector ALU stays below the memory rate.  Rows whose length is a multiple of
// 4 bytes take the vector path: a chunk is 4 pixels, one dword load and one
// 16-byte store, so a wave's loads cover 256 contiguous bytes and its stores
// 1 KiB.  Each thread keeps kUnroll chunks in flight.  Other rows take the
// byte path with the same structure and 1-pixel chunks.  Outputs of 32 MiB
// and more are written with streaming stores.
#include "fdl_internal.hpp"

#include <hip/hip_runtime.h>

#include <cstdint>

namespace fdl {

namespace {

constexpr int kGatherThreads = 256;
constexpr int kUnroll = 4;
constexpr int kChunksPerBlock = kGatherThreads * kUnroll;

template <int V> struct Pixels;
template <> struct Pixels<4> { using load_t = uint32_t; using store_t = float4; };
template <> struct Pixels<1> { using load_t = uint8_t; using store_t = float; };

// Pixel bytes become quotients through a 256-entry table in LDS that each
// block fills with one IEEE division per thread: the same bits as dividing
// every pixel, at a table read per pixel instead of a division.
static_assert(kGatherThreads == 256, "one table entry per thread");

__device__ __forceinline__ float4 convert(uint32_t w, const float* lut) {
    return make_float4(lut[w & 0xffu], lut[(w >> 8) & 0xffu], lut[(w >> 16) & 0xffu],
                       lut[w >> 24]);
}

__device__ __forceinline__ float convert(uint8_t p, const float* lut) { return lut[p]; }

// Streaming (non-temporal) stores for outputs far larger than the caches: a
// whole-set conversion's rows are not read back soon, and keeping them out of
// L2 and the Infinity Cache was measured 16-20% faster (60000x784 set:
// 40.8 -> 34.4 us).  A batch is stored normally, so that the GEMM reading it
// next finds it in L2.
constexpr int64_t kStreamingStoreBytes = int64_t(32) << 20;

typedef float nt_float4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ void store_pixels(float4* p, float4 v) {
    if constexpr (NT) {
        const nt_float4 w = {v.x, v.y, v.z, v.w};
        __builtin_nontemporal_store(w, reinterpret_cast<nt_float4*>(p));
    } else {
        *p = v;
    }
}

template <bool NT>
__device__ __forceinline__ void store_pixels(float* p, float v) {
    if constexpr (NT) {
        __builtin_nontemporal_store(v, p);
    } else {
        *p = v;
    }
}

template <class T> __device__ __forceinline__ T zero_pixels();
template <> __device__ __forceinline__ float4 zero_pixels<float4>() { return make_float4(0.f, 0.f, 0.f, 0.f); }
template <> __device__ __forceinline__ float zero_pixels<float>() { return 0.0f; }

// Chunk c of the output is (row b = c / row_chunks, chunk j = c % row_chunks).
// A thread's chunks are kGatherThreads apart, so after one division the next
// (b, j) follow by adding (step_q, step_r) = divmod(kGatherThreads,
// row_chunks) with a carry.  IdxT is uint32_t when every chunk number the
// grid reaches fits in it.  Blocks also cover the labels: thread g < batch
// writes y[g].
template <int V, class IdxT, bool NT>
__global__ void __launch_bounds__(kGatherThreads)
idx_gather_kernel(const typename Pixels<V>::load_t* __restrict__ images,
                  const uint8_t* __restrict__ labels, int64_t count, IdxT row_chunks,
                  IdxT step_q, IdxT step_r, const int64_t* __restrict__ index, IdxT batch,
                  float divisor, typename Pixels<V>::store_t* __restrict__ x,
                  int64_t* __restrict__ y) {
    using load_t = typename Pixels<V>::load_t;
    using store_t = typename Pixels<V>::store_t;
    if (x != nullptr) {
        __shared__ float lut[256];
        lut[threadIdx.x] = static_cast<float>(threadIdx.x) / divisor;
        __syncthreads();
        // total >= 1 here: x is non-null only for rows of at least one chunk.
        // Loads are unconditional, at addresses clamped into the inputs, so
        // that all kUnroll index loads and then all kUnroll pixel loads are in
        // flight together; out-of-range results are discarded after the load.
        const IdxT total = batch * row_chunks;
        const IdxT base = static_cast<IdxT>(blockIdx.x) * kChunksPerBlock + threadIdx.x;
        const IdxT c0 = base < total ? base : total - 1;
        IdxT b = c0 / row_chunks;
        IdxT jj = c0 - b * row_chunks;
        int64_t r[kUnroll];
        IdxT j[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            if (u > 0) {
                b += step_q;
                jj += step_r;
                if (jj >= row_chunks) {
                    jj -= row_chunks;
                    ++b;
                }
            }
            const IdxT bc = b < batch ? b : batch - 1;  // chunks past the end: any valid row
            j[u] = jj;
            r[u] = index != nullptr ? index[bc] : static_cast<int64_t>(bc);
        }
        load_t w[kUnroll] = {};
        bool ok[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) ok[u] = r[u] >= 0 && r[u] < count;
        if (count > 0) {  // count == 0 leaves no row to clamp to: nothing is loaded
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int64_t rr = ok[u] ? r[u] : 0;
                w[u] = images[rr * static_cast<int64_t>(row_chunks) + j[u]];
            }
        }
        store_t v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) v[u] = ok[u] ? convert(w[u], lut) : zero_pixels<store_t>();
        // Every block but the last stores without per-chunk branches, which
        // keeps the stores back to back (a branch around each would make the
        // next one wait for the previous store's completion count).
        if ((static_cast<IdxT>(blockIdx.x) + 1) * kChunksPerBlock <= total) {
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) store_pixels<NT>(&x[base + static_cast<IdxT>(u) * kGatherThreads], v[u]);
        } else {
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const IdxT c = base + static_cast<IdxT>(u) * kGatherThreads;
                if (c < total) store_pixels<NT>(&x[c], v[u]);
            }
        }
    }
    if (y != nullptr) {
        const IdxT g = static_cast<IdxT>(blockIdx.x) * kGatherThreads + threadIdx.x;
        if (g < batch) {
            const int64_t r = index != nullptr ? index[g] : static_cast<int64_t>(g);
            y[g] = (r >= 0 && r < count) ? static_cast<int64_t>(static_cast<int8_t>(labels[r])) : -1;
        }
    }
}

template <int V, class IdxT, bool NT>
hipError_t launch_gather(int64_t blocks, const uint8_t* images, const uint8_t* labels,
                         int64_t count, int64_t row_bytes, const int64_t* index, int64_t batch,
                         float divisor, float* x, int64_t* y, hipStream_t stream) {
    using load_t = typename Pixels<V>::load_t;
    using store_t = typename Pixels<V>::store_t;
    const int64_t row_chunks = row_bytes / V;
    // row_chunks may be 0 only when x is null (labels only); the steps are then unused.
    const int64_t step_q = row_chunks > 0 ? kGatherThreads / row_chunks : 0;
    const int64_t step_r = row_chunks > 0 ? kGatherThreads % row_chunks : 0;
    hipLaunchKernelGGL((idx_gather_kernel<V, IdxT, NT>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kGatherThreads), 0, stream, reinterpret_cast<const load_t*>(images),
                       labels, count, static_cast<IdxT>(row_chunks), static_cast<IdxT>(step_q),
                       static_cast<IdxT>(step_r), index, static_cast<IdxT>(batch), divisor,
                       reinterpret_cast<store_t*>(x), y);
    return hipGetLastError();
}

template <int V>
hipError_t launch_gather_v(const uint8_t* images, const uint8_t* labels, int64_t count,
                           int64_t row_bytes, const int64_t* index, int64_t batch, float divisor,
                           float* x, int64_t* y, hipStream_t stream) {
    const int64_t chunks = batch * (row_bytes / V);
    const int64_t pixel_blocks = x ? (chunks + kChunksPerBlock - 1) / kChunksPerBlock : 0;
    const int64_t label_blocks = y ? (batch + kGatherThreads - 1) / kGatherThreads : 0;
    const int64_t blocks = pixel_blocks > label_blocks ? pixel_blocks : label_blocks;
    if (blocks == 0) return hipSuccess;
    if (blocks > INT32_MAX) return hipErrorInvalidConfiguration;
    // 32-bit chunk arithmetic when every thread's largest chunk number fits.
    const bool small = blocks * kChunksPerBlock <= static_cast<int64_t>(UINT32_MAX);
    if (x != nullptr && batch * row_bytes * 4 >= kStreamingStoreBytes) {
        return small ? launch_gather<V, uint32_t, true>(blocks, images, labels, count, row_bytes,
                                                        index, batch, divisor, x, y, stream)
                     : launch_gather<V, uint64_t, true>(blocks, images, labels, count, row_bytes,
                                                        index, batch, divisor, x, y, stream);
    }
    return small ? launch_gather<V, uint32_t, false>(blocks, images, labels, count, row_bytes,
                                                     index, batch, divisor, x, y, stream)
                 : launch_gather<V, uint64_t, false>(blocks, images, labels, count, row_bytes,
                                                     index, batch, divisor, x, y, stream);
}

}  // namespace

bool idx_gather_vectorized(const uint8_t* images, int64_t row_bytes, const float* x) {
    return row_bytes % 4 == 0 && reinterpret_cast<uintptr_t>(images) % 4 == 0 &&
           reinterpret_cast<uintptr_t>(x) % 16 == 0;
}

hipError_t launch_idx_gather(const uint8_t* images, const uint8_t* labels, int64_t count,
                             int64_t row_bytes, const int64_t* index, int64_t batch,
                             float divisor, float* x, int64_t* y, hipStream_t stream) {
    if (batch == 0) return hipSuccess;
    if (row_bytes == 0) x = nullptr;
    if (x == nullptr || idx_gather_vectorized(images, row_bytes, x)) {
        return launch_gather_v<4>(images, labels, count, row_bytes, index, batch, divisor, x, y,
                                  stream);
    }
    return launch_gather_v<1>(images, labels, count, row_bytes, index, batch, divisor, x, y,
                              stream);
}

}  // namespace fdl
