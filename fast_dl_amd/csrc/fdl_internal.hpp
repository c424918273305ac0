// Internal declarations shared by the HIP translation units of libfastdl_gemm.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace fdl {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

enum Epilogue : int {
    EPI_NONE = 0,
    EPI_BIAS = 1,
    EPI_BIAS_RELU = 2,
    EPI_RELU = 3,
    EPI_RELU_GRAD = 4,
    // Internal (not in the C-ABI enum): C = v and upd[i][j] -= lr * v, i.e. a
    // weight-gradient GEMM that also applies the SGD step to the weight.
    EPI_SGD = 5,
};

// One strided-batched GEMM problem, already validated on the host.
// Sizes fit in int32 (the reference's own API is int-sized); offsets are int64.
struct GemmParams {
    const float* A;
    const float* B;
    float* C;
    const float* bias;  // length N, or null
    const float* aux;   // same layout as C (ldc, strideC), or null
    float* upd;         // EPI_SGD: parameter updated in place, same layout as C
    float lr;           // EPI_SGD: learning rate
    int64_t lda, ldb, ldc;
    int64_t strideA, strideB, strideC;
    int M, N, K;
    int epilogue;
};

// Kernel families; the host dispatcher picks one per call.  Values match
// fdl_kernel in include/fastdl_gemm.h.
enum class GemmKernel : int {
    Tiled128 = 0,     // 128x128x16 tile, 4 waves of 64x64
    Tiled64 = 1,      // 64x64x16 tile, 4 waves of 32x32
    SplitK32 = 2,     // 32x32 output tile, K split over the waves of a block
    Skinny = 3,       // VALU strip kernel for M <= 8 with B not transposed
    Tiled256 = 4,     // 256x256x16 tile, 8 waves of 128x64
    Tiled256x128 = 5, // 256x128x16 tile, 8 waves of 64x64
    Tiled128W8 = 6,   // 128x128x16 tile, 8 waves of 32x64
    SplitK16 = 7,     // 16x16 output tile (16x16x4 MFMA), K split over waves
    Dma256 = 8,       // 256x256x16 tile, global -> LDS copies without VGPR staging
    Dma128 = 9,       // 128x128x32 tile, global -> LDS copies, two blocks per CU
    Dma64 = 10,       // 64x64x64 tile, global -> LDS copies, two sets of four 32x32 waves
    Dma128W8 = 11,    // 128x128x64 tile, global -> LDS copies, eight waves of 64x32
    Dma64U = 12,      // Dma64 with 4-byte copies (any K, leading dimension, alignment)
    Dma128W8U = 13,   // Dma128W8 with 4-byte copies
    Dma64S = 14,      // 64x64x16 tile, four K-tiles in flight, four 32x32 waves
    Dma96x32U = 15,   // 96x32x64 tile, 4-byte copies, four sets of three 32x32 waves
    Auto = -1,
};

// Whether a direct-to-LDS kernel can run this problem.  The 16-byte-copy
// ones (Dma256, Dma128, Dma64, Dma128W8) need K a multiple of 4 and both
// operands 16-byte vectorisable; the 4-byte-copy ones (Dma64U, Dma128W8U)
// need leading dimensions up to 2^24 and 4-byte-aligned pointers.
bool dma_supported(GemmKernel kernel, const GemmParams& p, bool transA, bool transB,
                   int64_t batch);

// One job of a grouped launch (launch_group): a split-K GEMM (32x32 output
// tiles, four waves per block, any epilogue), a column sum with the bias SGD
// step, an SGD update p -= lr * g, the final reduction of the MLP head's
// partial records (xent_finalize_body), or the head's loss, db2 and b2 step
// from its stored logits and G2 (head_finalize_body).
struct GroupJob {
    // kGemm16: the same GEMM on 16x16 output tiles (v_mfma_f32_16x16x4_f32), for
    // outputs at most 16 wide, where a 32x32 tile would waste most of its work.
    enum Kind { kGemm, kColsumSgd, kSgd, kXentFinalize, kHeadFinalize, kGemm16 };
    Kind kind = kGemm;
    GemmParams p{};              // kGemm, kGemm16
    bool ta = false, tb = false;
    const float* x = nullptr;    // kColsumSgd: rows x cols input; kSgd: gradient;
                                 // kXentFinalize: the partial records;
                                 // kHeadFinalize: logits
    const float* x2 = nullptr;   // kHeadFinalize: G2
    const int64_t* labels = nullptr;  // kHeadFinalize
    float* out = nullptr;        // kColsumSgd, kXentFinalize, kHeadFinalize: column sums (db)
    float* out2 = nullptr;       // kXentFinalize, kHeadFinalize: loss
    float* param = nullptr;      // kColsumSgd, kSgd, k*Finalize: the parameter updated
    float lr = 0.0f;
    int64_t rows = 0, cols = 0;  // kSgd: rows is the element count;
                                 // kXentFinalize: records, classes;
                                 // kHeadFinalize: batch, classes (<= 32)
};

// Runs n (2 to 4) independent jobs in one launch, job 0 on the first blocks
// of the grid.  Supported sequences are the ones the MLP step uses:
// (NT GEMM, TN GEMM), (NT GEMM, column sum), (TN GEMM, SGD),
// (NT GEMM, column sum, TN GEMM, finalize), (column sum, TN GEMM,
// finalize) and (TN GEMM, column sum, TN GEMM, head finalize), the second TN
// GEMM of the last either kind; others return hipErrorInvalidValue.
hipError_t launch_group(const GroupJob* jobs, int n, hipStream_t stream);
inline hipError_t launch_group2(const GroupJob& j0, const GroupJob& j1, hipStream_t stream) {
    const GroupJob jobs[2] = {j0, j1};
    return launch_group(jobs, 2, stream);
}

// K-split form of the skinny family (sgemm.hip): B's columns in bands of
// kSplitBand, K in `slices` slices of `rows` rows, one block per (band,
// slice) writing an mr x kSplitBand partial, then a pass adding the slices.
// slices == 0: the problem does not take the split (not one skinny problem
// with B not transposed and N % 4 == 0, or too little of B to pay for the
// second pass).
constexpr int kSplitBand = 256;
constexpr int kSplitMaxSlices = 64;
struct SkinnySplit {
    int mr = 0, bands = 0, slices = 0, rows = 0;
    size_t bytes = 0;  // workspace the partials take
};
SkinnySplit skinny_split_plan(const GemmParams& p, bool transA, bool transB, int64_t batch);

// Launches `batch` problems (grid.y indexes the batch).  Returns a hipError_t.
// With a workspace of at least skinny_split_plan(...).bytes, a problem the
// skinny family runs takes the K-split form (when B is 16-byte
// vectorisable); the workspace is written on `stream`.
hipError_t launch_sgemm(const GemmParams& p, bool transA, bool transB,
                        int64_t batch, GemmKernel kernel, hipStream_t stream,
                        float* workspace = nullptr, size_t workspace_bytes = 0);

// Kernel the dispatcher would pick for this problem.
GemmKernel choose_kernel(const GemmParams& p, bool transA, bool transB,
                         int64_t batch);

const char* kernel_name(GemmKernel k);

// Elementwise / row kernels (mlp_kernels.hip).
hipError_t launch_add_row_bias(float* out, const float* bias, int64_t rows,
                               int64_t cols, hipStream_t stream);
hipError_t launch_relu(const float* in, float* out, int64_t n,
                       hipStream_t stream);
hipError_t launch_relu_backward(const float* g, const float* act, float* out,
                                int64_t n, hipStream_t stream);
hipError_t launch_colsum(const float* x, float* out, int64_t rows, int64_t cols,
                         hipStream_t stream);
// out = column sums of x, then param -= lr * out (param may be null).
hipError_t launch_colsum_sgd(const float* x, float* out, float* param, float lr,
                             int64_t rows, int64_t cols, hipStream_t stream);
hipError_t launch_softmax(const float* in, float* out, int64_t rows,
                          int64_t cols, hipStream_t stream);
hipError_t launch_softmax_xent(const float* logits, const int64_t* labels,
                               float* loss, float* grad, int64_t batch,
                               int64_t classes, hipStream_t stream);
// As launch_softmax_xent, and also db = column sums of the gradient and
// bparam -= lr * db (the bias step of the layer that produced the logits).
// Needs grad, db and bparam; classes <= kXentFusedMaxClasses.
constexpr int kXentFusedMaxClasses = 32;
hipError_t launch_softmax_xent_db_sgd(const float* logits, const int64_t* labels,
                                      float* loss, float* grad, float* db, float* bparam,
                                      float lr, int64_t batch, int64_t classes,
                                      hipStream_t stream);
// The MLP step's head, kHeadRows rows per block: logits = H W2 + b2, loss
// and G2 = dL/dlogits as launch_softmax_xent, G1 = (G2 W2^T) * [H > 0], and
// each block's partial record (column sums of its G2 rows, then its loss
// share) at part + block * (classes + 1).  xent_finalize_body reduces the
// records.  W2 is staged in LDS with rows padded to 16 or 32 classes, which
// bounds the shapes: classes <= 16 with hidden <= 1024, or classes <= 32
// with hidden <= 512.
constexpr int kHeadRows = 8;
inline bool head_supported(int64_t hidden, int64_t classes) {
    return hidden >= 1 && classes >= 1 &&
           ((classes <= 16 && hidden <= 1024) || (classes <= 32 && hidden <= 512));
}
inline int64_t head_blocks(int64_t batch) { return (batch + kHeadRows - 1) / kHeadRows; }
hipError_t launch_mlp_head(const float* H, const float* W2, const float* b2,
                           const int64_t* labels, float* logits, float* G2, float* G1,
                           float* part, int64_t batch, int64_t hidden, int64_t classes,
                           hipStream_t stream);
// The head fused with dX = G1 W1^T (mlp_head_dx_kernel): kHdxRows rows and
// kHdxCols columns of dX per block, each block recomputing the head for its
// rows; the blocks of the first column chunk store logits, G2 and G1.  No
// loss and no records: the loss, db2 and the b2 step come from the stored
// logits and G2 (head_finalize_body).  Needs hidden <= 256 with hidden % 4
// == 0, classes <= 32, and H and W1 16-byte aligned.
constexpr int kHdxRows = 16;
constexpr int kHdxCols = 64;
inline bool head_dx_supported(int64_t batch, int64_t in_features, int64_t hidden,
                              int64_t classes, const float* H, const float* W1) {
    return batch >= 1 && (batch + kHdxRows - 1) / kHdxRows <= 65535 && in_features >= 1 &&
           in_features <= INT32_MAX && hidden >= 4 && hidden <= 256 && hidden % 4 == 0 &&
           classes >= 1 && classes <= 32 && (reinterpret_cast<uintptr_t>(H) & 15u) == 0 &&
           (reinterpret_cast<uintptr_t>(W1) & 15u) == 0;
}
hipError_t launch_mlp_head_dx(const float* H, const float* W2, const float* b2,
                              const int64_t* labels, const float* W1, float* logits, float* G2,
                              float* G1, float* dX, int64_t batch, int64_t in_features,
                              int64_t hidden, int64_t classes, hipStream_t stream);
hipError_t launch_sgd(float* param, const float* grad, float lr, int64_t n,
                      hipStream_t stream);
// Up to four (param, grad, n) updates in one launch.
hipError_t launch_sgd_multi(int count, float* const* params,
                            const float* const* grads, const int64_t* sizes,
                            float lr, hipStream_t stream);
// data[0 .. bytes) = 0 by a kernel (capturable, unlike a memset node).
hipError_t launch_zero_fill(void* data, int64_t bytes, hipStream_t stream);
hipError_t launch_fill_uniform(float* data, int64_t n, float low, float high,
                               uint64_t seed, hipStream_t stream);
hipError_t launch_fill_normal(float* data, int64_t n, float mean, float stddev,
                              uint64_t seed, hipStream_t stream);

// IDX batch gather (data_kernels.hip), arguments as fdl_idx_gather.  The
// 4-pixel vector path needs row_bytes % 4 == 0, images 4-byte and x 16-byte
// aligned; anything else takes the byte path.
bool idx_gather_vectorized(const uint8_t* images, int64_t row_bytes, const float* x);
hipError_t launch_idx_gather(const uint8_t* images, const uint8_t* labels, int64_t count,
                             int64_t row_bytes, const int64_t* index, int64_t batch,
                             float divisor, float* x, int64_t* y, hipStream_t stream);

}  // namespace fdl
