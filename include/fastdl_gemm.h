/*
 * fastdl_gemm.h -- C-ABI of the MI355X (gfx950) fp32 GEMM path.
 *
 * Plain C: pointers, sizes and status codes only.  Every pointer argument that
 * names a matrix or vector is a device pointer (HBM) on the calling thread's
 * current HIP device.  `stream` is a hipStream_t passed as void*; NULL means
 * the device's null stream, which is what the reference's implicit
 * legacy-default-stream launches used.
 *
 * No entry point allocates device memory and none throws.  All but the
 * graph create/destroy pair (which build host-side HIP graph objects) allocate
 * no host memory either, and all others are asynchronous with respect to the
 * host: they only validate arguments and enqueue kernels.  A non-zero return is one of the negative fdl_status
 * codes; fdl_last_error() returns a message for the last failure on the
 * calling thread.
 *
 * Layout convention: row-major everywhere, as in the reference.  For the
 * general entry point, with op(X) = X or X^T:
 *
 *   C[b][i][j] = epi( sum_k op(A)[b][i][k] * op(B)[b][k][j] ,  i, j )
 *
 *   op(A)[i][k] = A[i*lda + k]  (transA == FDL_OP_N)  A holds M x K
 *               = A[k*lda + i]  (transA == FDL_OP_T)  A holds K x M
 *   op(B)[k][j] = B[k*ldb + j]  (transB == FDL_OP_N)  B holds K x N
 *               = B[j*ldb + k]  (transB == FDL_OP_T)  B holds N x K
 *
 * C is overwritten (beta = 0), as cublasSgemm was called with beta = 0 in
 * the reference (src/kernels/cuda/gemm.cu:172-175).
 */
#ifndef FASTDL_GEMM_H
#define FASTDL_GEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum fdl_status {
    FDL_SUCCESS = 0,
    FDL_ERROR_INVALID_VALUE = -1,   /* bad size, leading dimension, pointer or enum */
    FDL_ERROR_NOT_SUPPORTED = -2,   /* valid request this build does not implement */
    FDL_ERROR_LAUNCH = -3,          /* kernel launch failed (hipGetLastError) */
    FDL_ERROR_RUNTIME = -4          /* other HIP runtime failure */
} fdl_status;

typedef enum fdl_operation {
    FDL_OP_N = 0,
    FDL_OP_T = 1
} fdl_operation;

/* Epilogue applied to each accumulated element v = sum_k(...) at (i, j). */
typedef enum fdl_epilogue {
    FDL_EPILOGUE_NONE = 0,       /* C = v                                      */
    FDL_EPILOGUE_BIAS = 1,       /* C = v + bias[j]                            */
    FDL_EPILOGUE_BIAS_RELU = 2,  /* C = fmaxf(0, v + bias[j])                  */
    FDL_EPILOGUE_RELU = 3,       /* C = fmaxf(0, v)                            */
    FDL_EPILOGUE_RELU_GRAD = 4   /* C = aux[i][j] > 0 ? v : 0  (ReLU backward; */
                                 /*     aux has C's ldc and strideC)           */
} fdl_epilogue;

/*
 * General strided-batched fp32 GEMM with optional fused epilogue.
 *
 * Replaces cublasSgemm in launch_gemm_cublas (src/kernels/cuda/gemm.cu:166-177)
 * and the separate add_row_bias pass that ops::linear runs after it
 * (src/ops/Linear.cpp:38-44, src/kernels/cuda/bias.cu:5-12).  Transposed
 * operands serve the NT / TN products of linear backward
 * (legacy/src/ops/Layers.cpp:36,40).
 *
 * M, N, K >= 0; batch >= 0 (0 or an empty C is a no-op, K == 0 gives
 * C = epi(0)).  lda >= max(1, columns of A as stored), same for ldb, ldc.
 * Strides are in elements and may be 0 (broadcast), except strideC which
 * must be >= M*ldc when batch > 1 so that batches do not overlap.
 * bias (length N, shared by every batch) is required for the BIAS epilogues;
 * aux is required for RELU_GRAD.
 */
int fdl_sgemm_ex(int transA, int transB,
                 int64_t M, int64_t N, int64_t K,
                 const float* A, int64_t lda, int64_t strideA,
                 const float* B, int64_t ldb, int64_t strideB,
                 float* C, int64_t ldc, int64_t strideC,
                 int64_t batch,
                 const float* bias, const float* aux, int epilogue,
                 void* stream);

/* Kernel families behind fdl_sgemm_ex (what GemmAlgo selected in the
 * reference, include/dl/kernels/gemm.hpp:7-12; the set is this build's own). */
typedef enum fdl_kernel {
    FDL_KERNEL_AUTO = -1,      /* size heuristic (what fdl_sgemm_ex uses)       */
    FDL_KERNEL_TILED128 = 0,   /* 128x128x16 LDS double-buffered MFMA tile, 4 waves */
    FDL_KERNEL_TILED64 = 1,    /* 64x64x16 LDS double-buffered MFMA tile, 4 waves   */
    FDL_KERNEL_SPLITK32 = 2,   /* 32x32 MFMA tile, K split over 8 waves              */
    FDL_KERNEL_SKINNY = 3,     /* VALU strip kernel, M <= 8 and transB == N         */
    FDL_KERNEL_TILED256 = 4,   /* 256x256x16 LDS double-buffered MFMA tile, 8 waves */
    FDL_KERNEL_TILED256X128 = 5, /* 256x128x16 tile, 8 waves                        */
    FDL_KERNEL_TILED128W8 = 6, /* 128x128x16 tile, 8 waves of 32x64                 */
    FDL_KERNEL_SPLITK16 = 7,   /* 16x16 tile (16x16x4 MFMA), K split over waves     */
    FDL_KERNEL_DMA256 = 8,     /* 256x256x16 tile fed by direct global->LDS copies;
                                  needs K % 4 == 0 and 16-byte-vectorisable operands
                                  (base, ld and batch stride multiples of 4 floats,
                                  the contiguous extent a multiple of 4)          */
    FDL_KERNEL_DMA128 = 9,     /* 128x128x32 tile, two blocks per CU, same copies  */
    FDL_KERNEL_DMA64 = 10,     /* 64x64x64 tile, same copies; two sets of four
                                  32x32 waves split each K-tile                    */
    FDL_KERNEL_DMA128W8 = 11,  /* 128x128x64 tile, eight waves of 64x32, one block
                                  per CU, same copies                              */
    FDL_KERNEL_DMA64U = 12,    /* FDL_KERNEL_DMA64 with 4-byte copies: any K, any
                                  leading dimension up to 2^24, any 4-byte-aligned
                                  operand (odd shapes, unaligned views)            */
    FDL_KERNEL_DMA128W8U = 13, /* FDL_KERNEL_DMA128W8 with 4-byte copies          */
    FDL_KERNEL_DMA64S = 14,    /* 64x64x16 tile, 16-byte copies, four K-tiles in
                                  flight, four 32x32 waves: short-K batches       */
    FDL_KERNEL_DMA96X32U = 15  /* 96x32x64 tile, 4-byte copies, four k-group sets
                                  of three 32x32 waves: mid sizes whose 64x64
                                  tiles leave CUs idle                            */
} fdl_kernel;

/*
 * fdl_sgemm_ex with the kernel family forced, for tests and benchmarks that
 * must cover every family on the same shape (the reference benchmark ran all
 * of its GemmAlgo variants the same way, tests/benchmarks/gemm/
 * gemm_benchmark.cu:86-100).  FDL_KERNEL_SKINNY with M > 8 or transB == T
 * returns FDL_ERROR_NOT_SUPPORTED.
 */
int fdl_sgemm_ex_select(int transA, int transB,
                        int64_t M, int64_t N, int64_t K,
                        const float* A, int64_t lda, int64_t strideA,
                        const float* B, int64_t ldb, int64_t strideB,
                        float* C, int64_t ldc, int64_t strideC,
                        int64_t batch,
                        const float* bias, const float* aux, int epilogue,
                        int kernel, void* stream);

/* Kernel family fdl_sgemm_ex would use for this problem (FDL_KERNEL_*). */
int fdl_sgemm_kernel_choice(int transA, int transB,
                            int64_t M, int64_t N, int64_t K, int64_t batch);

/*
 * Workspace, in bytes, that fdl_sgemm_ex_ws can use for this problem; 0 when
 * it would use none.  Non-zero only for one problem (batch == 1) that the
 * skinny family runs (M <= 8, transB == N) with N % 4 == 0 and enough work
 * to pay for a second pass (K >= 4096, or N * K >= 2^23).  This build's own extension: the
 * reference called cublasSgemm, which takes no workspace
 * (src/kernels/cuda/gemm.cu:166-177).
 */
size_t fdl_sgemm_workspace_size(int transA, int transB,
                                int64_t M, int64_t N, int64_t K, int64_t batch);

/*
 * fdl_sgemm_ex with a caller-owned device workspace (16-byte aligned, or
 * NULL).  Given at least fdl_sgemm_workspace_size() bytes, and B 16-byte
 * vectorisable, a skinny problem splits K over blocks: each block streams a
 * 256-column band of B over one slice of K and writes partial sums to the
 * workspace, and a second launch adds the slices in slice order and applies
 * the epilogue.  Results repeat bit for bit, and differ from fdl_sgemm_ex's
 * single pass only in the order of the fp32 additions.  Every other problem,
 * or a smaller workspace, runs exactly as fdl_sgemm_ex.  The workspace is
 * written on `stream`: work on other streams must not use it until the call's
 * work there has finished.
 */
int fdl_sgemm_ex_ws(int transA, int transB,
                    int64_t M, int64_t N, int64_t K,
                    const float* A, int64_t lda, int64_t strideA,
                    const float* B, int64_t ldb, int64_t strideB,
                    float* C, int64_t ldc, int64_t strideC,
                    int64_t batch,
                    const float* bias, const float* aux, int epilogue,
                    void* workspace, size_t workspace_bytes,
                    void* stream);

/*
 * fdl_sgemm_ex_ws with the library's own scratch in place of a workspace
 * argument: allocates nothing (no hipMalloc, no hipFree, no allocating
 * library call), for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation).  It has no
 * counterpart in the reference.  The scratch is a static device array of
 * 4 MiB per GPU, held until the process ends; a problem whose
 * fdl_sgemm_workspace_size exceeds it returns FDL_ERROR_INVALID_VALUE.
 * Every call on one GPU shares that GPU's scratch: calls whose work overlaps
 * on one GPU (on different streams, or from different threads without
 * ordering between their streams) race and may return wrong results.
 * Results equal fdl_sgemm_ex_ws's bit for bit.
 */
int fdl_sgemm_ex_noalloc(int transA, int transB,
                         int64_t M, int64_t N, int64_t K,
                         const float* A, int64_t lda, int64_t strideA,
                         const float* B, int64_t ldb, int64_t strideB,
                         float* C, int64_t ldc, int64_t strideC,
                         int64_t batch,
                         const float* bias, const float* aux, int epilogue,
                         void* stream);

/*
 * C[m,n] = A[m,k] . B[k,n], row-major, contiguous, null stream.
 * Same contract as dl::kernels::gemm (include/dl/kernels/gemm.hpp:16-17,
 * src/kernels/cuda/gemm.cu:197-213) with the algorithm choice internal.
 */
int fdl_gemm(const float* a, const float* b, float* c, int m, int n, int k);

/*
 * out[r, c] += bias[c] in place over a rows x cols row-major matrix.
 * Replaces dl::kernels::add_row_bias (include/dl/kernels/bias.hpp:5,
 * src/kernels/cuda/bias.cu:5-28).
 */
int fdl_add_row_bias(float* out, const float* bias, int64_t rows, int64_t cols,
                     void* stream);

/*
 * out[i] = fmaxf(0, in[i]).  Replaces the ReLU branch of
 * dl::kernels::activation (src/kernels/cuda/activation.cu:6-17,74-78).
 */
int fdl_relu(const float* in, float* out, int64_t n, void* stream);

/*
 * grad_in[i] = act[i] > 0 ? grad_out[i] : 0, where act is the ReLU input or
 * output (both are > 0 at the same places).  No reference counterpart exists
 * (the reference has no ReLU backward); the rule follows the derivative with
 * the value at exactly 0 taken as 0.
 */
int fdl_relu_backward(const float* grad_out, const float* act, float* grad_in,
                      int64_t n, void* stream);

/*
 * out[c] = sum_r x[r, c] (rows summed in increasing r order).  The db term of
 * linear backward, legacy/src/ops/Layers.cpp:44.
 */
int fdl_colsum(const float* x, float* out, int64_t rows, int64_t cols,
               void* stream);

/*
 * Row softmax, out[r, :] = exp(x - max) / sum(exp(x - max)).
 * Replaces dl::kernels::softmax as called by ops::softmax
 * (src/ops/Softmax.cpp:33-38, src/kernels/cuda/softmax.cu:131-254).
 */
int fdl_softmax(const float* in, float* out, int64_t rows, int64_t cols,
                void* stream);

/*
 * Mean softmax cross-entropy over a batch, and optionally its gradient.
 *   loss[0] = (1/batch) * sum over rows with 0 <= label < classes of
 *             (log(sum_c exp(z_c - max)) + max - z_label)
 *   grad[r, c] = (softmax(z_r)_c - [c == label_r]) / batch   (if grad != NULL)
 * loss follows dl::kernels::cross_entropy (src/kernels/cuda/cross_entropy.cu:
 * 9-35): rows with an invalid label add nothing but still count in batch.
 * grad follows legacy SoftmaxCrossEntropyLoss::backward
 * (legacy/src/ops/SoftmaxCrossEntropyLoss.cpp:39-51).  loss is written, not
 * accumulated, so it needs no prior zeroing.
 */
int fdl_softmax_xent(const float* logits, const int64_t* labels,
                     float* loss, float* grad, int64_t batch, int64_t classes,
                     void* stream);

/*
 * param[i] -= lr * grad[i].  SGD::step, legacy/include/dl/optim/Optimizer.hpp:
 * 24-34.
 */
int fdl_sgd_update(float* param, const float* grad, float lr, int64_t n,
                   void* stream);

/*
 * One training step of the two-layer MLP  in -> hidden (ReLU) -> classes with
 * softmax cross-entropy and SGD, weights in the active API's [in, out] layout
 * (src/nn/Linear.cpp:27).  Step order follows legacy Network
 * (legacy/src/runtime/Network.cpp:7-34): forward, loss, backward through every
 * layer (dX of the first layer included when dX != NULL), then the update.
 *
 *   H      = relu(X W1 + b1)              [batch, hidden]
 *   logits = H W2 + b2                    [batch, classes]
 *   G2     = (softmax(logits) - onehot)/batch, loss as fdl_softmax_xent
 *   dW2 = H^T G2, db2 = colsum(G2), G1 = (G2 W2^T) * [H > 0]
 *   dW1 = X^T G1, db1 = colsum(G1), dX = G1 W1^T
 *   W -= lr dW, b -= lr db for both layers
 *
 * Every buffer belongs to the caller; the step allocates nothing.  H, logits,
 * G2, G1, dW1, db1, dW2, db2 hold the step's intermediates on return.
 * The step is 4 launches when classes <= 16 and hidden <= 1024, or
 * classes <= 32 and hidden <= 512, and ceil(batch / 8) * (classes + 1) <=
 * in_features * hidden: then dW1 holds per-block partial sums of the loss
 * and db2 until the last launch writes the weight gradient into it.
 * Otherwise it is 6 launches.
 */
int fdl_mlp2_train_step(const float* X, const int64_t* labels,
                        int64_t batch, int64_t in_features,
                        int64_t hidden, int64_t classes,
                        float* W1, float* b1, float* W2, float* b2, float lr,
                        float* H, float* logits, float* G2, float* G1,
                        float* dW1, float* db1, float* dW2, float* db2,
                        float* dX, float* loss, void* stream);

/*
 * The same training step captured once into a HIP graph and replayed: one
 * launch per step instead of six, for loops that keep the same buffers
 * (refill X and labels in place between steps).  create captures
 * fdl_mlp2_train_step with these exact pointers on `stream` (a temporary
 * stream when NULL) and instantiates it; launch replays it on `stream`;
 * destroy releases the graph.  Nothing runs at create time.  No reference
 * counterpart (the reference has no training step on the GPU); this is the
 * host-launch side of the step's runtime.
 */
typedef struct fdl_mlp2_graph fdl_mlp2_graph;

int fdl_mlp2_graph_create(fdl_mlp2_graph** graph,
                          const float* X, const int64_t* labels,
                          int64_t batch, int64_t in_features,
                          int64_t hidden, int64_t classes,
                          float* W1, float* b1, float* W2, float* b2, float lr,
                          float* H, float* logits, float* G2, float* G1,
                          float* dW1, float* db1, float* dW2, float* db2,
                          float* dX, float* loss, void* stream);
/*
 * The same with `steps` (>= 1) consecutive training steps in the one graph,
 * so that a replay runs them all for one host launch: each step reads the
 * parameters the one before it updated, as the same number of
 * fdl_mlp2_train_step calls would.  fdl_mlp2_graph_create is steps = 1.
 * No reference counterpart, as above.
 */
int fdl_mlp2_graph_create_steps(fdl_mlp2_graph** graph, int steps,
                                const float* X, const int64_t* labels,
                                int64_t batch, int64_t in_features,
                                int64_t hidden, int64_t classes,
                                float* W1, float* b1, float* W2, float* b2, float lr,
                                float* H, float* logits, float* G2, float* G1,
                                float* dW1, float* db1, float* dW2, float* db2,
                                float* dX, float* loss, void* stream);
int fdl_mlp2_graph_launch(fdl_mlp2_graph* graph, void* stream);
int fdl_mlp2_graph_destroy(fdl_mlp2_graph* graph);

/*
 * Sets `bytes` bytes at `data` to zero, with a kernel on `stream` (null: the
 * null stream).  Replaces the cudaMemset of TensorImpl::zero_
 * (src/tensor/TensorImpl.cpp:143-154); a kernel rather than a memset, so that
 * dl:: work captured into a graph replays correctly.
 */
int fdl_zero_fill(void* data, int64_t bytes, void* stream);

/*
 * Fill with uniform values in (low, high] or normal values, from a
 * counter-based Philox4x32-10 stream keyed by seed (element i uses counter i).
 * Replaces the cuRAND fills of dl::kernels::uniform_float32 / normal_float32
 * (src/kernels/cuda/random.cu:7-54); the values are NOT bit-identical to
 * cuRAND's, only the distribution and same-seed determinism match.
 */
int fdl_fill_uniform(float* data, int64_t n, float low, float high,
                     uint64_t seed, void* stream);
int fdl_fill_normal(float* data, int64_t n, float mean, float stddev,
                    uint64_t seed, void* stream);

/* Message for the last non-zero status returned on the calling thread. */
const char* fdl_last_error(void);

/* Name of a status code. */
const char* fdl_status_string(int status);

/* Build identification string (target architecture and version). */
const char* fdl_version(void);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* FASTDL_GEMM_H */
