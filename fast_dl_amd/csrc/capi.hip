// extern "C" entry points declared in include/fastdl_gemm.h: argument
// validation, status codes and dispatch onto the kernels.  Nothing here
// allocates memory or synchronises the stream.  fdl_sgemm_ex_noalloc's scratch
// is a static device array (one per GPU, for the life of the process).
#include "fdl_internal.hpp"

#include "../../include/fastdl_data.h"
#include "../../include/fastdl_gemm.h"

#include <climits>
#include <cstdint>
#include <cmath>
#include <cstdio>
#include <mutex>
#include <string>

namespace {

thread_local std::string g_last_error;

int fail(int status, const std::string& msg) {
    g_last_error = msg;
    return status;
}

int check_hip(hipError_t err, const char* what) {
    if (err == hipSuccess) return FDL_SUCCESS;
    return fail(FDL_ERROR_LAUNCH, std::string(what) + ": " + hipGetErrorString(err));
}

bool fits_int(int64_t v) { return v >= 0 && v <= INT_MAX; }

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace

namespace {

// fdl_sgemm_ex_select with an optional workspace (fdl_sgemm_ex_ws).
int sgemm_impl(int transA, int transB, int64_t M, int64_t N, int64_t K, const float* A,
               int64_t lda, int64_t strideA, const float* B, int64_t ldb, int64_t strideB,
               float* C, int64_t ldc, int64_t strideC, int64_t batch, const float* bias,
               const float* aux, int epilogue, int kernel, void* workspace,
               size_t workspace_bytes, void* stream) {
    if (kernel < FDL_KERNEL_AUTO || kernel > FDL_KERNEL_DMA96X32U) {
        return fail(FDL_ERROR_INVALID_VALUE, "sgemm: unknown kernel family");
    }
    if ((transA != FDL_OP_N && transA != FDL_OP_T) ||
        (transB != FDL_OP_N && transB != FDL_OP_T)) {
        return fail(FDL_ERROR_INVALID_VALUE, "sgemm: transA/transB must be FDL_OP_N or FDL_OP_T");
    }
    if (!fits_int(M) || !fits_int(N) || !fits_int(K)) {
        return fail(FDL_ERROR_INVALID_VALUE, "sgemm: M, N, K must be in [0, INT_MAX]");
    }
    if (batch < 0) return fail(FDL_ERROR_INVALID_VALUE, "sgemm: batch must be >= 0");
    if (epilogue < FDL_EPILOGUE_NONE || epilogue > FDL_EPILOGUE_RELU_GRAD) {
        return fail(FDL_ERROR_INVALID_VALUE, "sgemm: unknown epilogue");
    }
    const bool ta = transA == FDL_OP_T;
    const bool tb = transB == FDL_OP_T;
    const int64_t a_cols = ta ? M : K;
    const int64_t b_cols = tb ? K : N;
    if (lda < std::max<int64_t>(1, a_cols)) return fail(FDL_ERROR_INVALID_VALUE, "sgemm: lda too small");
    if (ldb < std::max<int64_t>(1, b_cols)) return fail(FDL_ERROR_INVALID_VALUE, "sgemm: ldb too small");
    if (ldc < std::max<int64_t>(1, N)) return fail(FDL_ERROR_INVALID_VALUE, "sgemm: ldc too small");
    if (strideA < 0 || strideB < 0 || strideC < 0) {
        return fail(FDL_ERROR_INVALID_VALUE, "sgemm: strides must be >= 0");
    }
    if (batch == 0 || M == 0 || N == 0) return FDL_SUCCESS;
    if (batch > 1 && strideC < (M - 1) * ldc + N) {
        return fail(FDL_ERROR_INVALID_VALUE, "sgemm: strideC makes output batches overlap");
    }
    if (C == nullptr) return fail(FDL_ERROR_INVALID_VALUE, "sgemm: C is null");
    if (K > 0 && (A == nullptr || B == nullptr)) {
        return fail(FDL_ERROR_INVALID_VALUE, "sgemm: A or B is null");
    }
    if ((epilogue == FDL_EPILOGUE_BIAS || epilogue == FDL_EPILOGUE_BIAS_RELU) && bias == nullptr) {
        return fail(FDL_ERROR_INVALID_VALUE, "sgemm: bias epilogue needs a bias pointer");
    }
    if (epilogue == FDL_EPILOGUE_RELU_GRAD && aux == nullptr) {
        return fail(FDL_ERROR_INVALID_VALUE, "sgemm: RELU_GRAD epilogue needs an aux pointer");
    }

    fdl::GemmParams p{};
    p.A = A;
    p.B = B;
    p.C = C;
    p.bias = bias;
    p.aux = (epilogue == FDL_EPILOGUE_RELU_GRAD) ? aux : nullptr;
    p.lda = lda;
    p.ldb = ldb;
    p.ldc = ldc;
    p.strideA = strideA;
    p.strideB = strideB;
    p.strideC = strideC;
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    p.epilogue = epilogue;
    const fdl::GemmKernel kern = static_cast<fdl::GemmKernel>(kernel);
    if (kern == fdl::GemmKernel::Skinny && (tb || M > 8)) {
        return fail(FDL_ERROR_NOT_SUPPORTED, "sgemm: skinny kernel needs M <= 8 and B not transposed");
    }
    if ((kern == fdl::GemmKernel::Dma256 || kern == fdl::GemmKernel::Dma128 ||
         kern == fdl::GemmKernel::Dma64 || kern == fdl::GemmKernel::Dma128W8 ||
         kern == fdl::GemmKernel::Dma64S) &&
        !fdl::dma_supported(kern, p, ta, tb, batch)) {
        return fail(FDL_ERROR_NOT_SUPPORTED,
                    "sgemm: the 16-byte direct-to-LDS kernels need K % 4 == 0, "
                    "16-byte-vectorisable operands and leading dimensions up to 2^22");
    }
    if ((kern == fdl::GemmKernel::Dma64U || kern == fdl::GemmKernel::Dma128W8U ||
         kern == fdl::GemmKernel::Dma96x32U) &&
        !fdl::dma_supported(kern, p, ta, tb, batch)) {
        return fail(FDL_ERROR_NOT_SUPPORTED,
                    "sgemm: the 4-byte direct-to-LDS kernels need leading dimensions up to 2^24 "
                    "and 4-byte-aligned operands");
    }
    if (workspace != nullptr && (reinterpret_cast<uintptr_t>(workspace) & 15u) != 0) {
        return fail(FDL_ERROR_INVALID_VALUE, "sgemm: workspace must be 16-byte aligned");
    }
    return check_hip(fdl::launch_sgemm(p, ta, tb, batch, kern, as_stream(stream),
                                       static_cast<float*>(workspace),
                                       workspace ? workspace_bytes : 0),
                     "sgemm launch failed");
}

// Scratch of fdl_sgemm_ex_noalloc: the partial sums of the skinny family's
// K split (at most 4 MiB: M <= 8, N = K = 4096).  Each GPU holds its own copy
// at its own address; host code reaches it only through the address
// hipGetSymbolAddress returns for the current device.
constexpr size_t kScratchBytes = size_t(4) << 20;
constexpr int kScratchDevices = 64;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

std::mutex g_scratch_mu;
float* g_scratch_ptr[kScratchDevices] = {};

// The current device's scratch address, looked up (with that device
// current) on the first call on the device.  Returns an fdl status.
int device_scratch(float** out) {
    int device = 0;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess) {
        return fail(FDL_ERROR_RUNTIME,
                    std::string("sgemm_noalloc: hipGetDevice: ") + hipGetErrorString(err));
    }
    if (device < 0 || device >= kScratchDevices) {
        return fail(FDL_ERROR_NOT_SUPPORTED, "sgemm_noalloc: device index beyond the scratch table");
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[device] == nullptr) {
        void* ptr = nullptr;
        err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (err != hipSuccess || ptr == nullptr) {
            return fail(FDL_ERROR_RUNTIME, std::string("sgemm_noalloc: hipGetSymbolAddress: ") +
                                               hipGetErrorString(err));
        }
        g_scratch_ptr[device] = static_cast<float*>(ptr);
    }
    *out = g_scratch_ptr[device];
    return FDL_SUCCESS;
}

}  // namespace

extern "C" {

int fdl_sgemm_ex_select(int transA, int transB, int64_t M, int64_t N, int64_t K,
                        const float* A, int64_t lda, int64_t strideA, const float* B,
                        int64_t ldb, int64_t strideB, float* C, int64_t ldc,
                        int64_t strideC, int64_t batch, const float* bias,
                        const float* aux, int epilogue, int kernel, void* stream) {
    return sgemm_impl(transA, transB, M, N, K, A, lda, strideA, B, ldb, strideB, C, ldc,
                      strideC, batch, bias, aux, epilogue, kernel, nullptr, 0, stream);
}

int fdl_sgemm_ex_ws(int transA, int transB, int64_t M, int64_t N, int64_t K,
                    const float* A, int64_t lda, int64_t strideA, const float* B,
                    int64_t ldb, int64_t strideB, float* C, int64_t ldc,
                    int64_t strideC, int64_t batch, const float* bias,
                    const float* aux, int epilogue, void* workspace,
                    size_t workspace_bytes, void* stream) {
    return sgemm_impl(transA, transB, M, N, K, A, lda, strideA, B, ldb, strideB, C, ldc,
                      strideC, batch, bias, aux, epilogue, FDL_KERNEL_AUTO, workspace,
                      workspace_bytes, stream);
}

int fdl_sgemm_ex_noalloc(int transA, int transB, int64_t M, int64_t N, int64_t K,
                         const float* A, int64_t lda, int64_t strideA, const float* B,
                         int64_t ldb, int64_t strideB, float* C, int64_t ldc,
                         int64_t strideC, int64_t batch, const float* bias,
                         const float* aux, int epilogue, void* stream) {
    const size_t need = fdl_sgemm_workspace_size(transA, transB, M, N, K, batch);
    if (need > kScratchBytes) {
        return fail(FDL_ERROR_INVALID_VALUE,
                    "sgemm_noalloc: the problem needs " + std::to_string(need) +
                        " bytes of scratch, more than the " + std::to_string(kScratchBytes) +
                        " the library holds per device");
    }
    float* ws = nullptr;
    if (need > 0 && M > 0 && N > 0) {
        const int status = device_scratch(&ws);
        if (status != FDL_SUCCESS) return status;
    }
    return sgemm_impl(transA, transB, M, N, K, A, lda, strideA, B, ldb, strideB, C, ldc,
                      strideC, batch, bias, aux, epilogue, FDL_KERNEL_AUTO, ws,
                      ws ? kScratchBytes : 0, stream);
}

size_t fdl_sgemm_workspace_size(int transA, int transB, int64_t M, int64_t N, int64_t K,
                                int64_t batch) {
    if (!fits_int(M) || !fits_int(N) || !fits_int(K) || batch < 1) return 0;
    fdl::GemmParams p{};
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    return fdl::skinny_split_plan(p, transA == FDL_OP_T, transB == FDL_OP_T, batch).bytes;
}

int fdl_sgemm_ex(int transA, int transB, int64_t M, int64_t N, int64_t K,
                 const float* A, int64_t lda, int64_t strideA, const float* B,
                 int64_t ldb, int64_t strideB, float* C, int64_t ldc,
                 int64_t strideC, int64_t batch, const float* bias,
                 const float* aux, int epilogue, void* stream) {
    return fdl_sgemm_ex_select(transA, transB, M, N, K, A, lda, strideA, B, ldb, strideB,
                               C, ldc, strideC, batch, bias, aux, epilogue,
                               FDL_KERNEL_AUTO, stream);
}

int fdl_sgemm_kernel_choice(int transA, int transB, int64_t M, int64_t N, int64_t K,
                            int64_t batch) {
    if (!fits_int(M) || !fits_int(N) || !fits_int(K) || batch < 1) return FDL_KERNEL_AUTO;
    fdl::GemmParams p{};
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    return static_cast<int>(fdl::choose_kernel(p, transA == FDL_OP_T, transB == FDL_OP_T, batch));
}

int fdl_gemm(const float* a, const float* b, float* c, int m, int n, int k) {
    if (m < 0 || n < 0 || k < 0) return fail(FDL_ERROR_INVALID_VALUE, "gemm: negative size");
    return fdl_sgemm_ex(FDL_OP_N, FDL_OP_N, m, n, k, a, std::max(k, 1), 0, b,
                        std::max(n, 1), 0, c, std::max(n, 1), 0, 1, nullptr, nullptr,
                        FDL_EPILOGUE_NONE, nullptr);
}

int fdl_add_row_bias(float* out, const float* bias, int64_t rows, int64_t cols,
                     void* stream) {
    if (rows < 0 || cols < 0) return fail(FDL_ERROR_INVALID_VALUE, "add_row_bias: negative size");
    if (rows * cols == 0) return FDL_SUCCESS;
    if (!out || !bias) return fail(FDL_ERROR_INVALID_VALUE, "add_row_bias: null pointer");
    return check_hip(fdl::launch_add_row_bias(out, bias, rows, cols, as_stream(stream)),
                     "add_row_bias launch failed");
}

int fdl_relu(const float* in, float* out, int64_t n, void* stream) {
    if (n < 0) return fail(FDL_ERROR_INVALID_VALUE, "relu: negative size");
    if (n == 0) return FDL_SUCCESS;
    if (!in || !out) return fail(FDL_ERROR_INVALID_VALUE, "relu: null pointer");
    return check_hip(fdl::launch_relu(in, out, n, as_stream(stream)), "relu launch failed");
}

int fdl_relu_backward(const float* grad_out, const float* act, float* grad_in,
                      int64_t n, void* stream) {
    if (n < 0) return fail(FDL_ERROR_INVALID_VALUE, "relu_backward: negative size");
    if (n == 0) return FDL_SUCCESS;
    if (!grad_out || !act || !grad_in) {
        return fail(FDL_ERROR_INVALID_VALUE, "relu_backward: null pointer");
    }
    return check_hip(fdl::launch_relu_backward(grad_out, act, grad_in, n, as_stream(stream)),
                     "relu_backward launch failed");
}

int fdl_colsum(const float* x, float* out, int64_t rows, int64_t cols, void* stream) {
    if (rows < 0 || cols < 0) return fail(FDL_ERROR_INVALID_VALUE, "colsum: negative size");
    if (cols == 0) return FDL_SUCCESS;
    if (!out || (rows > 0 && !x)) return fail(FDL_ERROR_INVALID_VALUE, "colsum: null pointer");
    return check_hip(fdl::launch_colsum(x, out, rows, cols, as_stream(stream)),
                     "colsum launch failed");
}

int fdl_softmax(const float* in, float* out, int64_t rows, int64_t cols, void* stream) {
    if (rows <= 0 || cols <= 0) {
        return fail(FDL_ERROR_INVALID_VALUE, "softmax: rows and cols must be non-zero");
    }
    if (!in || !out) return fail(FDL_ERROR_INVALID_VALUE, "softmax: null pointer");
    return check_hip(fdl::launch_softmax(in, out, rows, cols, as_stream(stream)),
                     "softmax launch failed");
}

int fdl_softmax_xent(const float* logits, const int64_t* labels, float* loss,
                     float* grad, int64_t batch, int64_t classes, void* stream) {
    if (batch <= 0) return fail(FDL_ERROR_INVALID_VALUE, "softmax_xent: batch must be positive");
    if (classes <= 0) {
        return fail(FDL_ERROR_INVALID_VALUE, "softmax_xent: class count must be positive");
    }
    if (!logits || !labels || (!loss && !grad)) {
        return fail(FDL_ERROR_INVALID_VALUE, "softmax_xent: null pointer");
    }
    return check_hip(fdl::launch_softmax_xent(logits, labels, loss, grad, batch, classes,
                                              as_stream(stream)),
                     "softmax_xent launch failed");
}

int fdl_sgd_update(float* param, const float* grad, float lr, int64_t n, void* stream) {
    if (n < 0) return fail(FDL_ERROR_INVALID_VALUE, "sgd_update: negative size");
    if (n == 0) return FDL_SUCCESS;
    if (!param || !grad) return fail(FDL_ERROR_INVALID_VALUE, "sgd_update: null pointer");
    return check_hip(fdl::launch_sgd(param, grad, lr, n, as_stream(stream)),
                     "sgd_update launch failed");
}

int fdl_mlp2_train_step(const float* X, const int64_t* labels, int64_t batch,
                        int64_t in_features, int64_t hidden, int64_t classes,
                        float* W1, float* b1, float* W2, float* b2, float lr,
                        float* H, float* logits, float* G2, float* G1, float* dW1,
                        float* db1, float* dW2, float* db2, float* dX, float* loss,
                        void* stream) {
    if (batch <= 0 || in_features <= 0 || hidden <= 0 || classes <= 0 ||
        !fits_int(batch) || !fits_int(in_features) || !fits_int(hidden) ||
        !fits_int(classes)) {
        return fail(FDL_ERROR_INVALID_VALUE, "mlp2_train_step: sizes must be positive ints");
    }
    if (!X || !labels || !W1 || !b1 || !W2 || !b2 || !H || !logits || !G2 || !G1 ||
        !dW1 || !db1 || !dW2 || !db2 || !loss) {
        return fail(FDL_ERROR_INVALID_VALUE, "mlp2_train_step: null pointer");
    }
    const int64_t B = batch, I = in_features, Hd = hidden, Cc = classes;
    const hipStream_t hs = as_stream(stream);
    int st;
    auto gemm_job = [&](bool ta, bool tb, int64_t M, int64_t N, int64_t K, const float* A,
                        int64_t lda, const float* Bm, int64_t ldb, float* C, int epi,
                        const float* aux, float* upd) {
        fdl::GroupJob j;
        j.kind = fdl::GroupJob::kGemm;
        j.ta = ta;
        j.tb = tb;
        j.p.A = A;
        j.p.B = Bm;
        j.p.C = C;
        j.p.aux = aux;
        j.p.upd = upd;
        j.p.lr = lr;
        j.p.lda = lda;
        j.p.ldb = ldb;
        j.p.ldc = N;
        j.p.M = (int)M;
        j.p.N = (int)N;
        j.p.K = (int)K;
        j.p.epilogue = epi;
        return j;
    };
    fdl::GroupJob db1_job;  // db1 = colsum(G1), b1 -= lr * db1
    db1_job.kind = fdl::GroupJob::kColsumSgd;
    db1_job.x = G1;
    db1_job.out = db1;
    db1_job.param = b1;
    db1_job.lr = lr;
    db1_job.rows = B;
    db1_job.cols = Hd;
    fdl::GroupJob w2_job;  // W2 -= lr * dW2
    w2_job.kind = fdl::GroupJob::kSgd;
    w2_job.x = dW2;
    w2_job.param = W2;
    w2_job.lr = lr;
    w2_job.rows = Hd * Cc;
    // The last launch of either sequence: dW1 = X^T G1 (TN) with W1 -= lr * dW1
    // in the epilogue, and W2 -= lr * dW2.
    auto last_launch = [&]() {
        return check_hip(fdl::launch_group2(gemm_job(true, false, I, Hd, B, X, I, G1, Hd, dW1,
                                                     fdl::EPI_SGD, nullptr, W1),
                                            w2_job, hs),
                         "mlp2_train_step dW1/W2 failed");
    };

    // Forward layer 1: H = relu(X W1 + b1).
    st = fdl_sgemm_ex(FDL_OP_N, FDL_OP_N, B, Hd, I, X, I, 0, W1, Hd, 0, H, Hd, 0, 1, b1,
                      nullptr, FDL_EPILOGUE_BIAS_RELU, stream);
    if (st) return st;

    // Three launches when dX's product can join the head (or dX is not
    // asked for): launch 2 makes logits, G2, G1 and dX = G1 W1^T; launch 3
    // makes dW1 = X^T G1 with the W1 step in its epilogue, db1 with the b1
    // step, dW2 = H^T G2 with the W2 step, and the loss, db2 and the b2 step
    // from the stored logits and G2.  Every parameter is updated in a later
    // launch than its last read: W1 is read by launches 1 and 2, b1 by
    // launch 1, W2 and b2 by launch 2; all four are updated in launch 3.
    const bool three = Cc <= fdl::kXentFusedMaxClasses &&
                       (dX ? fdl::head_dx_supported(B, I, Hd, Cc, H, W1)
                           : fdl::head_supported(Hd, Cc) &&
                                 fdl::head_blocks(B) * (Cc + 1) <= I * Hd);
    if (three) {
        if (dX) {
            st = check_hip(fdl::launch_mlp_head_dx(H, W2, b2, labels, W1, logits, G2, G1, dX, B,
                                                   I, Hd, Cc, hs),
                           "mlp2_train_step head failed");
        } else {
            // the head's records land in dW1, which launch 3 overwrites unread
            st = check_hip(fdl::launch_mlp_head(H, W2, b2, labels, logits, G2, G1, dW1, B, Hd,
                                                Cc, hs),
                           "mlp2_train_step head failed");
        }
        if (st) return st;
        fdl::GroupJob fin;
        fin.kind = fdl::GroupJob::kHeadFinalize;
        fin.x = logits;
        fin.x2 = G2;
        fin.labels = labels;
        fin.out = db2;
        fin.out2 = loss;
        fin.param = b2;
        fin.lr = lr;
        fin.rows = B;
        fin.cols = Cc;
        fdl::GroupJob jobs[4] = {
            gemm_job(true, false, I, Hd, B, X, I, G1, Hd, dW1, fdl::EPI_SGD, nullptr, W1), db1_job,
            gemm_job(true, false, Hd, Cc, B, H, Hd, G2, Cc, dW2, fdl::EPI_SGD, nullptr, W2), fin};
        // dW2 is Hd x Cc: with at most 16 classes, 16x16 output tiles
        if (Cc <= 16) jobs[2].kind = fdl::GroupJob::kGemm16;
        return check_hip(fdl::launch_group(jobs, 4, hs), "mlp2_train_step backward failed");
    }

    // Otherwise four launches when the head fits one block per kHeadRows rows
    // (W2 in LDS) and its per-block records fit in dW1, which holds them until
    // the last launch overwrites it with the weight gradient.  Every parameter is
    // updated in a later launch than its last read: b2 and W2 are read by the
    // head (launch 2), b2 is updated in launch 3 and W2 in launch 4; b1 is
    // read by launch 1 and updated in launch 3; W1 is read by launch 1 and by
    // the dX product (launch 3) and updated in launch 4.
    const int64_t records = fdl::head_blocks(B);
    const bool fused_head = fdl::head_supported(Hd, Cc) && records * (Cc + 1) <= I * Hd;
    if (fused_head) {
        // Launch 2: logits, loss shares, G2 and G1 = (G2 W2^T) * [H > 0].
        st = check_hip(fdl::launch_mlp_head(H, W2, b2, labels, logits, G2, G1, dW1, B, Hd, Cc,
                                            hs),
                       "mlp2_train_step head failed");
        if (st) return st;
        // Launch 3: dX = G1 W1^T (NT), db1 with the b1 step, dW2 = H^T G2
        // (TN), and the records' reduction into loss, db2 and the b2 step.
        fdl::GroupJob fin;
        fin.kind = fdl::GroupJob::kXentFinalize;
        fin.x = dW1;
        fin.out = db2;
        fin.out2 = loss;
        fin.param = b2;
        fin.lr = lr;
        fin.rows = records;
        fin.cols = Cc;
        const fdl::GroupJob dw2_job = gemm_job(true, false, Hd, Cc, B, H, Hd, G2, Cc, dW2,
                                               fdl::EPI_NONE, nullptr, nullptr);
        if (dX) {
            const fdl::GroupJob jobs[4] = {gemm_job(false, true, B, I, Hd, G1, Hd, W1, Hd, dX,
                                                    fdl::EPI_NONE, nullptr, nullptr),
                                           db1_job, dw2_job, fin};
            st = check_hip(fdl::launch_group(jobs, 4, hs), "mlp2_train_step backward failed");
        } else {
            const fdl::GroupJob jobs[3] = {db1_job, dw2_job, fin};
            st = check_hip(fdl::launch_group(jobs, 3, hs), "mlp2_train_step backward failed");
        }
        if (st) return st;
        return last_launch();
    }

    // Otherwise six launches.  logits = H W2 + b2.
    st = fdl_sgemm_ex(FDL_OP_N, FDL_OP_N, B, Cc, Hd, H, Hd, 0, W2, Cc, 0, logits, Cc, 0, 1,
                      b2, nullptr, FDL_EPILOGUE_BIAS, stream);
    if (st) return st;
    // Loss, G2 = dL/dlogits, db2 = colsum(G2) and b2 -= lr * db2 in one kernel
    // (two launches when the class count is too large to stage in LDS).
    if (Cc <= fdl::kXentFusedMaxClasses) {
        st = check_hip(fdl::launch_softmax_xent_db_sgd(logits, labels, loss, G2, db2, b2, lr, B,
                                                       Cc, hs),
                       "mlp2_train_step loss failed");
        if (st) return st;
    } else {
        st = fdl_softmax_xent(logits, labels, loss, G2, B, Cc, stream);
        if (st) return st;
        st = check_hip(fdl::launch_colsum_sgd(G2, db2, b2, lr, B, Cc, hs),
                       "mlp2_train_step db2 failed");
        if (st) return st;
    }
    // The backward pass runs as three grouped launches of independent jobs.
    // Updates are ordered after every read of the old value: W2 is read by
    // the G1 GEMM (first launch) and updated in the third, W1 is read by the
    // dX GEMM (second launch) and updated in the third.
    // G1 = (G2 W2^T) masked by H > 0 (NT, ReLU-gradient epilogue) and
    // dW2 = H^T G2 (TN).
    st = check_hip(fdl::launch_group2(
                       gemm_job(false, true, B, Hd, Cc, G2, Cc, W2, Cc, G1,
                                fdl::EPI_RELU_GRAD, H, nullptr),
                       gemm_job(true, false, Hd, Cc, B, H, Hd, G2, Cc, dW2, fdl::EPI_NONE,
                                nullptr, nullptr),
                       hs),
                   "mlp2_train_step G1/dW2 failed");
    if (st) return st;
    // dX = G1 W1^T (NT) and db1 = colsum(G1) with b1 -= lr * db1.
    if (dX) {
        st = check_hip(fdl::launch_group2(gemm_job(false, true, B, I, Hd, G1, Hd, W1, Hd, dX,
                                                   fdl::EPI_NONE, nullptr, nullptr),
                                          db1_job, hs),
                       "mlp2_train_step dX/db1 failed");
    } else {
        st = check_hip(fdl::launch_colsum_sgd(G1, db1, b1, lr, B, Hd, hs),
                       "mlp2_train_step db1 failed");
    }
    if (st) return st;
    return last_launch();
}

}  // extern "C"

struct fdl_mlp2_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

extern "C" {

int fdl_mlp2_graph_create_steps(fdl_mlp2_graph** out, int steps, const float* X,
                                const int64_t* labels, int64_t batch, int64_t in_features,
                                int64_t hidden, int64_t classes, float* W1, float* b1, float* W2,
                                float* b2, float lr, float* H, float* logits, float* G2,
                                float* G1, float* dW1, float* db1, float* dW2, float* db2,
                                float* dX, float* loss, void* stream) {
    if (!out) return fail(FDL_ERROR_INVALID_VALUE, "mlp2_graph_create: null handle pointer");
    *out = nullptr;
    if (steps < 1) return fail(FDL_ERROR_INVALID_VALUE, "mlp2_graph_create: steps must be >= 1");
    hipStream_t s = as_stream(stream);
    hipStream_t own = nullptr;
    if (s == nullptr) {
        hipError_t e = hipStreamCreateWithFlags(&own, hipStreamNonBlocking);
        if (e != hipSuccess) return check_hip(e, "mlp2_graph_create: stream");
        s = own;
    }
    auto cleanup = [&] {
        if (own) (void)hipStreamDestroy(own);
    };
    hipError_t e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) {
        cleanup();
        return check_hip(e, "mlp2_graph_create: begin capture");
    }
    int st = FDL_SUCCESS;
    for (int i = 0; i < steps && st == FDL_SUCCESS; ++i) {
        st = fdl_mlp2_train_step(X, labels, batch, in_features, hidden, classes, W1, b1, W2, b2,
                                 lr, H, logits, G2, G1, dW1, db1, dW2, db2, dX, loss, s);
    }
    hipGraph_t graph = nullptr;
    e = hipStreamEndCapture(s, &graph);
    if (st != FDL_SUCCESS || e != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        cleanup();
        return st != FDL_SUCCESS ? st : check_hip(e, "mlp2_graph_create: end capture");
    }
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    cleanup();
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return check_hip(e, "mlp2_graph_create: instantiate");
    }
    auto* g = new fdl_mlp2_graph;
    g->graph = graph;
    g->exec = exec;
    *out = g;
    return FDL_SUCCESS;
}

int fdl_mlp2_graph_create(fdl_mlp2_graph** out, const float* X, const int64_t* labels,
                          int64_t batch, int64_t in_features, int64_t hidden, int64_t classes,
                          float* W1, float* b1, float* W2, float* b2, float lr, float* H,
                          float* logits, float* G2, float* G1, float* dW1, float* db1,
                          float* dW2, float* db2, float* dX, float* loss, void* stream) {
    return fdl_mlp2_graph_create_steps(out, 1, X, labels, batch, in_features, hidden, classes,
                                       W1, b1, W2, b2, lr, H, logits, G2, G1, dW1, db1, dW2,
                                       db2, dX, loss, stream);
}

int fdl_mlp2_graph_launch(fdl_mlp2_graph* g, void* stream) {
    if (!g || !g->exec) return fail(FDL_ERROR_INVALID_VALUE, "mlp2_graph_launch: null graph");
    return check_hip(hipGraphLaunch(g->exec, as_stream(stream)), "mlp2_graph_launch failed");
}

int fdl_mlp2_graph_destroy(fdl_mlp2_graph* g) {
    if (!g) return FDL_SUCCESS;
    hipError_t e1 = g->exec ? hipGraphExecDestroy(g->exec) : hipSuccess;
    hipError_t e2 = g->graph ? hipGraphDestroy(g->graph) : hipSuccess;
    delete g;
    if (e1 != hipSuccess) return check_hip(e1, "mlp2_graph_destroy");
    return check_hip(e2, "mlp2_graph_destroy");
}

int fdl_zero_fill(void* data, int64_t bytes, void* stream) {
    if (bytes < 0) return fail(FDL_ERROR_INVALID_VALUE, "zero_fill: negative size");
    if (bytes == 0) return FDL_SUCCESS;
    if (!data) return fail(FDL_ERROR_INVALID_VALUE, "zero_fill: null pointer");
    return check_hip(fdl::launch_zero_fill(data, bytes, as_stream(stream)),
                     "zero_fill launch failed");
}

int fdl_fill_uniform(float* data, int64_t n, float low, float high, uint64_t seed,
                     void* stream) {
    if (n < 0) return fail(FDL_ERROR_INVALID_VALUE, "fill_uniform: negative size");
    if (n == 0) return FDL_SUCCESS;
    if (!data) return fail(FDL_ERROR_INVALID_VALUE, "fill_uniform: null pointer");
    return check_hip(fdl::launch_fill_uniform(data, n, low, high, seed, as_stream(stream)),
                     "fill_uniform launch failed");
}

int fdl_fill_normal(float* data, int64_t n, float mean, float stddev, uint64_t seed,
                    void* stream) {
    if (n < 0) return fail(FDL_ERROR_INVALID_VALUE, "fill_normal: negative size");
    if (n == 0) return FDL_SUCCESS;
    if (!data) return fail(FDL_ERROR_INVALID_VALUE, "fill_normal: null pointer");
    return check_hip(fdl::launch_fill_normal(data, n, mean, stddev, seed, as_stream(stream)),
                     "fill_normal launch failed");
}

int fdl_idx_gather(const uint8_t* images, const uint8_t* labels, int64_t count,
                   int64_t row_bytes, const int64_t* index, int64_t batch, float divisor,
                   float* x, int64_t* y, void* stream) {
    if (count < 0 || row_bytes < 0 || batch < 0) {
        return fail(FDL_ERROR_INVALID_VALUE, "idx_gather: negative size");
    }
    if (!std::isfinite(divisor) || divisor == 0.0f) {
        return fail(FDL_ERROR_INVALID_VALUE, "idx_gather: divisor must be finite and non-zero");
    }
    if (row_bytes > 0 && (count > INT64_MAX / row_bytes || batch > INT64_MAX / 4 / row_bytes)) {
        return fail(FDL_ERROR_INVALID_VALUE, "idx_gather: sizes overflow");
    }
    if (batch == 0) return FDL_SUCCESS;
    if (!x && !y) return fail(FDL_ERROR_INVALID_VALUE, "idx_gather: x and y are both null");
    if (x && row_bytes > 0 && count > 0 && !images) {
        return fail(FDL_ERROR_INVALID_VALUE, "idx_gather: images is null");
    }
    if (y && count > 0 && !labels) {
        return fail(FDL_ERROR_INVALID_VALUE, "idx_gather: labels is null");
    }
    if (!index && batch > count) {
        return fail(FDL_ERROR_INVALID_VALUE, "idx_gather: batch exceeds count with no index");
    }
    return check_hip(fdl::launch_idx_gather(images, labels, count, row_bytes, index, batch,
                                            divisor, x, y, as_stream(stream)),
                     "idx_gather launch failed");
}

const char* fdl_last_error(void) { return g_last_error.c_str(); }

const char* fdl_status_string(int status) {
    switch (status) {
        case FDL_SUCCESS: return "FDL_SUCCESS";
        case FDL_ERROR_INVALID_VALUE: return "FDL_ERROR_INVALID_VALUE";
        case FDL_ERROR_NOT_SUPPORTED: return "FDL_ERROR_NOT_SUPPORTED";
        case FDL_ERROR_LAUNCH: return "FDL_ERROR_LAUNCH";
        case FDL_ERROR_RUNTIME: return "FDL_ERROR_RUNTIME";
    }
    return "FDL_UNKNOWN_STATUS";
}

const char* fdl_version(void) { return "fastdl_gemm 0.1.0 gfx950"; }

}  // extern "C"
