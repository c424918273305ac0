// dl::kernels raw-pointer launchers on top of the C-ABI (include/fastdl_gemm.h).
// Each maps one reference launcher (include/dl/kernels/*.hpp of the
// reference) onto this build's gfx950 kernels and turns a non-zero status
// into std::runtime_error.
#include "sgemm_call.hpp"
#include "../tensor/block_cache.hpp"

#include <dl/core/HipUtils.hpp>
#include <dl/core/Stream.hpp>
#include <dl/kernels/kernels.hpp>

#include <fastdl_gemm.h>

#include <hip/hip_runtime_api.h>

#include <stdexcept>
#include <string>

namespace dl::detail {

int sgemm_auto(int transA, int transB, int64_t M, int64_t N, int64_t K, const float* A,
               int64_t lda, int64_t strideA, const float* B, int64_t ldb, int64_t strideB,
               float* C, int64_t ldc, int64_t strideC, int64_t batch, const float* bias,
               const float* aux, int epilogue, void* stream) {
    const size_t bytes = fdl_sgemm_workspace_size(transA, transB, M, N, K, batch);
    if (bytes == 0) {
        return fdl_sgemm_ex(transA, transB, M, N, K, A, lda, strideA, B, ldb, strideB, C, ldc,
                            strideC, batch, bias, aux, epilogue, stream);
    }
    int device = 0;
    hip::check(hipGetDevice(&device), "cudaGetDevice failed");
    BlockCache& cache = device_block_cache();
    void* ws = cache.acquire(device, bytes, stream);
    const int status = fdl_sgemm_ex_ws(transA, transB, M, N, K, A, lda, strideA, B, ldb,
                                       strideB, C, ldc, strideC, batch, bias, aux, epilogue, ws,
                                       bytes, stream);
    cache.release(device, bytes, ws, stream, {});
    return status;
}

}  // namespace dl::detail

namespace dl::kernels {

const char* to_string(GemmAlgo algo) {
    switch (algo) {
        case GemmAlgo::Naive: return "naive";
        case GemmAlgo::Tiled: return "tiled";
        case GemmAlgo::Register: return "register";
        case GemmAlgo::Cublas: return "cublas";
        case GemmAlgo::Auto: return "auto";
        case GemmAlgo::MfmaTiled128: return "mfma_tiled128";
        case GemmAlgo::MfmaTiled64: return "mfma_tiled64";
        case GemmAlgo::MfmaSplitK: return "mfma_splitk32";
        case GemmAlgo::Skinny: return "skinny";
        case GemmAlgo::MfmaDma256: return "mfma_dma256";
        case GemmAlgo::MfmaDma128: return "mfma_dma128";
        case GemmAlgo::MfmaDma64: return "mfma_dma64";
        case GemmAlgo::MfmaDma128W8: return "mfma_dma128w8";
        case GemmAlgo::MfmaDma64U: return "mfma_dma64u";
        case GemmAlgo::MfmaDma128W8U: return "mfma_dma128w8u";
        case GemmAlgo::MfmaDma64S: return "mfma_dma64s";
        case GemmAlgo::MfmaDma96x32U: return "mfma_dma96x32u";
    }
    return "unknown";
}

namespace {

int kernel_id(GemmAlgo algo) {
    switch (algo) {
        case GemmAlgo::Naive: return FDL_KERNEL_SPLITK32;
        case GemmAlgo::Tiled: return FDL_KERNEL_TILED64;
        case GemmAlgo::Register: return FDL_KERNEL_TILED128;
        case GemmAlgo::Cublas: return FDL_KERNEL_AUTO;
        case GemmAlgo::Auto: return FDL_KERNEL_AUTO;
        case GemmAlgo::MfmaTiled128: return FDL_KERNEL_TILED128;
        case GemmAlgo::MfmaTiled64: return FDL_KERNEL_TILED64;
        case GemmAlgo::MfmaSplitK: return FDL_KERNEL_SPLITK32;
        case GemmAlgo::Skinny: return FDL_KERNEL_SKINNY;
        case GemmAlgo::MfmaDma256: return FDL_KERNEL_DMA256;
        case GemmAlgo::MfmaDma128: return FDL_KERNEL_DMA128;
        case GemmAlgo::MfmaDma64: return FDL_KERNEL_DMA64;
        case GemmAlgo::MfmaDma128W8: return FDL_KERNEL_DMA128W8;
        case GemmAlgo::MfmaDma64U: return FDL_KERNEL_DMA64U;
        case GemmAlgo::MfmaDma128W8U: return FDL_KERNEL_DMA128W8U;
        case GemmAlgo::MfmaDma64S: return FDL_KERNEL_DMA64S;
        case GemmAlgo::MfmaDma96x32U: return FDL_KERNEL_DMA96X32U;
    }
    return FDL_KERNEL_AUTO;
}

int epilogue_id(Epilogue e) {
    switch (e) {
        case Epilogue::None: return FDL_EPILOGUE_NONE;
        case Epilogue::Bias: return FDL_EPILOGUE_BIAS;
        case Epilogue::BiasRelu: return FDL_EPILOGUE_BIAS_RELU;
        case Epilogue::Relu: return FDL_EPILOGUE_RELU;
        case Epilogue::ReluGrad: return FDL_EPILOGUE_RELU_GRAD;
    }
    return FDL_EPILOGUE_NONE;
}

}  // namespace

void gemm(const float* a, const float* b, float* c, int m, int n, int k, GemmAlgo algo) {
    gemm_ex(Transpose::No, Transpose::No, m, n, k, a, k > 0 ? k : 1, 0, b, n > 0 ? n : 1, 0, c,
            n > 0 ? n : 1, 0, 1, nullptr, nullptr, Epilogue::None, algo, current_stream());
}

void gemm_ex(Transpose trans_a, Transpose trans_b, int64_t m, int64_t n, int64_t k,
             const float* a, int64_t lda, int64_t stride_a, const float* b, int64_t ldb,
             int64_t stride_b, float* c, int64_t ldc, int64_t stride_c, int64_t batch,
             const float* bias, const float* aux, Epilogue epilogue, GemmAlgo algo,
             void* stream) {
    const int ta = trans_a == Transpose::Yes ? FDL_OP_T : FDL_OP_N;
    const int tb = trans_b == Transpose::Yes ? FDL_OP_T : FDL_OP_N;
    // Cublas named the reference's production path; here that is the automatic choice.
    if (algo == GemmAlgo::Auto || algo == GemmAlgo::Cublas) {
        hip::check_fdl(detail::sgemm_auto(ta, tb, m, n, k, a, lda, stride_a, b, ldb, stride_b, c,
                                          ldc, stride_c, batch, bias, aux, epilogue_id(epilogue),
                                          stream),
                       "gemm failed");
        return;
    }
    hip::check_fdl(fdl_sgemm_ex_select(ta, tb, m, n, k, a, lda, stride_a, b, ldb, stride_b, c, ldc,
                                       stride_c, batch, bias, aux, epilogue_id(epilogue),
                                       kernel_id(algo), stream),
                   "gemm failed");
}

void add_row_bias(float* output, const float* bias, int rows, int cols) {
    hip::check_fdl(fdl_add_row_bias(output, bias, rows, cols, current_stream()), "add_row_bias failed");
}

const char* to_string(ActivationOp op) {
    switch (op) {
        case ActivationOp::ReLU: return "relu";
        case ActivationOp::LeakyReLU: return "leaky_relu";
        case ActivationOp::GELU: return "gelu";
        case ActivationOp::Sigmoid: return "sigmoid";
        case ActivationOp::Tanh: return "tanh";
    }
    return "unknown";
}

void activation(const float* a, float* b, int n, ActivationOp op, float /*alpha*/) {
    if (op != ActivationOp::ReLU) {
        throw std::runtime_error(std::string("activation '") + to_string(op) +
                                 "' is not provided by this build (only relu is on the GEMM path)");
    }
    hip::check_fdl(fdl_relu(a, b, n, current_stream()), "relu failed");
}

void relu_backward(const float* grad_out, const float* act, float* grad_in, int64_t n) {
    hip::check_fdl(fdl_relu_backward(grad_out, act, grad_in, n, current_stream()), "relu_backward failed");
}

const char* to_string(SoftmaxAlgo algo) {
    switch (algo) {
        case SoftmaxAlgo::Naive: return "naive";
        case SoftmaxAlgo::SharedMemory: return "shared_memory";
        case SoftmaxAlgo::WarpShuffleRegCache: return "warp_shuffle_reg_cache";
    }
    return "unknown";
}

void softmax(const float* input, float* output, std::size_t rows, std::size_t cols,
             SoftmaxAlgo /*algo*/) {
    hip::check_fdl(fdl_softmax(input, output, static_cast<int64_t>(rows),
                               static_cast<int64_t>(cols), current_stream()),
                   "softmax failed");
}

void cross_entropy(const float* logits, const int64_t* labels, float* loss, int batch,
                   int classes) {
    hip::check_fdl(fdl_softmax_xent(logits, labels, loss, nullptr, batch, classes, current_stream()),
                   "cross_entropy failed");
}

void cross_entropy_backward(const float* logits, const int64_t* labels, float* loss,
                            float* grad, int batch, int classes) {
    hip::check_fdl(fdl_softmax_xent(logits, labels, loss, grad, batch, classes, current_stream()),
                   "cross_entropy_backward failed");
}

void uniform_float32(float* data, int64_t n, float low, float high, uint64_t seed) {
    if (n <= 0) return;
    hip::check_fdl(fdl_fill_uniform(data, n, low, high, seed, current_stream()), "uniform fill failed");
}

void normal_float32(float* data, int64_t n, float mean, float stddev, uint64_t seed) {
    if (n <= 0) return;
    hip::check_fdl(fdl_fill_normal(data, n, mean, stddev, seed, current_stream()), "normal fill failed");
}

void colsum(const float* x, float* out, int64_t rows, int64_t cols) {
    hip::check_fdl(fdl_colsum(x, out, rows, cols, current_stream()), "colsum failed");
}

void sgd_update(float* param, const float* grad, float lr, int64_t n) {
    hip::check_fdl(fdl_sgd_update(param, grad, lr, n, current_stream()), "sgd_update failed");
}

}  // namespace dl::kernels
