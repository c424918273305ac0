#pragma once
// Raw-pointer GEMM launchers (reference include/dl/kernels/gemm.hpp).
//
// gemm() keeps the reference's signature and contract: row-major
// C[m,n] = A[m,k] . B[k,n], C overwritten, enqueued on the calling thread's
// current stream (dl/core/Stream.hpp; the null stream unless the caller
// chose another, as in the reference).  GemmAlgo keeps the reference's four
// enumerators (include/dl/kernels/gemm.hpp:7-12 there; src/ops/Matmul.cpp:42
// and tests/benchmarks/gemm/gemm_benchmark.cu:87-99 name them), each mapped
// to the gfx950 family closest to the kernel it named; Cublas, the
// reference's production path, is the automatic choice.  The remaining
// enumerators name this build's kernel families; Auto (the default) picks
// one by shape, as the reference's default picked cuBLAS.

#include <cstddef>
#include <cstdint>

namespace dl::kernels {

enum class GemmAlgo {
    Naive,          // reference: direct K loop, no shared memory -> MfmaSplitK (operands
                    // straight from L2 into MFMA registers)
    Tiled,          // reference: 16x16 shared-memory tiles -> MfmaTiled64
    Register,       // reference: 128x128 block tile, register blocking -> MfmaTiled128
    Cublas,         // reference: cublasSgemm, the production path -> Auto
    Auto,
    MfmaTiled128,   // 128x128x16 LDS double-buffered fp32 MFMA tile
    MfmaTiled64,    // 64x64x16 LDS double-buffered fp32 MFMA tile
    MfmaSplitK,     // 32x32 MFMA tile, K split over the waves of a block
    Skinny,         // VALU streaming kernel for m <= 8
    MfmaDma256,     // 256x256x16 tile fed by direct global->LDS copies (k % 4 == 0,
                    // 16-byte-aligned operands; std::runtime_error otherwise)
    MfmaDma128,     // 128x128x32 tile, same copies, two blocks per CU
    MfmaDma64,      // 64x64x64 tile, same copies, for mid-size problems
    MfmaDma128W8,   // 128x128x64 tile, same copies, eight waves, one block per CU
    MfmaDma64U,     // MfmaDma64 with 4-byte copies: any k, leading dimension, alignment
    MfmaDma128W8U,  // MfmaDma128W8 with 4-byte copies
    MfmaDma64S,     // 64x64x16 tile, same copies as MfmaDma64, all K-tiles in flight (k <= 128)
    MfmaDma96x32U,  // 96x32x64 tile, 4-byte copies, twelve waves (mid sizes short of tiles)
};

const char* to_string(GemmAlgo algo);

void gemm(const float* a, const float* b, float* c, int m, int n, int k,
          GemmAlgo algo = GemmAlgo::Auto);

enum class Transpose { No, Yes };

enum class Epilogue {
    None,        // C = acc
    Bias,        // C = acc + bias[j]
    BiasRelu,    // C = max(0, acc + bias[j])
    Relu,        // C = max(0, acc)
    ReluGrad,    // C = aux[i][j] > 0 ? acc : 0
};

// General strided-batched form (fdl_sgemm_ex in include/fastdl_gemm.h):
// C[b] = epi(op(A[b]) . op(B[b])), row-major, with leading dimensions and
// element strides.  `stream` is a hipStream_t (nullptr: null stream).
// Throws std::runtime_error on invalid arguments or launch failure.
void gemm_ex(Transpose trans_a, Transpose trans_b, int64_t m, int64_t n, int64_t k,
             const float* a, int64_t lda, int64_t stride_a,
             const float* b, int64_t ldb, int64_t stride_b,
             float* c, int64_t ldc, int64_t stride_c, int64_t batch,
             const float* bias = nullptr, const float* aux = nullptr,
             Epilogue epilogue = Epilogue::None, GemmAlgo algo = GemmAlgo::Auto,
             void* stream = nullptr);

}  // namespace dl::kernels
