/*
 * oracle.h -- CPU restatement of the reference's fp32 GEMM path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (fast_dl_amd/, include/)
 * links, loads or calls this code; only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg use it, as the checker or the timed CPU
 * baseline.  Each function names the reference file:line it follows.
 *
 * Parity pinning (what fixes each function independently of its own text):
 *   oracle_gemm_cpu / oracle_sgemm_ex  reference fixture matmul_tensor_test.cpp:30-42
 *       (non-square, so a transposed operand fails), fp64 dot products, NT/TN
 *       identities via explicit transposes, batch == loop of single GEMMs,
 *       integer-valued inputs that are exact in fp32.
 *   bias / relu epilogues  linear_tensor_test.cpp:38-53 fixture, relu_module_test
 *       .cpp:22-29 fixture.
 *   oracle_cross_entropy   cross_entropy_tensor_test.cpp:40-44 fixture
 *       (0.4076059), closed form log-sum-exp at uniform logits (= log C).
 *   oracle_softmax         softmax_tensor_test.cpp:43-46 input, row sums = 1,
 *       shift invariance.
 *   oracle_softmax_xent_grad  central finite differences of the fp64 loss;
 *       rows of the gradient sum to 0 for valid labels.
 *   oracle_mlp2_train_step    central finite differences of the fp64 MLP
 *       loss for every parameter of a small network; the fp32 and fp64 twins
 *       agree; SGD closed form p - lr*g.
 *   oracle_idx_read_labels    the reference's own MNIST label files (record
 *       counts 60000 / 10000, the published per-class counts and first
 *       labels), synthetic files with asymmetric header words (a byte-order
 *       slip fails), a byte >= 128 read through a signed char.
 *   oracle_idx_read_images / oracle_idx_gather  synthetic IDX3 files built
 *       byte by byte in the tests; every byte value against the correctly
 *       rounded quotient b/255 found from exact rationals; a gather equals
 *       indexing the whole converted set.
 */
#ifndef FASTDL_ORACLE_H
#define FASTDL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* tests/benchmarks/gemm/gemm_benchmark.cu:14-26: row -> col -> kk, float sum. */
void oracle_gemm_cpu(const float* a, const float* b, float* c, size_t m, size_t n, size_t k);

/* Rows [row0, row1) of oracle_gemm_cpu only (bounded CPU-baseline sample). */
void oracle_gemm_cpu_rows(const float* a, const float* b, float* c, size_t m, size_t n,
                          size_t k, size_t row0, size_t row1);

/*
 * General form with the same loop order and fp32 accumulator, op(A)/op(B)
 * and epilogue as documented in include/fastdl_gemm.h.  The bias is added
 * after the complete sum (tests/tensor/linear_tensor_test.cpp:24,
 * src/kernels/cuda/bias.cu:10); ReLU is std::max(0, v)
 * (tests/tensor/activation_tensor_test.cpp:29).
 */
void oracle_sgemm_ex(int transA, int transB, int64_t M, int64_t N, int64_t K,
                     const float* A, int64_t lda, int64_t strideA,
                     const float* B, int64_t ldb, int64_t strideB,
                     float* C, int64_t ldc, int64_t strideC, int64_t batch,
                     const float* bias, const float* aux, int epilogue);

/*
 * fp64 twin of oracle_sgemm_ex for error attribution.  C64 gets the fp64
 * result (epilogue applied in fp64); ABS64 (if non-null) gets
 * sum_k |op(A)_ik| |op(B)_kj| + |bias_j| for the elementwise error bound.
 */
void oracle_sgemm_ex_f64(int transA, int transB, int64_t M, int64_t N, int64_t K,
                         const float* A, int64_t lda, int64_t strideA,
                         const float* B, int64_t ldb, int64_t strideB,
                         double* C64, double* ABS64, int64_t ldc, int64_t strideC,
                         int64_t batch, const float* bias, const float* aux, int epilogue);

/* tests/tensor/linear_tensor_test.cpp:9-29 (weight is [in, out]). */
void oracle_linear(const float* x, const float* w, const float* bias, float* y,
                   size_t batch, size_t in_features, size_t out_features);

/* tests/tensor/activation_tensor_test.cpp:26-32. */
void oracle_relu(const float* x, float* y, size_t n);

/* ReLU backward: g_in = act > 0 ? g_out : 0 (no reference counterpart). */
void oracle_relu_backward(const float* g, const float* act, float* out, size_t n);

/* legacy/src/ops/Layers.cpp:44 colwise sum, rows added in order. */
void oracle_colsum(const float* x, float* out, size_t rows, size_t cols);

/* tests/tensor/softmax_tensor_test.cpp:10-35. */
void oracle_softmax(const float* x, float* y, size_t rows, size_t cols);

/*
 * tests/tensor/cross_entropy_tensor_test.cpp:9-32, with the invalid-label
 * rule of src/kernels/cuda/cross_entropy.cu:16-19 (skipped, still counted).
 */
float oracle_cross_entropy(const float* logits, const int64_t* labels, size_t batch,
                           size_t classes);

/*
 * legacy/src/ops/SoftmaxCrossEntropyLoss.cpp:13-23 (probabilities) and
 * :39-51 (gradient (p - onehot) / batch).
 */
void oracle_softmax_xent_grad(const float* logits, const int64_t* labels, float* grad,
                              size_t batch, size_t classes);

/* legacy/include/dl/optim/Optimizer.hpp:24-34: p -= lr * g. */
void oracle_sgd(float* p, const float* g, float lr, size_t n);

/*
 * One MLP step in -> hidden (ReLU) -> classes, weights [in, out], in the
 * order of legacy/src/runtime/Network.cpp:7-34, every GEMM through
 * oracle_sgemm_ex.  Same buffers and meaning as fdl_mlp2_train_step.
 */
void oracle_mlp2_train_step(const float* X, const int64_t* labels, int64_t batch,
                            int64_t in_features, int64_t hidden, int64_t classes,
                            float* W1, float* b1, float* W2, float* b2, float lr,
                            float* H, float* logits, float* G2, float* G1,
                            float* dW1, float* db1, float* dW2, float* db2,
                            float* dX, float* loss);

/* fp64 loss of the same MLP (forward only), for finite differences. */
double oracle_mlp2_loss_f64(const double* X, const int64_t* labels, int64_t batch,
                            int64_t in_features, int64_t hidden, int64_t classes,
                            const double* W1, const double* b1, const double* W2,
                            const double* b2);

/* fp64 gradients of the same MLP loss (analytic backward in fp64). */
void oracle_mlp2_grads_f64(const double* X, const int64_t* labels, int64_t batch,
                           int64_t in_features, int64_t hidden, int64_t classes,
                           const double* W1, const double* b1, const double* W2,
                           const double* b2, double* dW1, double* db1, double* dW2,
                           double* db2, double* dX);

/*
 * IDX (MNIST) files, legacy/src/data/DataLoader.cpp.  Header words are
 * big-endian 32-bit integers (to_int, :22-25).
 *
 * oracle_idx_read_images follows load_images (:27-72): magic 0x803, the
 * record count cut to num when 0 < num < count (:43), rows, cols, then each
 * pixel as (float)byte / 255.0f (:66).  With images == NULL only the header
 * is read.  *count, *rows, *cols receive the sizes after the num limit.
 * oracle_idx_read_labels follows load_labels (:74-93): magic 0x801, the same
 * num limit (:85), each label byte read through a signed char (:88-89).
 * With labels == NULL only the header is read.
 * Both return 0, or -1 (cannot open), -2 (wrong magic), -3 (truncated file;
 * the reference reads past the end unchecked), -4 (negative num or count).
 */
int oracle_idx_read_images(const char* path, int64_t num, int64_t* count, int64_t* rows,
                           int64_t* cols, float* images);
int oracle_idx_read_labels(const char* path, int64_t num, int64_t* count, int64_t* labels);

/*
 * The batch gather of fdl_idx_gather: r = index ? index[b] : b;
 * x[b][j] = (float)images[r][j] / divisor and y[b] = (int8_t)labels[r] for
 * r in [0, count), else x[b][:] = 0 and y[b] = -1.  x or y may be NULL.
 */
void oracle_idx_gather(const uint8_t* images, const uint8_t* labels, int64_t count,
                       int64_t row_bytes, const int64_t* index, int64_t batch, float divisor,
                       float* x, int64_t* y);

#ifdef __cplusplus
}
#endif

#endif
